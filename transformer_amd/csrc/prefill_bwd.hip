// Backward of the causal MLA prefill attention (gfx950): dQ, dK, dV.
//
// Given dO, O and the forward's LSE (natural log), with P = exp(S - LSE):
//   D   = rowsum(dO o O)                     (bwd_rowdot_kernel, which also stores LSE
//                                             in log2 units beside D, per 32 queries)
//   dV  = P^T dO,    dP = dO V^T,  dS = P o (dP - D)
//   dK  = dS^T Q * scale                     (bwd_dkdv_kernel: one key tile per workgroup)
//   dQ  = dS K * scale                       (bwd_dq_ds_kernel from the dS blocks the
//                                             dK/dV kernel stores, or bwd_dq_kernel, which
//                                             recomputes S and dP: one query tile per workgroup)
// which is the autograd backward of SDPA at transformer.py:314 (recomputed under
// activation checkpointing, :330-335).  dK and dQ are produced by separate kernels
// so every output element is written by exactly one workgroup: no atomics, and the
// result is bitwise reproducible.  A shared k_rope head (stride 0 over heads) gets
// sum_h dk_rope[h], accumulated in fp32 per head and reduced in head order (in the tail of
// bwd_dq_ds_kernel, or by bwd_dkrope_reduce_kernel after the recomputing dQ kernel).
//
// MFMA layout (v_mfma_f32_32x32x16_bf16, see mla_common.h); every tile is staged once,
// row-major and swizzled, and transposed operands come from ds_read_b64_tr_b16:
//   dK/dV kernel, wave = 32 keys, loop over 32-query blocks (Q, dO, LSE, D in LDS):
//     S  (32q x 32k) = Q . K^T        A = Q rows (LDS),  B = K rows (registers)
//     dP (32q x 32k) = dO . V^T       A = dO rows (LDS), B = V rows (registers)
//       -> lanes own a key column, registers run over queries, so P and dS feed
//          the next products' B operand directly:
//     dV^T (128 x 32k) += dO^T . P    A = dO^T (transpose read)
//     dK^T (DQK x 32k) += Q^T . dS    A = Q^T  (transpose read)
//   dQ kernel, wave = 32 queries, loop over 32-key blocks (K, V in LDS):
//     S^T (32k x 32q) = K . Q^T,  dP^T = V . dO^T   (lanes own a query)
//     dQ^T (DQK x 32q) += K^T . dS^T                (K^T by transpose read)
// Workgroups take mirrored pairs of tiles of one (b, h) so causal work is balanced.
#include <type_traits>

#include "mla_common.h"

namespace mla {

struct BwdParams {
  const bf16 *dout, *qn, *qr, *kn, *kr, *v, *o;
  const float* lse;
  bf16 *dqn, *dqr, *dkn, *dkr, *dv;
  float* ld;       // [B][H][ceil(Tq / 32)][64]: LSE * log2(e) of 32 queries, then their D
  float* dkr_ws;   // [B][Tk][H][64] fp32 per-head dk_rope (shared k_rope only)
  bf16* ds_ws;     // stored dS blocks (32 x 32, 2 KiB): per (b, h) the visible blocks of query
                   // block 0, then of block 1, ... (ds_prefix gives the offsets)
  int nkb32;       // ceil(Tk / 32)
  int ds_e;        // (31 + max(q_offset, 0)) / 32: the causal rows' extra visible key blocks
  int64_t ds_bh_blocks;  // stored blocks per (b, h)
  int B, H, Tq, Tk;
  int shared_rope;
  mla_strides do_s, qn_s, qr_s, kn_s, kr_s, v_s, o_s;
  mla_strides dqn_s, dqr_s, dkn_s, dkr_s, dv_s;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
  int causal;
  int64_t q_offset;
  // RoPE folded into the dQ epilogue (rope_cos non-null): q_rope was rotated in the forward's
  // Q load, so dq_rope is rotated back (by the opposite angle, at position q_pos_offset + t)
  // before it is rounded and stored
  const bf16 *rope_cos, *rope_sin;
  int64_t q_pos_offset;
};

// dQ of one lane's query, scaled in place for its store (times the softmax scale).  Rope dims
// 8 i + 4 g + j of block NLO (register 4 i + j) pair with dims 32 + 8 i + 4 g + j of block
// NLO + 1, so with the tables the pair is rotated back (R^T, the gradient of the forward's
// rotation) in fp32 before the one rounding.  NLO < 0: the blocks hold no rope dims.
template <int NLO, int NB, typename Acc>
__device__ __forceinline__ void dq_scale_rope_back(Acc (&acc)[NB], const BwdParams& p, int q_row, int g) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] *= p.scale;
  if constexpr (NLO < 0) return;
  else {
    static_assert(NLO + 1 < NB, "both blocks of a rotation pair are in the array");
    if (!p.rope_cos) return;
    const int64_t pos = p.q_pos_offset + q_row;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2 cw = ldg8(p.rope_cos + pos * 32 + 8 * i + 4 * g), sw = ldg8(p.rope_sin + pos * 32 + 8 * i + 4 * g);
      const float c[4] = {lo_bf16(cw[0]), hi_bf16(cw[0]), lo_bf16(cw[1]), hi_bf16(cw[1])};
      const float sn[4] = {lo_bf16(sw[0]), hi_bf16(sw[0]), lo_bf16(sw[1]), hi_bf16(sw[1])};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float y1, y2;
        rope_pair(acc[NLO][4 * i + j], acc[NLO + 1][4 * i + j], c[j], -sn[j], y1, y2);
        acc[NLO][4 * i + j] = y1;
        acc[NLO + 1][4 * i + j] = y2;
      }
    }
  }
}

// ---------------------------------------------------------------- D = rowsum(dO o O)
// One workgroup per (b, h, block of 32 queries): 8 lanes per query row, 16 values each.
// The workgroup writes the block's 64-float record in one coalesced store: LSE * log2(e)
// of the 32 queries, then their D.  Queries past Tq get 0 and 0 (with zero Q and dO
// rows their P = 1 meets dO = 0 and dS = 0, so they add nothing).
__global__ __launch_bounds__(256) void bwd_rowdot_kernel(BwdParams p) {
  __shared__ float d_s[32];
  const int nqb = (p.Tq + 31) >> 5;
  // workgroups walk (b, query block, head) with the head fastest, so consecutive workgroups read
  // the heads' adjacent 256-byte row segments of the same queries; the record stays (b, h, qb)
  const int64_t wg = blockIdx.x;
  const int64_t h = wg % p.H, bq = wg / p.H;
  const int qb = (int)(bq % nqb);
  const int64_t b = bq / nqb;
  const int64_t bh = b * p.H + h;
  const int64_t rec_id = bh * nqb + qb;
  const int r = threadIdx.x >> 3, part = threadIdx.x & 7;
  const int64_t q = (int64_t)qb * 32 + r;
  float acc = 0.f;
  if (q < p.Tq) {
    const bf16* dop = p.dout + b * p.do_s.b + q * p.do_s.t + h * p.do_s.h + 16 * part;
    const bf16* op = p.o + b * p.o_s.b + q * p.o_s.t + h * p.o_s.h + 16 * part;
    const u32x4 a0 = ldg16(dop), a1 = ldg16(dop + 8), c0 = ldg16(op), c1 = ldg16(op + 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc += lo_bf16(a0[i]) * lo_bf16(c0[i]) + hi_bf16(a0[i]) * hi_bf16(c0[i]);
      acc += lo_bf16(a1[i]) * lo_bf16(c1[i]) + hi_bf16(a1[i]) * hi_bf16(c1[i]);
    }
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) acc += wave_shfl_xor(acc, m);
  if (part == 0) d_s[r] = acc;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int i = threadIdx.x & 31;
    const int64_t qi = (int64_t)qb * 32 + i;
    float v;
    if (threadIdx.x < 32) v = qi < p.Tq ? p.lse[bh * p.Tq + qi] * kLog2e : 0.f;
    else v = d_s[i];
    p.ld[rec_id * 64 + threadIdx.x] = v;
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Stored dS blocks before query block Q of a (b, h).  Query block i (queries 32 i .. 32 i + 31)
// sees key blocks 0 .. c(i) - 1 with c(i) = min(nkb, i + 1 + e), e = (31 + q_offset) / 32 under
// the causal mask (a key block is visible when its first key is seen by the block's last
// query), and c(i) = nkb without it.  Only those blocks are stored, row after row.
__host__ __device__ inline int64_t ds_prefix(int64_t Q, int64_t nkb, int64_t q_offset, bool causal) {
  if (!causal) return Q * nkb;
  const int64_t e = (31 + (q_offset > 0 ? q_offset : 0)) / 32;
  const int64_t t = nkb - 1 - e;  // rows i < t hold i + 1 + e blocks, later rows nkb
  if (t <= 0) return Q * nkb;
  const int64_t m = Q < t ? Q : t;
  return m * (m + 1) / 2 + m * e + (Q - m) * nkb;
}
// The same in 32-bit arithmetic for the kernels, with e = (31 + max(q_offset, 0)) / 32 given: the
// blocks are stored only when all of them fit kDsCap (8 GiB), so a (b, h) holds fewer than 2^22.
__device__ __forceinline__ int ds_prefix32(int Q, int nkb, int e, bool causal) {
  const int t = nkb - 1 - e;
  if (!causal || t <= 0) return Q * nkb;
  const int m = Q < t ? Q : t;
  return (int)(((unsigned)m * (unsigned)(m + 1)) >> 1) + m * e + (Q - m) * nkb;
}

// workgroup id -> (b, h, the pair of tiles r and n - 1 - r of that (b, h)); XCD-contiguous
__device__ __forceinline__ void bwd_coords(int n_tiles, int H, int& b, int& h, int& ta, int& tb, int& n_items) {
  const int n = gridDim.x;
  int id = blockIdx.x;
  if ((n & 7) == 0) id = (id & 7) * (n >> 3) + (id >> 3);
  const int n_pairs = (n_tiles + 1) >> 1;
  const int bh = id / n_pairs;
  const int r = id - bh * n_pairs;
  ta = r;
  tb = n_tiles - 1 - r;
  n_items = ta == tb ? 1 : 2;
  b = bh / H;
  h = bh - b * H;
}

// ---------------------------------------------------------------- dK, dV (key-stationary)
// Workgroup = 8 waves over 128 keys, in two roles per 32-key block kb:
//   * producer (wave kb): keeps the K and V rows of its keys in registers (B operands of
//     S = Q K^T and dP = dO V^T), computes S, dP, P = 2^(S scale log2 e - LSE2) and
//     dS = P (dP - D) of each 32-query block (V held negated, so the dP chain starts at D
//     and ends at D - dP) and writes P and dS, packed as the
//     consumer's MFMA B operands, to an LDS exchange buffer (double-buffered);
//   * consumer (wave kb + 4): issues the block loads and accumulates dV^T += dO^T P and
//     dK^T += Q^T dS one block behind, with the transposed Q / dO read by
//     ds_read_b64_tr_b16; lanes own a key, so dV and dK rows are stored as 8-byte vectors.
// Each role fits 256 registers (the producer's 80 registers of K/V fragments and the
// consumer's 160 of accumulators are never live together), so a SIMD runs one producer
// and one consumer, which hide each other's latency.  The blocks (Q_nope, Q_rope, dO and
// the LSE/D record) are written by buffer loads straight into LDS: a ring of four stages,
// block t in stage t % 4, loaded two steps before the producers use it; one barrier per
// step orders the loads, the exchange and the stage reuse.
//
// LDS chunk swizzles (chunk c of row r at position c ^ f(r)): every tile is read both by
// rows (one row per lane) and transposed (per 16 lanes, 4 rows x 2 chunks); both patterns
// hit 16 distinct 16-byte bank groups per 16 lanes (32 per 32):
//   256-byte rows (Q_nope for DN = 128, dO):        f = 4 (r mod 4) + (r / 4) mod 4
//   128-byte rows (Q_rope, Q_nope for DN = 64):      f = 4 ((r / 2) mod 2) + (r / 4) mod 4
__device__ __forceinline__ int bsw256(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int bsw128(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

// a ^ k formed where it is used (the asm keeps the compiler from hoisting it into a register of
// its own): for the recomputing dQ kernel, which has no register to spare for its loop-invariant
// read addresses.  Kernels with room keep those addresses in registers instead: each at-use XOR
// is a VALU instruction on the read's critical path.
__device__ __forceinline__ int xor_at_use(int a, int k) {
  int r;
  asm volatile("v_xor_b32 %0, %1, %2" : "=v"(r) : "s"(k), "v"(a));
  return r;
}

template <int DN>
struct DkdvCfg {
  static constexpr int DR = 64, DV = 128, DQK = DN + DR;
  static constexpr int KS = DQK / 16, KNS = DN / 16;  // k-steps of S, of which over the nope dims
  static constexpr int NDQK = DQK / 32, NDN = DN / 32;
  static constexpr int BKV = 128, BQ = 32;            // keys per workgroup, queries per block
  static constexpr int QN_RB = DN * 2;                // Q_nope row bytes
  static constexpr int OFF_QR = BQ * QN_RB;           // stage: Q_nope | Q_rope | dO | LSE2, D
  static constexpr int OFF_DO = OFF_QR + BQ * 128;
  static constexpr int OFF_LD = OFF_DO + BQ * 256;
  static constexpr int STAGE = OFF_LD + 1024;
  // 1 KiB loads per block: Q_nope, Q_rope, dO (spread over the 4 waves), one for LSE2 / D
  static constexpr int T_QN = BQ * QN_RB / 1024, T_QR = BQ * 128 / 1024, T_DO = BQ * 256 / 1024;
  static constexpr int MK_QN = T_QN / 4, MK_QR = T_QR / 4, MK_DO = T_DO / 4;
  static constexpr int NL = MK_QN + MK_QR + MK_DO + 1;  // a wave's loads per block (at most)
  static constexpr int NM1 = KS + DV / 16;              // S and dP MFMAs per block
  static constexpr int NB2 = DV / 32 + NDQK;            // dV and dK MFMAs per 16 queries
  static_assert(T_QN % 4 == 0 && T_QR % 4 == 0 && T_DO % 4 == 0, "loads split evenly over 4 waves");
  static_assert(NL <= 6, "six load offsets are kept");
};
#ifndef BWD_S_AHEAD
#define BWD_S_AHEAD 3  // S / dP A fragments read ahead of their MFMA
#endif
#ifndef BWD_T_AHEAD
#define BWD_T_AHEAD 3  // transposed fragments read ahead of their dV / dK MFMA
#endif
// 32-query blocks per wave in bwd_dq_ds_kernel: 1 (a wave owns 32 queries and all 192 dims), or 2
// (a 2 x 2 grid of waves, 64 queries x 96 dims each: 10 instead of 14 KiB of LDS reads per wave and
// step, 165 instead of 243 VGPRs, bitwise equal, but 1.4 % slower on the kernel at B = 4, T = 4096)
#ifndef BWD_DQ_QBW
#define BWD_DQ_QBW 1
#endif

template <int DN>
__global__ __launch_bounds__(512, 1) void bwd_dkdv_kernel(BwdParams p) {
  using C = DkdvCfg<DN>;
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage3[C::STAGE];
  // P and dS of one block per key block (4 x 4 KiB), double-buffered between the producer
  // and the consumer of that key block
  __shared__ __attribute__((aligned(1024))) unsigned char xch0[4 * 4096];
  __shared__ __attribute__((aligned(1024))) unsigned char xch1[4 * 4096];
  auto stage = [&](auto s_tag) -> unsigned char* {
    constexpr int S = decltype(s_tag)::value % 4;
    return S == 0 ? stage0 : S == 1 ? stage1 : S == 2 ? stage2 : stage3;
  };
  auto stage_at = [&](int i) -> unsigned char* {
    i &= 3;
    return i == 0 ? stage0 : i == 1 ? stage1 : i == 2 ? stage2 : stage3;
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  const int n_kt = (p.Tk + C::BKV - 1) / C::BKV;
  int b, h, kt_a, kt_b, n_items;
  bwd_coords(n_kt, p.H, b, h, kt_a, kt_b, n_items);
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wv >= 0 && wv < 8);
  const int kb = wv & 3;  // key block of the wave (producer wv, consumer wv + 4)
  const int q_off = (int)p.q_offset;
  const int nqb = (p.Tq + C::BQ - 1) / C::BQ;

  {
    const u32x4 z{0u, 0u, 0u, 0u};
    for (int i = tid; i < C::STAGE / 16; i += 512) {
      sts16(stage0 + 16 * i, z);
      sts16(stage1 + 16 * i, z);
      sts16(stage2 + 16 * i, z);
      sts16(stage3 + 16 * i, z);
    }
    __syncthreads();
  }

  // first query block (walking from the last one down) and number of blocks of item `it`
  auto item_blocks = [&](int it, int& k0, int& n_steps) {
    k0 = (it == 0 ? kt_a : kt_b) * C::BKV;
    const int q_first = p.causal ? max(0, k0 - q_off) : 0;
    const int qb_begin = q_first < p.Tq ? q_first / C::BQ : nqb;
    n_steps = nqb - qb_begin;
  };
  // does query block j (from the last one down) hold a query that sees a key of key block kb?
  auto visible = [&](int j, int kw0) { return !p.causal || (nqb - 1 - j) * C::BQ + C::BQ - 1 + q_off >= kw0; };

  if (wv < 4) {
    // ============================ producer: S, dP, P, dS of each block of its 32 keys
    const int a_qn = DN == 128 ? l32 * 256 + 16 * (g ^ bsw256(l32)) : l32 * 128 + 16 * (g ^ bsw128(l32));
    const int a_qr = C::OFF_QR + l32 * 128 + 16 * (g ^ bsw128(l32));
    const int a_do = C::OFF_DO + l32 * 256 + 16 * (g ^ bsw256(l32));
    for (int item = 0; item < n_items; ++item) {
      int k0, n_steps;
      item_blocks(item, k0, n_steps);
      const int kw0 = k0 + 32 * kb;
      const int key = kw0 + l32;
      const int key_ld = key < p.Tk ? key : p.Tk - 1;
      bf16x8 kf[C::KS], vf[C::DV / 16];
      {
        const bf16* kn = p.kn + (int64_t)b * p.kn_s.b + (int64_t)key_ld * p.kn_s.t + (int64_t)h * p.kn_s.h;
        const bf16* kr = p.kr + (int64_t)b * p.kr_s.b + (int64_t)key_ld * p.kr_s.t + (int64_t)h * p.kr_s.h;
        const bf16* vp = p.v + (int64_t)b * p.v_s.b + (int64_t)key_ld * p.v_s.t + (int64_t)h * p.v_s.h;
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
          const int d = 16 * ks + 8 * g;
          kf[ks] = as_bf16x8(d < DN ? ldg16(kn + d) : ldg16(kr + (d - DN)));
        }
        // V is held negated (bf16 sign flips, once per item): the dP product then accumulates
        // D - dO V^T from an accumulator that starts at D, and dS = P (dP - D) = -(P acc) takes one
        // multiply (the negation is an operand modifier) instead of a subtract and a multiply
#pragma unroll
        for (int ks = 0; ks < C::DV / 16; ++ks) {
          const u32x4 v = ldg16(vp + 16 * ks + 8 * g);
          const uint32_t sg = 0x80008000u;
          vf[ks] = as_bf16x8(u32x4{v[0] ^ sg, v[1] ^ sg, v[2] ^ sg, v[3] ^ sg});
        }
      }
      bf16* const ds_bh = p.ds_ws ? p.ds_ws + ((int64_t)b * p.H + h) * p.ds_bh_blocks * 1024 : nullptr;
      auto afrag = [&](const unsigned char* st, int n) -> bf16x8 {
        constexpr int NI = C::DV / 16;
        const bool is_dp = n < 2 * NI && (n & 1);
        const int ks = n < 2 * NI ? (n >> 1) : n - NI;
        if (is_dp) return as_bf16x8(lds16(st + (a_do ^ (32 * ks))));
        return as_bf16x8(lds16(st + (ks < C::KNS ? (a_qn ^ (32 * ks)) : (a_qr ^ (32 * (ks - C::KNS))))));
      };
      auto produce = [&](int j, const unsigned char* st, unsigned char* xb) {
        if (!visible(j, kw0)) return;
        const int q0 = (nqb - 1 - j) * C::BQ;
        // LSE2 and D of the block's queries 8 r4 + 4 g + [0, 4), read before the MFMAs so their
        // latency hides under them
        f32x4 lq[4], dd[4];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          lq[r4] = *reinterpret_cast<const f32x4*>(st + C::OFF_LD + 4 * (8 * r4 + 4 * g));
          dd[r4] = *reinterpret_cast<const f32x4*>(st + C::OFF_LD + 128 + 4 * (8 * r4 + 4 * g));
        }
        f32x16 sc = f32x16{};
        // starts at D of each register's query (register 4 r4 + i <-> dd[r4][i]); after the chain
        // it holds D - dP
        f32x16 dp = f32x16{dd[0][0], dd[0][1], dd[0][2], dd[0][3], dd[1][0], dd[1][1], dd[1][2], dd[1][3],
                           dd[2][0], dd[2][1], dd[2][2], dd[2][3], dd[3][0], dd[3][1], dd[3][2], dd[3][3]};
        {
          bf16x8 a[C::NM1];
#pragma unroll
          for (int n = 0; n < BWD_S_AHEAD; ++n) a[n] = afrag(st, n);
#pragma unroll
          for (int n = 0; n < C::NM1; ++n) {
            if (n + BWD_S_AHEAD < C::NM1) a[n + BWD_S_AHEAD] = afrag(st, n + BWD_S_AHEAD);
            constexpr int NI = C::DV / 16;
            const int ks = n < 2 * NI ? (n >> 1) : n - NI;
            if (n < 2 * NI && (n & 1)) dp = mfma32(a[n], vf[ks], dp);
            else sc = mfma32(a[n], kf[ks], sc);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        if ((p.causal && kw0 + 31 > q0 + q_off) || q0 + C::BQ > p.Tq || kw0 + 31 >= p.Tk) {
          // query q sees the key iff lim <= q < Tq; a key past Tk (a clamped copy of the last
          // one) gets p = 0, so its stored dS is 0
          const int lim = key >= p.Tk ? p.Tq : p.causal ? key - q_off : 0;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int q = q0 + 8 * (r >> 2) + 4 * g + (r & 3);
            sc[r] = q >= lim && q < p.Tq ? sc[r] : -INFINITY;
          }
        }
        // register r = 4 r4 + i holds query 8 r4 + 4 g + i: P, dS packed as the consumer's B
        // operands (K slot (g, e) of operand s <-> registers 8 s + e), 16 bytes per lane each
        unsigned char* xs = xb + kb * 4096 + lane * 16;
        // the stored block (a key block wholly past Tk has none).  Layout [s][key][g][8]: this
        // lane's 16 bytes (queries 16 s + 4 g + [0, 4), then 16 s + 8 + 4 g + [0, 4), of its key)
        // at 1024 s + 32 key + 16 g, so one store of the wave writes 1 KiB contiguously
        bf16* blk = p.ds_ws && kw0 < p.Tk
                        ? ds_bh + (int64_t)(ds_prefix32(q0 >> 5, p.nkb32, p.ds_e, p.causal) + (kw0 >> 5)) * 1024
                        : nullptr;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          uint32_t pk[4], dk[4];
#pragma unroll
          for (int r4 = 2 * s; r4 < 2 * s + 2; ++r4) {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
              const int r = 4 * r4 + i;
              const float p0 = fast_exp2(__builtin_fmaf(sc[r], p.scale_log2, -lq[r4][i]));
              const float p1 = fast_exp2(__builtin_fmaf(sc[r + 1], p.scale_log2, -lq[r4][i + 1]));
              pk[(r - 8 * s) >> 1] = pack_bf16x2(p0, p1);
              dk[(r - 8 * s) >> 1] = pack_bf16x2(p0 * -dp[r], p1 * -dp[r + 1]);  // P (dP - D)
            }
          }
          sts16(xs + 1024 * s, u32x4{pk[0], pk[1], pk[2], pk[3]});
          sts16(xs + 2048 + 1024 * s, u32x4{dk[0], dk[1], dk[2], dk[3]});
          // non-temporal: 2 KiB per block over the whole pass, read once by the dQ pass
          if (blk)
            __builtin_nontemporal_store(u32x4{dk[0], dk[1], dk[2], dk[3]},
                                        reinterpret_cast<u32x4*>(blk + 512 * s + 16 * l32 + 8 * g));
        }
      };
      auto pstep = [&](int j, auto par_tag) {
        constexpr int P = decltype(par_tag)::value;
        __syncthreads();
        produce(j, stage(par_tag), P % 2 == 0 ? xch0 : xch1);
      };
      for (int j = 0; j < n_steps; j += 4) {
        pstep(j, S0{});
        if (j + 1 < n_steps) pstep(j + 1, S1{});
        if (j + 2 < n_steps) pstep(j + 2, S2{});
        if (j + 3 < n_steps) pstep(j + 3, S3{});
      }
      __syncthreads();  // the last block's P, dS are written
      __syncthreads();  // every wave is done with the stages
    }
  } else {
    // ============================ consumer: the block loads, dV^T += dO^T P, dK^T += Q^T dS
    const bf16* qn_b = p.qn + (int64_t)b * p.qn_s.b + (int64_t)h * p.qn_s.h;
    const bf16* qr_b = p.qr + (int64_t)b * p.qr_s.b + (int64_t)h * p.qr_s.h;
    const bf16* do_b = p.dout + (int64_t)b * p.do_s.b + (int64_t)h * p.do_s.h;
    const float* ld_b = p.ld + ((int64_t)b * p.H + h) * nqb * 64;
    const int qn_st = (int)p.qn_s.t, qr_st = (int)p.qr_s.t, do_st = (int)p.do_s.t;
    const int w = kb;  // the consumer waves issue the loads: wave w takes loads I = w + 4 k
    auto load_voff = [&](int n) -> uint32_t {
      if (n < C::MK_QN) {
        const int I = w + 4 * n;
        if (DN == 128) {
          const int r = 4 * I + (lane >> 4);
          return (uint32_t)(r * qn_st * 2 + ((lane & 15) ^ bsw256(r)) * 16);
        }
        const int r = 8 * I + (lane >> 3);
        return (uint32_t)(r * qn_st * 2 + ((lane & 7) ^ bsw128(r)) * 16);
      }
      if (n < C::MK_QN + C::MK_QR) {
        const int r = 8 * (w + 4 * (n - C::MK_QN)) + (lane >> 3);
        return (uint32_t)(r * qr_st * 2 + ((lane & 7) ^ bsw128(r)) * 16);
      }
      if (n < C::MK_QN + C::MK_QR + C::MK_DO) {
        const int r = 4 * (w + 4 * (n - C::MK_QN - C::MK_QR)) + (lane >> 4);
        return (uint32_t)(r * do_st * 2 + ((lane & 15) ^ bsw256(r)) * 16);
      }
      return (uint32_t)(16 * lane);
    };
    const uint32_t vl0 = load_voff(0), vl1 = C::NL > 1 ? load_voff(1) : 0u, vl2 = C::NL > 2 ? load_voff(2) : 0u,
                   vl3 = C::NL > 3 ? load_voff(3) : 0u, vl4 = C::NL > 4 ? load_voff(4) : 0u,
                   vl5 = C::NL > 5 ? load_voff(5) : 0u;
    struct BlockLoads {
      buf_rsrc rqn, rqr, rdo, rld;
      unsigned char* st;
    };
    auto block_loads = [&](int qb, unsigned char* st, bool live) {
      const int q0 = live ? qb * C::BQ : 0;
      const int nv = live ? min(p.Tq - q0, C::BQ) : 0;
      return BlockLoads{make_rsrc(qn_b + (int64_t)q0 * qn_st, rows_bytes(nv, qn_st, C::QN_RB)),
                        make_rsrc(qr_b + (int64_t)q0 * qr_st, rows_bytes(nv, qr_st, 128)),
                        make_rsrc(do_b + (int64_t)q0 * do_st, rows_bytes(nv, do_st, 256)),
                        make_rsrc(ld_b + (int64_t)(live ? qb : 0) * 64, live ? 256u : 0u), st};
    };
    auto issue = [&](const BlockLoads& bl, int n) {
      const uint32_t vo = n == 0 ? vl0 : n == 1 ? vl1 : n == 2 ? vl2 : n == 3 ? vl3 : n == 4 ? vl4 : vl5;
      if (n < C::MK_QN) {
        dma16(bl.rqn, vo, lds_addr(bl.st + 1024 * (w + 4 * n)));
      } else if (n < C::MK_QN + C::MK_QR) {
        dma16(bl.rqr, vo, lds_addr(bl.st + C::OFF_QR + 1024 * (w + 4 * (n - C::MK_QN))));
      } else if (n < C::MK_QN + C::MK_QR + C::MK_DO) {
        dma16(bl.rdo, vo, lds_addr(bl.st + C::OFF_DO + 1024 * (w + 4 * (n - C::MK_QN - C::MK_QR))));
      } else if (n < C::NL) {
        if (w == 0) dma16(bl.rld, vo, lds_addr(bl.st + C::OFF_LD));
      }
    };
    const int loads = C::NL - 1 + (w == 0 ? 1 : 0);
    auto load_block = [&](int j, unsigned char* st, int n_steps) {
      const BlockLoads bl = block_loads(nqb - 1 - j, st, j < n_steps);
#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(bl, n);
    };

    const int l16 = lane & 15;
    const int cl = 2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1), half8 = 8 * (l16 & 1);
    const int rlo = 4 * g + (l16 >> 2), rhi = rlo + 8;
    const int t_do_lo = C::OFF_DO + rlo * 256 + 16 * (cl ^ bsw256(rlo)) + half8;
    const int t_do_hi = C::OFF_DO + rhi * 256 + 16 * (cl ^ bsw256(rhi)) + half8;
    const int t_qn_lo = DN == 128 ? rlo * 256 + 16 * (cl ^ bsw256(rlo)) + half8 : rlo * 128 + 16 * (cl ^ bsw128(rlo)) + half8;
    const int t_qn_hi = DN == 128 ? rhi * 256 + 16 * (cl ^ bsw256(rhi)) + half8 : rhi * 128 + 16 * (cl ^ bsw128(rhi)) + half8;
    const int t_qr_lo = C::OFF_QR + rlo * 128 + 16 * (cl ^ bsw128(rlo)) + half8;
    const int t_qr_hi = C::OFF_QR + rhi * 128 + 16 * (cl ^ bsw128(rhi)) + half8;

    for (int item = 0; item < n_items; ++item) {
      int k0, n_steps;
      item_blocks(item, k0, n_steps);
      const int kw0 = k0 + 32 * kb;
      const int key = kw0 + l32;
      f32x16 dvacc[C::DV / 32], dkacc[C::NDQK];
#pragma unroll
      for (int i = 0; i < C::DV / 32; ++i) dvacc[i] = f32x16{};
#pragma unroll
      for (int i = 0; i < C::NDQK; ++i) dkacc[i] = f32x16{};

      auto consume = [&](int j, const unsigned char* st, const unsigned char* xb) {
        if (!visible(j, kw0)) return;
        const unsigned char* xs = xb + kb * 4096 + lane * 16;
        const bf16x8 pb0 = as_bf16x8(lds16(xs)), pb1 = as_bf16x8(lds16(xs + 1024));
        const bf16x8 db0 = as_bf16x8(lds16(xs + 2048)), db1 = as_bf16x8(lds16(xs + 3072));
        // the read addresses (base ^ constant, + an immediate offset) are loop-invariant and stay in
        // registers (246 in all): formed at each read, their 40 VALU instructions per block made the
        // backward 4 % slower, on the SIMD the producer's softmax shares
        auto tfrag = [&](int n) -> bf16x8 {  // n = NB2 s + m
          const int s = n / C::NB2, m = n % C::NB2;
          int lo, hi;
          if (m < C::DV / 32) {
            lo = (t_do_lo ^ (64 * m)) + 16 * s * 256;
            hi = (t_do_hi ^ (64 * m)) + 16 * s * 256;
          } else if (m - C::DV / 32 < C::NDN) {
            const int nb = m - C::DV / 32;
            lo = (t_qn_lo ^ (64 * nb)) + 16 * s * C::QN_RB;
            hi = (t_qn_hi ^ (64 * nb)) + 16 * s * C::QN_RB;
          } else {
            const int nb = m - C::DV / 32 - C::NDN;
            lo = (t_qr_lo ^ (64 * nb)) + 16 * s * 128;
            hi = (t_qr_hi ^ (64 * nb)) + 16 * s * 128;
          }
          const s16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(st + lo));
          const s16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(st + hi));
          const u32x2 l2 = __builtin_bit_cast(u32x2, vlo), h2 = __builtin_bit_cast(u32x2, vhi);
          return as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]});
        };
        constexpr int NM2 = 2 * C::NB2;
        bf16x8 t[NM2];
#pragma unroll
        for (int n = 0; n < BWD_T_AHEAD; ++n) t[n] = tfrag(n);
#pragma unroll
        for (int n = 0; n < NM2; ++n) {
          if (n + BWD_T_AHEAD < NM2) t[n + BWD_T_AHEAD] = tfrag(n + BWD_T_AHEAD);
          const int s = n / C::NB2, m = n % C::NB2;
          if (m < C::DV / 32) dvacc[m] = mfma32(t[n], s ? pb1 : pb0, dvacc[m]);
          else dkacc[m - C::DV / 32] = mfma32(t[n], s ? db1 : db0, dkacc[m - C::DV / 32]);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      // step j: block j is loaded (blocks j and j + 1 were in flight); after the barrier the
      // producers work on block j, this wave loads block j + 2 into the stage of block j - 2
      // and consumes block j - 1
      auto cstep = [&](int j, auto par_tag) {
        constexpr int P = decltype(par_tag)::value;
        wait_vmem(loads);
        __syncthreads();
        load_block(j + 2, stage(std::integral_constant<int, P + 2>{}), n_steps);
        if (j > 0) consume(j - 1, stage(std::integral_constant<int, P + 3>{}), P % 2 == 0 ? xch1 : xch0);
      };
      if (n_steps > 0) {
        load_block(0, stage(S0{}), n_steps);
        load_block(1, stage(S1{}), n_steps);
      }
      for (int j = 0; j < n_steps; j += 4) {
        cstep(j, S0{});
        if (j + 1 < n_steps) cstep(j + 1, S1{});
        if (j + 2 < n_steps) cstep(j + 2, S2{});
        if (j + 3 < n_steps) cstep(j + 3, S3{});
      }
      __syncthreads();  // the last block's P, dS are written
      if (n_steps > 0) consume(n_steps - 1, stage_at(n_steps - 1), (n_steps - 1) % 2 == 0 ? xch0 : xch1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // every wave is done with the stages

      // ---- store: lane = key; register r of block n holds column 32 n + 8 (r / 4) + 4 g + r % 4
      if (key < p.Tk) {
        bf16* dvp = p.dv + (int64_t)b * p.dv_s.b + (int64_t)key * p.dv_s.t + (int64_t)h * p.dv_s.h;
#pragma unroll
        for (int dvb = 0; dvb < C::DV / 32; ++dvb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            stg8(dvp + 32 * dvb + 8 * i + 4 * g,
                 u32x2{pack_bf16x2(dvacc[dvb][4 * i], dvacc[dvb][4 * i + 1]),
                       pack_bf16x2(dvacc[dvb][4 * i + 2], dvacc[dvb][4 * i + 3])});
        bf16* dkp = p.dkn + (int64_t)b * p.dkn_s.b + (int64_t)key * p.dkn_s.t + (int64_t)h * p.dkn_s.h;
#pragma unroll
        for (int nb = 0; nb < C::NDQK; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int col = 32 * nb + 8 * i + 4 * g;
            const float v0 = dkacc[nb][4 * i] * p.scale, v1 = dkacc[nb][4 * i + 1] * p.scale;
            const float v2 = dkacc[nb][4 * i + 2] * p.scale, v3 = dkacc[nb][4 * i + 3] * p.scale;
            if (col < DN) {
              stg8(dkp + col, u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)});
            } else if (p.shared_rope) {
              *reinterpret_cast<f32x4*>(p.dkr_ws + (((int64_t)b * p.Tk + key) * p.H + h) * 64 + (col - DN)) =
                  f32x4{v0, v1, v2, v3};
            } else {
              stg8(p.dkr + (int64_t)b * p.dkr_s.b + (int64_t)key * p.dkr_s.t + (int64_t)h * p.dkr_s.h + (col - DN),
                   u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)});
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- dQ (query-stationary)
// Workgroup = 4 waves x 32 queries (the lane's Q and dO rows stay in registers as the B
// operands of S^T and dP^T); the loop walks 32-key blocks of K_nope, K_rope and V written
// by buffer loads straight into LDS, through the same four-stage ring as the dK/dV kernel.
// Step j computes S^T = K Q^T and dP^T = V dO^T of block j, then P^T = 2^(S^T scale log2 e
// - LSE2) and dS^T = P^T (dP^T - D) (one query per lane, so LSE2 and D are per-lane
// scalars), then accumulates dQ^T += K^T dS^T with K^T read by ds_read_b64_tr_b16.  K
// tiles use the dual-purpose swizzles of the dK/dV kernel's Q tiles; V tiles are read by
// rows only.  The kernel fits 256 registers, so two workgroups share a CU and the two
// waves of a SIMD hide each other's softmax and load latency (no software pipelining of
// the scores, whose second set of accumulators would not fit).
//
// The per-k-step LDS addresses (base ^ constant) are formed where they are used
// (xor_at_use): kept in registers they would push the kernel past 256.
template <int DN>
struct DqCfg {
  static constexpr int DR = 64, DV = 128, DQK = DN + DR;
  static constexpr int KS = DQK / 16, KNS = DN / 16;
  static constexpr int NDQK = DQK / 32, NDN = DN / 32;
  static constexpr int BQQ = 128, BK = 32;            // queries per workgroup, keys per block
  static constexpr int KN_RB = DN * 2;
  static constexpr int OFF_KR = BK * KN_RB;           // stage: K_nope | K_rope | V
  static constexpr int OFF_V = OFF_KR + BK * 128;
  static constexpr int STAGE = OFF_V + BK * 256;
  static constexpr int T_KN = BK * KN_RB / 1024, T_KR = BK * 128 / 1024, T_V = BK * 256 / 1024;
  static constexpr int MK_KN = T_KN / 4, MK_KR = T_KR / 4, MK_V = T_V / 4;
  static constexpr int NL = MK_KN + MK_KR + MK_V;
  static constexpr int NM1 = KS + DV / 16;            // S^T and dP^T MFMAs per block
  static_assert(T_KN % 4 == 0 && T_KR % 4 == 0 && T_V % 4 == 0, "loads split evenly over 4 waves");
  static_assert(NL <= 6, "six load offsets are kept");
};

template <int DN>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(BwdParams p) {
  using C = DqCfg<DN>;
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage3[C::STAGE];
  auto stage = [&](auto s_tag) -> unsigned char* {
    constexpr int S = decltype(s_tag)::value % 4;
    return S == 0 ? stage0 : S == 1 ? stage1 : S == 2 ? stage2 : stage3;
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  const int n_qt = (p.Tq + C::BQQ - 1) / C::BQQ;
  int b, h, qt_a, qt_b, n_items;
  bwd_coords(n_qt, p.H, b, h, qt_b, qt_a, n_items);  // qt_a: the longer tile first
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(w >= 0 && w < 4);
  const int q_off = (int)p.q_offset;
  const int nqb = (p.Tq + 31) >> 5;
  const bf16* kn_b = p.kn + (int64_t)b * p.kn_s.b + (int64_t)h * p.kn_s.h;
  const bf16* kr_b = p.kr + (int64_t)b * p.kr_s.b + (int64_t)h * p.kr_s.h;
  const bf16* v_b = p.v + (int64_t)b * p.v_s.b + (int64_t)h * p.v_s.h;
  // key row strides (elements; the host keeps them below 2^24)
  const int kn_st = (int)p.kn_s.t, kr_st = (int)p.kr_s.t, v_st = (int)p.v_s.t;

  // The wave's loads of one block, n = 0 .. NL - 1: K_nope, K_rope, then V (load n of a
  // region is its 1 KiB load I = w + 4 k; layout as in the dK/dV kernel).
  auto load_voff = [&](int n) -> uint32_t {
    if (n < C::MK_KN) {
      const int I = w + 4 * n;
      if (DN == 128) {
        const int r = 4 * I + (lane >> 4);
        return (uint32_t)(r * kn_st * 2 + ((lane & 15) ^ bsw256(r)) * 16);
      }
      const int r = 8 * I + (lane >> 3);
      return (uint32_t)(r * kn_st * 2 + ((lane & 7) ^ bsw128(r)) * 16);
    }
    if (n < C::MK_KN + C::MK_KR) {
      const int r = 8 * (w + 4 * (n - C::MK_KN)) + (lane >> 3);
      return (uint32_t)(r * kr_st * 2 + ((lane & 7) ^ bsw128(r)) * 16);
    }
    const int r = 4 * (w + 4 * (n - C::MK_KN - C::MK_KR)) + (lane >> 4);
    return (uint32_t)(r * v_st * 2 + ((lane & 15) ^ bsw256(r)) * 16);
  };
  const uint32_t vl0 = load_voff(0), vl1 = C::NL > 1 ? load_voff(1) : 0u, vl2 = C::NL > 2 ? load_voff(2) : 0u,
                 vl3 = C::NL > 3 ? load_voff(3) : 0u, vl4 = C::NL > 4 ? load_voff(4) : 0u,
                 vl5 = C::NL > 5 ? load_voff(5) : 0u;
  // The loads of the key block at kv0 into a stage; tk = the end of the keys the q-tile
  // sees (0 for a block past it: no data, same count).  Lanes past the end write nothing:
  // such rows keep finite data and their p is masked to 0.
  struct BlockLoads {
    buf_rsrc rkn, rkr, rv;
    unsigned char* st;
  };
  auto block_loads = [&](int kv0, unsigned char* st, int tk) {
    const int nv = min(tk - kv0, C::BK);
    const int k_base = nv > 0 ? kv0 : 0;
    return BlockLoads{make_rsrc(kn_b + (int64_t)k_base * kn_st, rows_bytes(nv, kn_st, C::KN_RB)),
                      make_rsrc(kr_b + (int64_t)k_base * kr_st, rows_bytes(nv, kr_st, 128)),
                      make_rsrc(v_b + (int64_t)k_base * v_st, rows_bytes(nv, v_st, 256)), st};
  };
  auto issue = [&](const BlockLoads& bl, int n) {
    const uint32_t vo = n == 0 ? vl0 : n == 1 ? vl1 : n == 2 ? vl2 : n == 3 ? vl3 : n == 4 ? vl4 : vl5;
    if (n < C::MK_KN) {
      dma16(bl.rkn, vo, lds_addr(bl.st + 1024 * (w + 4 * n)));
    } else if (n < C::MK_KN + C::MK_KR) {
      dma16(bl.rkr, vo, lds_addr(bl.st + C::OFF_KR + 1024 * (w + 4 * (n - C::MK_KN))));
    } else if (n < C::NL) {
      dma16(bl.rv, vo, lds_addr(bl.st + C::OFF_V + 1024 * (w + 4 * (n - C::MK_KN - C::MK_KR))));
    }
  };
  constexpr int loads = C::NL;

  {
    const u32x4 z{0u, 0u, 0u, 0u};
    for (int i = tid; i < C::STAGE / 16; i += 256) {
      sts16(stage0 + 16 * i, z);
      sts16(stage1 + 16 * i, z);
      sts16(stage2 + 16 * i, z);
      sts16(stage3 + 16 * i, z);
    }
    __syncthreads();
  }

  // row reads (A of S^T and dP^T): key row l32, chunk 2 ks + g
  const int a_kn = DN == 128 ? l32 * 256 + 16 * (g ^ bsw256(l32)) : l32 * 128 + 16 * (g ^ bsw128(l32));
  const int a_kr = C::OFF_KR + l32 * 128 + 16 * (g ^ bsw128(l32));
  const int a_v = C::OFF_V + l32 * 256 + 16 * (g ^ bsw256(l32));
  // transpose reads (A of dQ^T = K^T): key rows 16 s + 4 g + r / 4 (+ 8), dims 32 nb + ...
  const int l16 = lane & 15;
  const int cl = 2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1), half8 = 8 * (l16 & 1);
  const int rlo = 4 * g + (l16 >> 2), rhi = rlo + 8;
  const int t_kn_lo = DN == 128 ? rlo * 256 + 16 * (cl ^ bsw256(rlo)) + half8 : rlo * 128 + 16 * (cl ^ bsw128(rlo)) + half8;
  const int t_kn_hi = DN == 128 ? rhi * 256 + 16 * (cl ^ bsw256(rhi)) + half8 : rhi * 128 + 16 * (cl ^ bsw128(rhi)) + half8;
  const int t_kr_lo = C::OFF_KR + rlo * 128 + 16 * (cl ^ bsw128(rlo)) + half8;
  const int t_kr_hi = C::OFF_KR + rhi * 128 + 16 * (cl ^ bsw128(rhi)) + half8;

  for (int item = 0; item < n_items; ++item) {
    const int qt = item == 0 ? qt_a : qt_b;
    const int q0 = qt * C::BQQ;
    const int qw0 = q0 + 32 * w;
    const int q_row = qw0 + l32;
    const int q_ld = q_row < p.Tq ? q_row : p.Tq - 1;

    // Q and dO rows of this lane's query (B operands), its LSE2 and D
    bf16x8 qf[C::KS], dof[C::DV / 16];
    float lse2, dsum;
    {
      const bf16* qn = p.qn + (int64_t)b * p.qn_s.b + (int64_t)q_ld * p.qn_s.t + (int64_t)h * p.qn_s.h;
      const bf16* qr = p.qr + (int64_t)b * p.qr_s.b + (int64_t)q_ld * p.qr_s.t + (int64_t)h * p.qr_s.h;
      const bf16* dop = p.dout + (int64_t)b * p.do_s.b + (int64_t)q_ld * p.do_s.t + (int64_t)h * p.do_s.h;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        const int d = 16 * ks + 8 * g;
        qf[ks] = as_bf16x8(d < DN ? ldg16(qn + d) : ldg16(qr + (d - DN)));
      }
#pragma unroll
      for (int ks = 0; ks < C::DV / 16; ++ks) dof[ks] = as_bf16x8(ldg16(dop + 16 * ks + 8 * g));
      const float* rec = p.ld + (((int64_t)b * p.H + h) * nqb + (q_ld >> 5)) * 64 + (q_ld & 31);
      lse2 = rec[0];
      dsum = rec[32];
    }

    // keys [0, kv_end) are seen by some query of the q-tile; lim: keys this lane's query sees
    int kv_end = p.Tk, lim = p.Tk;
    if (p.causal) {
      kv_end = (int)min((int64_t)p.Tk, (int64_t)q0 + C::BQQ + q_off);
      lim = min(p.Tk, q_row + q_off + 1);
    }
    const int wave_last = p.causal ? min(p.Tk - 1, qw0 + 31 + q_off) : p.Tk - 1;  // last key of the wave
    const int n_steps = (kv_end + C::BK - 1) / C::BK;

    f32x16 dqacc[C::NDQK];
#pragma unroll
    for (int i = 0; i < C::NDQK; ++i) dqacc[i] = f32x16{};

    if (n_steps > 0) {
      // A fragment of S^T / dP^T MFMA n (S and dP k-steps interleaved, then the rest of S)
      auto afrag = [&](const unsigned char* st, int n) -> bf16x8 {
        constexpr int NI = C::DV / 16;
        const bool is_dp = n < 2 * NI && (n & 1);
        const int ks = n < 2 * NI ? (n >> 1) : n - NI;
        if (is_dp) return as_bf16x8(lds16(st + xor_at_use(a_v, 32 * ks)));
        return as_bf16x8(lds16(st + (ks < C::KNS ? xor_at_use(a_kn, 32 * ks) : xor_at_use(a_kr, 32 * (ks - C::KNS)))));
      };

      // block j: S^T / dP^T (the next block's loads ride between the MFMAs), dS^T, dQ^T
      auto body = [&](int j, const unsigned char* cur, const BlockLoads& bl) {
        const int kv0 = j * C::BK;
        f32x16 sc = f32x16{}, dp = f32x16{};
        {
          bf16x8 a[C::NM1];
#pragma unroll
          for (int n = 0; n < BWD_S_AHEAD; ++n) a[n] = afrag(cur, n);
#pragma unroll
          for (int n = 0; n < C::NM1; ++n) {
            if (n + BWD_S_AHEAD < C::NM1) a[n + BWD_S_AHEAD] = afrag(cur, n + BWD_S_AHEAD);
            constexpr int NI = C::DV / 16;
            const int ks = n < 2 * NI ? (n >> 1) : n - NI;
            if (n < 2 * NI && (n & 1)) dp = mfma32(a[n], dof[ks], dp);
            else sc = mfma32(a[n], qf[ks], sc);
            if (n < C::NL) issue(bl, n);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        if (kv0 > wave_last) return;  // no key of the block is seen by this wave's queries
        // register r of S^T holds key kv0 + 8 (r / 4) + 4 g + r % 4 for this lane's query
        if ((p.causal && kv0 + C::BK - 1 > qw0 + q_off) || kv0 + C::BK > p.Tk) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kv = kv0 + 8 * (r >> 2) + 4 * g + (r & 3);
            sc[r] = kv < lim ? sc[r] : -INFINITY;
          }
        }
        // dS^T as the B operand of dQ^T += K^T dS^T: K slot (g, e) of operand s <-> key
        // 16 s + 8 (e / 4) + 4 g + e % 4, registers 8 s .. 8 s + 7
        uint32_t pkw[8];
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const float p0 = fast_exp2(__builtin_fmaf(sc[2 * n], p.scale_log2, -lse2));
          const float p1 = fast_exp2(__builtin_fmaf(sc[2 * n + 1], p.scale_log2, -lse2));
          pkw[n] = pack_bf16x2(p0 * (dp[2 * n] - dsum), p1 * (dp[2 * n + 1] - dsum));
        }
        const bf16x8 db0 = as_bf16x8(u32x4{pkw[0], pkw[1], pkw[2], pkw[3]});
        const bf16x8 db1 = as_bf16x8(u32x4{pkw[4], pkw[5], pkw[6], pkw[7]});
        auto tfrag = [&](int n) -> bf16x8 {  // n = NDQK s + nb
          const int s = n / C::NDQK, nb = n % C::NDQK;
          int lo, hi;
          if (nb < C::NDN) {
            lo = xor_at_use(t_kn_lo, 64 * nb) + 16 * s * C::KN_RB;
            hi = xor_at_use(t_kn_hi, 64 * nb) + 16 * s * C::KN_RB;
          } else {
            lo = xor_at_use(t_kr_lo, 64 * (nb - C::NDN)) + 16 * s * 128;
            hi = xor_at_use(t_kr_hi, 64 * (nb - C::NDN)) + 16 * s * 128;
          }
          const s16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + lo));
          const s16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + hi));
          const u32x2 l2 = __builtin_bit_cast(u32x2, vlo), h2 = __builtin_bit_cast(u32x2, vhi);
          return as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]});
        };
        constexpr int NM2 = 2 * C::NDQK;
        bf16x8 t[NM2];
#pragma unroll
        for (int n = 0; n < BWD_T_AHEAD; ++n) t[n] = tfrag(n);
#pragma unroll
        for (int n = 0; n < NM2; ++n) {
          if (n + BWD_T_AHEAD < NM2) t[n + BWD_T_AHEAD] = tfrag(n + BWD_T_AHEAD);
          const int s = n / C::NDQK, nb = n % C::NDQK;
          dqacc[nb] = mfma32(t[n], s ? db1 : db0, dqacc[nb]);
          __builtin_amdgcn_sched_barrier(0);
        }
      };

      // step j: entering it, the loads of blocks j .. j + 2 may be in flight; waiting until
      // at most two blocks' loads remain lands block j, and after the barrier every wave is
      // done with block j - 1, whose stage receives block j + 3.
      auto step = [&](int j, auto par_tag) {
        constexpr int P = decltype(par_tag)::value;
        const unsigned char* cur = stage(par_tag);
        unsigned char* fill = stage(std::integral_constant<int, P + 3>{});
        wait_vmem(2 * loads);
        __syncthreads();
        const int t = j + 3;
        body(j, cur, block_loads(t * C::BK, fill, t < n_steps ? kv_end : 0));
      };

#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(block_loads(0, stage(S0{}), kv_end), n);
#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(block_loads(C::BK, stage(S1{}), 1 < n_steps ? kv_end : 0), n);
#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(block_loads(2 * C::BK, stage(S2{}), 2 < n_steps ? kv_end : 0), n);

      for (int j = 0; j < n_steps; j += 4) {
        step(j, S0{});
        if (j + 1 < n_steps) step(j + 1, S1{});
        if (j + 2 < n_steps) step(j + 2, S2{});
        if (j + 3 < n_steps) step(j + 3, S3{});
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }

    // ---- store dQ (times scale): lane = query, registers = 4 consecutive dims per (nb, r / 4)
    if (q_row < p.Tq) {
      bf16* dqn = p.dqn + (int64_t)b * p.dqn_s.b + (int64_t)q_row * p.dqn_s.t + (int64_t)h * p.dqn_s.h;
      bf16* dqr = p.dqr + (int64_t)b * p.dqr_s.b + (int64_t)q_row * p.dqr_s.t + (int64_t)h * p.dqr_s.h;
      dq_scale_rope_back<DN / 32>(dqacc, p, q_row, g);
#pragma unroll
      for (int nb = 0; nb < C::NDQK; ++nb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * nb + 8 * i + 4 * g;
          const u32x2 v2{pack_bf16x2(dqacc[nb][4 * i], dqacc[nb][4 * i + 1]),
                         pack_bf16x2(dqacc[nb][4 * i + 2], dqacc[nb][4 * i + 3])};
          if (d < DN)
            stg8(dqn + d, v2);
          else
            stg8(dqr + (d - DN), v2);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- shared dk_rope = sum over heads
// Element idx of B * Tk * 16: (b, key, 4 columns); the heads' values are loaded together and
// added in head order.
__device__ __forceinline__ void dkrope_reduce_one(const BwdParams& p, int64_t idx) {
  const int c4 = (int)(idx & 15);
  const int64_t bt = idx >> 4;
  const int64_t t = bt % p.Tk, b = bt / p.Tk;
  const float* src = p.dkr_ws + (bt * p.H) * 64 + 4 * c4;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int h0 = 0; h0 < p.H; h0 += 16) {
    f32x4 v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (h0 + j < p.H) v[j] = *reinterpret_cast<const f32x4*>(src + (int64_t)(h0 + j) * 64);
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (h0 + j < p.H) acc += v[j];
  }
  bf16* dst = p.dkr + b * p.dkr_s.b + t * p.dkr_s.t + 4 * c4;
  stg8(dst, u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])});
}

// ---------------------------------------------------------------- dQ from the stored dS
// With the dS workspace, the dK/dV kernel's producers store every visible 32 x 32 dS block,
// and dQ = dS K scale needs no recomputation of S and dP: per block of 32 keys a wave runs
// 12 MFMAs instead of 32.  A block is 2 KiB laid out [s][key][g][8] (element (key, query q)
// at 512 s + 16 key + 8 g + 4 run + i for q = 16 s + 8 run + 4 g + i): the producer's
// registers go out in two contiguous 1 KiB stores, and every 4-query run of a key is 8
// contiguous bytes, which is what a transpose read takes from a lane.
//   dQ^T (DQK x 32q) += K^T . dS^T    A = K^T (transpose read of the K tile)
//                                     B = dS^T (transpose read of the stored block)
// Workgroup = 4 waves x 32 queries of one (b, h), mirrored pairs of q-tiles as in
// bwd_dq_kernel; a stage holds the K tile and the four waves' dS blocks of one key block.
template <int DN>
struct DqsCfg {
  static constexpr int DR = 64, DQK = DN + DR;
  static constexpr int NDQK = DQK / 32, NDN = DN / 32;
  static constexpr int BQQ = 128, BK = 32;
  static constexpr int KN_RB = DN * 2;
  static constexpr int OFF_KR = BK * KN_RB;         // stage: K_nope | K_rope | dS^T of waves 0..3
  static constexpr int OFF_DS = OFF_KR + BK * 128;
  static constexpr int STAGE = OFF_DS + 4 * 2048;
  static constexpr int T_KN = BK * KN_RB / 1024, T_KR = BK * 128 / 1024;
  static constexpr int MK_KN = T_KN / 4, MK_KR = T_KR / 4;
  static constexpr int NL = MK_KN + MK_KR + 2;     // K loads, then the wave's two dS loads
  static_assert(T_KN % 4 == 0 && T_KR % 4 == 0, "loads split evenly over 4 waves");
  static_assert(NL <= 6, "six load offsets are kept");
};

template <int DN>
__global__ __launch_bounds__(256, 2) void bwd_dq_ds_kernel(BwdParams p) {
  using C = DqsCfg<DN>;
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage3[C::STAGE];
  auto stage = [&](auto s_tag) -> unsigned char* {
    constexpr int S = decltype(s_tag)::value % 4;
    return S == 0 ? stage0 : S == 1 ? stage1 : S == 2 ? stage2 : stage3;
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  const int n_qt = (p.Tq + C::BQQ - 1) / C::BQQ;
  int b, h, qt_a, qt_b, n_items;
  bwd_coords(n_qt, p.H, b, h, qt_b, qt_a, n_items);  // qt_a: the longer tile first
  {
    // (b, h) in reverse order: the dK/dV pass walks each XCD's share of (b, h) upwards, so
    // the first workgroups here read the blocks it stored last, which may still sit in the
    // 256 MB last-level cache (config 4: dQ 294.7 -> 286.5 us)
    const int bh_r = p.B * p.H - 1 - (b * p.H + h);
    b = bh_r / p.H;
    h = bh_r - b * p.H;
  }
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(w >= 0 && w < 4);
  const int q_off = (int)p.q_offset;
  const int nqb = (p.Tq + 31) >> 5;
  const bf16* kn_b = p.kn + (int64_t)b * p.kn_s.b + (int64_t)h * p.kn_s.h;
  const bf16* kr_b = p.kr + (int64_t)b * p.kr_s.b + (int64_t)h * p.kr_s.h;
  const int kn_st = (int)p.kn_s.t, kr_st = (int)p.kr_s.t;

  // the wave's loads of one key block: K_nope, K_rope (load I = w + 4 k of a region, layout
  // as in bwd_dq_kernel), then its own dS block (two plain 1 KiB copies)
  auto load_voff = [&](int n) -> uint32_t {
    if (n < C::MK_KN) {
      const int I = w + 4 * n;
      if (DN == 128) {
        const int r = 4 * I + (lane >> 4);
        return (uint32_t)(r * kn_st * 2 + ((lane & 15) ^ bsw256(r)) * 16);
      }
      const int r = 8 * I + (lane >> 3);
      return (uint32_t)(r * kn_st * 2 + ((lane & 7) ^ bsw128(r)) * 16);
    }
    if (n < C::MK_KN + C::MK_KR) {
      const int r = 8 * (w + 4 * (n - C::MK_KN)) + (lane >> 3);
      return (uint32_t)(r * kr_st * 2 + ((lane & 7) ^ bsw128(r)) * 16);
    }
    return (uint32_t)(16 * lane + 1024 * (n - C::MK_KN - C::MK_KR));
  };
  const uint32_t vl0 = load_voff(0), vl1 = C::NL > 1 ? load_voff(1) : 0u, vl2 = C::NL > 2 ? load_voff(2) : 0u,
                 vl3 = C::NL > 3 ? load_voff(3) : 0u, vl4 = C::NL > 4 ? load_voff(4) : 0u,
                 vl5 = C::NL > 5 ? load_voff(5) : 0u;
  struct BlockLoads {
    buf_rsrc rkn, rkr, rds;
    unsigned char* st;
  };
  // key block at kv0 into a stage; tk = the end of the keys the q-tile sees (0: no K data);
  // ds: the wave's stored block (nullptr: nothing to copy).  Lanes past a descriptor's end
  // write nothing; such rows keep finite data and meet zero K rows or unused queries.
  auto block_loads = [&](int kv0, unsigned char* st, int tk, const bf16* ds) {
    const int nv = min(tk - kv0, C::BK);
    const int k_base = nv > 0 ? kv0 : 0;
    return BlockLoads{make_rsrc(kn_b + (int64_t)k_base * kn_st, rows_bytes(nv, kn_st, C::KN_RB)),
                      make_rsrc(kr_b + (int64_t)k_base * kr_st, rows_bytes(nv, kr_st, 128)),
                      make_rsrc(ds ? ds : p.ds_ws, ds ? 2048u : 0u), st};
  };
  auto issue = [&](const BlockLoads& bl, int n) {
    const uint32_t vo = n == 0 ? vl0 : n == 1 ? vl1 : n == 2 ? vl2 : n == 3 ? vl3 : n == 4 ? vl4 : vl5;
    if (n < C::MK_KN) {
      dma16(bl.rkn, vo, lds_addr(bl.st + 1024 * (w + 4 * n)));
    } else if (n < C::MK_KN + C::MK_KR) {
      dma16(bl.rkr, vo, lds_addr(bl.st + C::OFF_KR + 1024 * (w + 4 * (n - C::MK_KN))));
    } else if (n < C::NL) {
      dma16_nt(bl.rds, vo, lds_addr(bl.st + C::OFF_DS + 2048 * w + 1024 * (n - C::MK_KN - C::MK_KR)));
    }
  };
  constexpr int loads = C::NL;

  {
    const u32x4 z{0u, 0u, 0u, 0u};
    for (int i = tid; i < C::STAGE / 16; i += 256) {
      sts16(stage0 + 16 * i, z);
      sts16(stage1 + 16 * i, z);
      sts16(stage2 + 16 * i, z);
      sts16(stage3 + 16 * i, z);
    }
    __syncthreads();
  }

  // transpose reads.  K^T (A of dQ^T): key rows 16 s + 4 g + r / 4 (+ 8), dims 32 nb + ...
  // dS^T (B): keys 16 s + 4 g + r / 4 (+ 8), queries 16 nh + 4 (r % 4) + [0, 4) with
  // nh = (lane >> 4) & 1, i.e. block half nh, run (r % 4) / 2, g slot r % 2
  const int l16 = lane & 15;
  const int cl = 2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1), half8 = 8 * (l16 & 1);
  const int rlo = 4 * g + (l16 >> 2), rhi = rlo + 8;
  const int t_kn_lo = DN == 128 ? rlo * 256 + 16 * (cl ^ bsw256(rlo)) + half8 : rlo * 128 + 16 * (cl ^ bsw128(rlo)) + half8;
  const int t_kn_hi = DN == 128 ? rhi * 256 + 16 * (cl ^ bsw256(rhi)) + half8 : rhi * 128 + 16 * (cl ^ bsw128(rhi)) + half8;
  const int t_kr_lo = C::OFF_KR + rlo * 128 + 16 * (cl ^ bsw128(rlo)) + half8;
  const int t_kr_hi = C::OFF_KR + rhi * 128 + 16 * (cl ^ bsw128(rhi)) + half8;
  const int t_ds = C::OFF_DS + 1024 * ((lane >> 4) & 1) + rlo * 32 + 16 * (l16 & 1) + 8 * ((l16 >> 1) & 1);

  // The wave's share of the q-tile's dQ^T: QBW blocks of 32 queries (QBW wq + [0, QBW)) by
  // NBW blocks of 32 dims (NBW wd + [0, NBW)).  With two of each per wave (a 2 x 2 grid of
  // waves) a step reads 4 dS^T and 6 K^T fragments per wave instead of 2 and 12: each
  // fragment feeds two MFMAs, for the same 96 accumulator registers.  Every accumulator sees
  // the same MFMAs in the same order in both forms.
  constexpr int QBW = BWD_DQ_QBW, NBW = C::NDQK / QBW, NT = 2 * NBW;
  static_assert(C::NDQK % QBW == 0 && 4 % QBW == 0, "the waves tile the q-tile's dQ");
  static_assert(QBW == 1 || (C::NDN >= NBW && C::NDN + 1 < 2 * NBW), "the rope dims are in the second dim half");
  const int wq = QBW == 1 ? w : w >> 1, wd = QBW == 1 ? 0 : w & 1;

  for (int item = 0; item < n_items; ++item) {
    const int qt = item == 0 ? qt_a : qt_b;
    const int q0 = qt * C::BQQ;
    int kv_end = p.Tk;
    if (p.causal) kv_end = (int)min((int64_t)p.Tk, (int64_t)q0 + C::BQQ + q_off);
    const int n_steps = (kv_end + C::BK - 1) / C::BK;
    // query block x (queries q0 + 32 x + [0, 32)): its first stored block (nullptr past Tq)
    // and the last key its queries see
    struct DsRow {
      const bf16* base;
      int last;
    };
    auto ds_row = [&](int x) {
      const int qx0 = q0 + 32 * x;
      const int last = p.causal ? min(p.Tk - 1, qx0 + 31 + q_off) : p.Tk - 1;
      const bf16* base = qx0 < p.Tq ? p.ds_ws + (((int64_t)b * p.H + h) * p.ds_bh_blocks +
                                                 ds_prefix(qx0 >> 5, p.nkb32, p.q_offset, p.causal)) * 1024
                                    : nullptr;
      return DsRow{base, last};
    };
    // wave w loads query block w's stored blocks; it reads those of blocks QBW wq + [0, QBW)
    const DsRow ld_row = ds_row(w);
    DsRow rd_row[QBW];
#pragma unroll
    for (int i = 0; i < QBW; ++i) rd_row[i] = QBW == 1 ? ld_row : ds_row(QBW * wq + i);
    // the stored block at key block j, or nullptr where no query of the block sees its keys
    auto ds_at = [&](int j) -> const bf16* {
      return ld_row.base && j * C::BK <= ld_row.last && j < n_steps ? ld_row.base + (int64_t)j * 1024 : nullptr;
    };

    f32x16 dqacc[QBW][NBW];
#pragma unroll
    for (int i = 0; i < QBW; ++i)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) dqacc[i][nb] = f32x16{};

    if (n_steps > 0) {
      auto body = [&](int j, const unsigned char* cur, const BlockLoads& bl) {
        bool av[QBW], any = false;  // block QBW wq + i has a stored block at j
#pragma unroll
        for (int i = 0; i < QBW; ++i) {
          av[i] = rd_row[i].base && j * C::BK <= rd_row[i].last;
          any |= av[i];
        }
        if (!any) {
#pragma unroll
          for (int n = 0; n < C::NL; ++n) issue(bl, n);
          return;
        }
        auto dfrag = [&](int i, int s) -> bf16x8 {
          const unsigned char* a = cur + t_ds + 2048 * (QBW * wq + i) + 512 * s;
          const s16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a);
          const s16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a + 256));
          const u32x2 l2 = __builtin_bit_cast(u32x2, vlo), h2 = __builtin_bit_cast(u32x2, vhi);
          // a block without stored data holds stale (finite) LDS: its queries take zeros
          return av[i] ? as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]}) : as_bf16x8(u32x4{0u, 0u, 0u, 0u});
        };
        // loop-invariant read addresses, kept in registers (255 in all; formed at each read they
        // cost 24 VALU instructions per step, 0.4 % of the backward)
        auto tfrag = [&](int n) -> bf16x8 {  // n = NBW s + local dim block
          const int s = n / NBW, nb = NBW * wd + n % NBW;
          int lo, hi;
          if (nb < C::NDN) {
            lo = (t_kn_lo ^ (64 * nb)) + 16 * s * C::KN_RB;
            hi = (t_kn_hi ^ (64 * nb)) + 16 * s * C::KN_RB;
          } else {
            lo = (t_kr_lo ^ (64 * (nb - C::NDN))) + 16 * s * 128;
            hi = (t_kr_hi ^ (64 * (nb - C::NDN))) + 16 * s * 128;
          }
          const s16x4 vlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + lo));
          const s16x4 vhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + hi));
          const u32x2 l2 = __builtin_bit_cast(u32x2, vlo), h2 = __builtin_bit_cast(u32x2, vhi);
          return as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]});
        };
        bf16x8 db[QBW][2];
#pragma unroll
        for (int i = 0; i < QBW; ++i) {
          db[i][0] = dfrag(i, 0);
          db[i][1] = dfrag(i, 1);
        }
        bf16x8 t[NT];
#pragma unroll
        for (int n = 0; n < BWD_T_AHEAD; ++n) t[n] = tfrag(n);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          if (n + BWD_T_AHEAD < NT) t[n + BWD_T_AHEAD] = tfrag(n + BWD_T_AHEAD);
          const int s = n / NBW, nb = n % NBW;
#pragma unroll
          for (int i = 0; i < QBW; ++i) dqacc[i][nb] = mfma32(t[n], db[i][s], dqacc[i][nb]);
          if (n < C::NL) issue(bl, n);  // the next blocks' loads ride between the MFMAs
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int n = NT; n < C::NL; ++n) issue(bl, n);
      };

      // step j: blocks j .. j + 2 may be in flight; waiting until at most two blocks' loads
      // remain lands block j, and after the barrier every wave is done with block j - 1, whose
      // stage receives block j + 3
      auto step = [&](int j, auto par_tag) {
        constexpr int P = decltype(par_tag)::value;
        const unsigned char* cur = stage(par_tag);
        unsigned char* fill = stage(std::integral_constant<int, P + 3>{});
        wait_vmem(2 * loads);
        __syncthreads();
        const int t = j + 3;
        body(j, cur, block_loads(t * C::BK, fill, t < n_steps ? kv_end : 0, ds_at(t)));
      };

#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(block_loads(0, stage(S0{}), kv_end, ds_at(0)), n);
#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(block_loads(C::BK, stage(S1{}), 1 < n_steps ? kv_end : 0, ds_at(1)), n);
#pragma unroll
      for (int n = 0; n < C::NL; ++n) issue(block_loads(2 * C::BK, stage(S2{}), 2 < n_steps ? kv_end : 0, ds_at(2)), n);

      for (int j = 0; j < n_steps; j += 4) {
        step(j, S0{});
        if (j + 1 < n_steps) step(j + 1, S1{});
        if (j + 2 < n_steps) step(j + 2, S2{});
        if (j + 3 < n_steps) step(j + 3, S3{});
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }

    // ---- store dQ (times scale): lane = query, registers = 4 consecutive dims per (nb, r / 4)
#pragma unroll
    for (int i = 0; i < QBW; ++i) {
      const int q_row = q0 + 32 * (QBW * wq + i) + l32;
      if (q_row < p.Tq) {
        bf16* dqn = p.dqn + (int64_t)b * p.dqn_s.b + (int64_t)q_row * p.dqn_s.t + (int64_t)h * p.dqn_s.h;
        bf16* dqr = p.dqr + (int64_t)b * p.dqr_s.b + (int64_t)q_row * p.dqr_s.t + (int64_t)h * p.dqr_s.h;
        if (QBW == 1 || wd == 1)  // the rope blocks NDN, NDN + 1 are local NDN - NBW wd, + 1
          dq_scale_rope_back<C::NDN - NBW * (QBW == 1 ? 0 : 1)>(dqacc[i], p, q_row, g);
        else
          dq_scale_rope_back<-1>(dqacc[i], p, q_row, g);
#pragma unroll
        for (int nbl = 0; nbl < NBW; ++nbl) {
          const int nb = NBW * wd + nbl;
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int d = 32 * nb + 8 * r4 + 4 * g;
            const u32x2 v2{pack_bf16x2(dqacc[i][nbl][4 * r4], dqacc[i][nbl][4 * r4 + 1]),
                           pack_bf16x2(dqacc[i][nbl][4 * r4 + 2], dqacc[i][nbl][4 * r4 + 3])};
            if (d < DN)
              stg8(dqn + d, v2);
            else
              stg8(dqr + (d - DN), v2);
          }
        }
      }
    }
  }
  // the shared k_rope head's sum over heads (the dK/dV pass, which wrote the per-head rows, has
  // finished): the workgroups take its elements in turn, so the early finishers do most of it
  // while the rest still run, instead of a launch of its own after this one
  if (p.shared_rope) {
    const int64_t n = (int64_t)p.B * p.Tk * 16;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * 256)
      dkrope_reduce_one(p, idx);
  }
}

// The same head sum as a kernel of its own, after the recomputing dQ kernel: one thread per
// element.
__global__ __launch_bounds__(256) void bwd_dkrope_reduce_kernel(BwdParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over B * Tk * 16
  if (idx < (int64_t)p.B * p.Tk * 16) dkrope_reduce_one(p, idx);
}

template <int DN>
static int launch_bwd(const BwdParams& prm, hipStream_t s) {
  // every grid is checked before the first launch, so a rejected call does no work
  const int64_t n_rec = (int64_t)prm.B * prm.H * ((prm.Tq + 31) / 32);  // 32-query records
  const int64_t n_kt = (prm.Tk + DkdvCfg<DN>::BKV - 1) / DkdvCfg<DN>::BKV;
  const int64_t n_qt = (prm.Tq + DqCfg<DN>::BQQ - 1) / DqCfg<DN>::BQQ;
  const int64_t n_rope = prm.shared_rope ? (int64_t)prm.B * prm.Tk * 16 : 0;
  MLA_CHECK(n_rec < (1ll << 31) && (int64_t)prm.B * prm.H * n_kt < (1ll << 31) &&
                (int64_t)prm.B * prm.H * n_qt < (1ll << 31) && (n_rope + 255) / 256 < (1ll << 31),
            MLA_ERR_INVALID_ARG, "mla_prefill_bwd: grid too large");
  if (n_rec > 0) bwd_rowdot_kernel<<<dim3((unsigned)n_rec), dim3(256), 0, s>>>(prm);
  bwd_dkdv_kernel<DN><<<dim3((unsigned)(prm.B * prm.H * ((n_kt + 1) / 2))), dim3(512), 0, s>>>(prm);
  if (prm.ds_ws)
    bwd_dq_ds_kernel<DN><<<dim3((unsigned)(prm.B * prm.H * ((n_qt + 1) / 2))), dim3(256), 0, s>>>(prm);
  else
    bwd_dq_kernel<DN><<<dim3((unsigned)(prm.B * prm.H * ((n_qt + 1) / 2))), dim3(256), 0, s>>>(prm);
  if (n_rope > 0 && !prm.ds_ws)  // with the stored dS the dQ kernel runs it in its tail
    bwd_dkrope_reduce_kernel<<<dim3((unsigned)((n_rope + 255) / 256)), dim3(256), 0, s>>>(prm);
  return launch_status("mla_prefill_bwd");
}

// Workspace: the LSE / D records, the per-head dk_rope (shared k_rope), then the stored dS
// blocks (2 KiB per 32 x 32 block of every (b, h)).  The dS part is offered while it stays
// at or below kDsCap; a call whose workspace lacks it recomputes S and dP for dQ instead.
constexpr size_t kDsCap = (size_t)8 << 30;
static void bwd_ws_layout(const mla_prefill_bwd_args* a, size_t& d_bytes, size_t& ws_rope, size_t& ds_off,
                          size_t& ds_bytes) {
  d_bytes = (((size_t)a->B * a->H * ((a->Tq + 31) / 32) * 64 * sizeof(float)) + 255) & ~(size_t)255;
  const bool shared = a->k_rope_stride.h == 0 && a->H > 1;
  ws_rope = shared ? (size_t)a->B * a->Tk * a->H * 64 * sizeof(float) : 0;
  ds_off = (d_bytes + ws_rope + 255) & ~(size_t)255;
  // compared before it is multiplied out, so no product can wrap
  const int64_t per_bh = ds_prefix((a->Tq + 31) / 32, (a->Tk + 31) / 32, a->q_offset, a->causal != 0);
  const int64_t bh = a->B * a->H;
  ds_bytes = per_bh <= (int64_t)(kDsCap / 2048) / bh ? (size_t)bh * (size_t)per_bh * 2048 : 0;
}

// The sizes mla_prefill_bwd accepts (without its pointer and stride checks), tested before any
// arithmetic on them: the workspace queries answer 0 for anything else.
static bool bwd_sizes_ok(const mla_prefill_bwd_args* a) {
  if (a->B <= 0 || a->H <= 0 || a->Tq <= 0 || a->Tk <= 0 || a->B >= (1 << 20) || a->H >= (1 << 16) ||
      a->Tq >= (1 << 30) || a->Tk >= (1 << 30) || (a->causal && a->q_offset < 0) || a->q_offset >= (1 << 30))
    return false;
  const int64_t bh = a->B * a->H;
  return bh * ((a->Tq + 31) / 32) < (1ll << 31) && bh * ((a->Tk + 127) / 128) < (1ll << 31) &&
         bh * ((a->Tq + 127) / 128) < (1ll << 31) && a->B * a->Tk * 16 / 256 < (1ll << 31);
}

}  // namespace mla

using namespace mla;

extern "C" size_t mla_prefill_bwd_workspace_bytes(const mla_prefill_bwd_args* a) {
  if (!a || !bwd_sizes_ok(a)) return 0;
  size_t d, r, off, ds;
  bwd_ws_layout(a, d, r, off, ds);
  return ds ? off + ds : d + r;
}

extern "C" size_t mla_prefill_bwd_workspace_min_bytes(const mla_prefill_bwd_args* a) {
  if (!a || !bwd_sizes_ok(a)) return 0;
  size_t d, r, off, ds;
  bwd_ws_layout(a, d, r, off, ds);
  return d + r;
}

extern "C" int mla_prefill_bwd(const mla_prefill_bwd_args* a, void* stream) {
  const char* op = "mla_prefill_bwd";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_TRY(check_scale(op, a->scale));
  MLA_CHECK(a->d_rope == 64 && a->d_v == 128 && (a->d_nope == 128 || a->d_nope == 64), MLA_ERR_UNSUPPORTED,
            "%s: head dims (nope %lld, rope %lld, v %lld) not built", op, (long long)a->d_nope,
            (long long)a->d_rope, (long long)a->d_v);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->Tq >= 0 && a->Tk >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->B < (1 << 20) && a->H < (1 << 16) && a->Tq < (1 << 30) && a->Tk < (1 << 30), MLA_ERR_INVALID_ARG,
            "%s: size out of range", op);
  if (a->B == 0 || a->H == 0 || (a->Tq == 0 && a->Tk == 0)) return MLA_OK;
  MLA_CHECK(a->Tq > 0 && a->Tk > 0, MLA_ERR_INVALID_ARG, "%s: Tq and Tk must be positive", op);
  MLA_CHECK(!a->causal || a->q_offset >= 0, MLA_ERR_INVALID_ARG, "%s: q_offset must be >= 0", op);
  MLA_CHECK(a->q_offset < (1 << 30), MLA_ERR_INVALID_ARG, "%s: q_offset out of range", op);
  MLA_CHECK(a->q_nope_stride.t < (1 << 24) && a->q_rope_stride.t < (1 << 24) && a->dout_stride.t < (1 << 24),
            MLA_ERR_INVALID_ARG, "%s: query row strides must be below 2^24 elements", op);
  MLA_TRY(check_operand(op, "dout", a->dout, a->dout_stride));
  MLA_TRY(check_operand(op, "q_nope", a->q_nope, a->q_nope_stride));
  MLA_TRY(check_operand(op, "q_rope", a->q_rope, a->q_rope_stride));
  MLA_TRY(check_operand(op, "k_nope", a->k_nope, a->k_nope_stride));
  MLA_TRY(check_operand(op, "k_rope", a->k_rope, a->k_rope_stride));
  MLA_TRY(check_operand(op, "v", a->v, a->v_stride));
  MLA_TRY(check_operand(op, "o", a->o, a->o_stride));
  MLA_TRY(check_operand(op, "dq_nope", a->dq_nope, a->dq_nope_stride));
  MLA_TRY(check_operand(op, "dq_rope", a->dq_rope, a->dq_rope_stride));
  MLA_TRY(check_operand(op, "dk_nope", a->dk_nope, a->dk_nope_stride));
  MLA_TRY(check_operand(op, "dk_rope", a->dk_rope, a->dk_rope_stride));
  MLA_TRY(check_operand(op, "dv", a->dv, a->dv_stride));
  MLA_CHECK(a->lse, MLA_ERR_INVALID_ARG, "%s: lse is null", op);
  MLA_CHECK(!a->rope_cos == !a->rope_sin, MLA_ERR_INVALID_ARG, "%s: rope_cos and rope_sin go together", op);
  if (a->rope_cos) {
    MLA_CHECK(((uintptr_t)a->rope_cos & 7) == 0 && ((uintptr_t)a->rope_sin & 7) == 0, MLA_ERR_INVALID_ARG,
              "%s: RoPE tables must be 8-byte aligned", op);
    MLA_CHECK(a->q_pos_offset >= 0 && a->q_pos_offset + a->Tq <= a->rope_rows, MLA_ERR_INVALID_ARG,
              "%s: query positions %lld..%lld exceed the RoPE table (%lld rows)", op, (long long)a->q_pos_offset,
              (long long)(a->q_pos_offset + a->Tq - 1), (long long)a->rope_rows);
  }
  const bool shared = a->k_rope_stride.h == 0 && a->H > 1;
  MLA_CHECK(!shared || a->dk_rope_stride.h == 0, MLA_ERR_INVALID_ARG,
            "%s: a shared k_rope needs a shared dk_rope (head stride 0)", op);
  size_t d_bytes, ws_rope, ds_off, ds_bytes;
  bwd_ws_layout(a, d_bytes, ws_rope, ds_off, ds_bytes);
  MLA_CHECK(a->workspace && a->workspace_bytes >= d_bytes + ws_rope, MLA_ERR_WORKSPACE,
            "%s: workspace of %zu bytes required (got %zu)", op, d_bytes + ws_rope, a->workspace_bytes);
  MLA_CHECK(((uintptr_t)a->workspace & 255) == 0, MLA_ERR_WORKSPACE, "%s: workspace must be 256-byte aligned", op);

  BwdParams prm;
  prm.dout = (const bf16*)a->dout;
  prm.qn = (const bf16*)a->q_nope;
  prm.qr = (const bf16*)a->q_rope;
  prm.kn = (const bf16*)a->k_nope;
  prm.kr = (const bf16*)a->k_rope;
  prm.v = (const bf16*)a->v;
  prm.o = (const bf16*)a->o;
  prm.lse = a->lse;
  prm.dqn = (bf16*)a->dq_nope;
  prm.dqr = (bf16*)a->dq_rope;
  prm.dkn = (bf16*)a->dk_nope;
  prm.dkr = (bf16*)a->dk_rope;
  prm.dv = (bf16*)a->dv;
  prm.ld = (float*)a->workspace;
  prm.dkr_ws = shared ? (float*)((char*)a->workspace + d_bytes) : nullptr;
  // dQ from stored dS when the workspace holds the blocks, else recomputed
  const bool store_ds = ds_bytes > 0 && a->workspace_bytes >= ds_off + ds_bytes;
  prm.ds_ws = store_ds ? (bf16*)((char*)a->workspace + ds_off) : nullptr;
  prm.nkb32 = (int)((a->Tk + 31) / 32);
  prm.ds_bh_blocks = ds_prefix((a->Tq + 31) / 32, prm.nkb32, a->q_offset, a->causal != 0);
  prm.ds_e = (int)((31 + (a->q_offset > 0 ? a->q_offset : 0)) / 32);
  prm.B = (int)a->B;
  prm.H = (int)a->H;
  prm.Tq = (int)a->Tq;
  prm.Tk = (int)a->Tk;
  prm.shared_rope = shared ? 1 : 0;
  prm.do_s = a->dout_stride;
  prm.qn_s = a->q_nope_stride;
  prm.qr_s = a->q_rope_stride;
  prm.kn_s = a->k_nope_stride;
  prm.kr_s = a->k_rope_stride;
  prm.v_s = a->v_stride;
  prm.o_s = a->o_stride;
  prm.dqn_s = a->dq_nope_stride;
  prm.dqr_s = a->dq_rope_stride;
  prm.dkn_s = a->dk_nope_stride;
  prm.dkr_s = a->dk_rope_stride;
  prm.dv_s = a->dv_stride;
  prm.scale = a->scale;
  prm.scale_log2 = a->scale * kLog2e;
  prm.causal = a->causal ? 1 : 0;
  prm.q_offset = a->q_offset;
  prm.rope_cos = (const bf16*)a->rope_cos;
  prm.rope_sin = (const bf16*)a->rope_sin;
  prm.q_pos_offset = a->q_pos_offset;
  hipStream_t s = (hipStream_t)stream;
  return a->d_nope == 128 ? launch_bwd<128>(prm, s) : launch_bwd<64>(prm, s);
}
