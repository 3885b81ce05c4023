// Causal flash-attention forward over the decoupled-RoPE MLA heads (gfx950).
//
// Computes, per (batch b, head h):
//   S = (q_nope k_nope^T + q_rope k_rope^T) * scale,  S[i][j] = -inf if causal and
//   j > i + q_offset;  O = softmax(S) V;  LSE = log(sum_j exp S[i][j]).
// This is F.scaled_dot_product_attention(cat[q_nope,q_rope], cat[k_nope,k_rope], v,
// is_causal=True) at transformer.py:311-314 (q_offset = 0), and the absorbed branch's
// bottom-right mask triu(diagonal = pos_offset + 1) at transformer.py:273-281.
//
// Work decomposition: one workgroup = 4 waves = 128 query rows of one (b, h);
// each wave owns 32 query rows and keeps its Q fragment in registers.  The key
// loop walks 64-key tiles that buffer loads write straight into LDS (no staging
// registers), double-buffered: tile j + 1 streams into one stage while tile j is
// consumed from the other, one barrier per tile.
//
// Per 64-key tile and wave:
//   S^T (64 x 32)  = K (64 x DQK) . Q^T (DQK x 32)     2 x DQK/16 MFMA 32x32x16
//   O^T (128 x 32) += V^T (128 x 64) . P^T (64 x 32)   4 x 4     MFMA 32x32x16
// Computing S^T rather than S puts one query row per lane (column of the MFMA
// output), so the running max / sum / rescale of the online softmax are per-lane
// scalars; the row max needs one cross-lane exchange (lanes l and l ^ 32).
// P^T goes straight from the S^T accumulators into the PV MFMA's B operand; V^T comes
// from row-major V through ds_read_b64_tr_b16.
#include <type_traits>

#include "mla_common.h"

namespace mla {

struct FwdParams {
  const bf16 *qn, *qr, *kn, *kr, *v;
  bf16* o;
  float* lse;
  int B, H, Tq, Tk, n_qt;
  mla_strides qn_s, qr_s, kn_s, kr_s, v_s, o_s;
  float scale_log2;  // scale * log2(e)
  int causal;
  int64_t q_offset;
};

// LDS stage of one 64-key tile: three row-major regions, rows unpadded (a direct-to-LDS
// load writes 64 lanes x 16 bytes contiguously), chunks XOR-swizzled per row:
//   K_nope [64][DN]  (DN = 128: 256-byte rows; DN = 64: 128-byte rows)
//   K_rope [64][64]  (128-byte rows)
//   V      [64][128] (256-byte rows)
template <int DN>
struct FwdCfg {
  static constexpr int DR = 64, DV = 128, DQK = DN + DR;
  static constexpr int BM = 128, BN = 64;
  static constexpr int KS = DQK / 16;   // MFMA k-steps of S^T
  static constexpr int KNS = DN / 16;   // of which over the nope dims
  static constexpr int KN_RB = DN * 2;  // K_nope row bytes
  static constexpr int OFF_KR = BN * KN_RB;
  static constexpr int OFF_V = OFF_KR + BN * 128;
  static constexpr int STAGE = OFF_V + BN * 256;
  // 1 KiB direct-to-LDS loads per tile and wave (wave w issues loads w, w + 4, ...)
  static constexpr int N_KN = BN * KN_RB / 1024 / 4, N_KR = BN * 128 / 1024 / 4, N_V = BN * 256 / 1024 / 4;
};

// Chunk swizzles (a row's 16-byte chunk c sits at position c ^ f(row)):
//  - 256-byte rows read by rows (K_nope, DN = 128): f = row mod 16, so the 16 rows that one
//    16-lane group reads at one chunk fall on 16 distinct 16-byte bank groups;
//  - 128-byte rows read by rows (K_rope, K_nope for DN = 64): f = (row ^ row / 8) mod 8,
//    distinct over any 8 consecutive rows and, paired with row parity, over 16;
//  - V (256-byte rows, transpose reads of 4 rows x 4 chunks per 32 lanes): f = 4 (row mod 4).
__device__ __forceinline__ int swz256(int r) { return r & 15; }
__device__ __forceinline__ int swz128(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int swzv(int r) { return 4 * (r & 3); }

// growth of a row's running max (log2 units) that triggers a rescale of O (safe form)
constexpr float kFwdRescale = 8.0f;
// a row sum beyond this (or not finite) under the fixed reference max sends the q-tile to
// the safe form; p <= 2^127 per key keeps every finite sum of the fast form exact up to it
constexpr float kFwdSumLimit = 0x1p120f;

// Maps the linear workgroup id to (b, h) and its pair of q-tiles.  A workgroup runs q-tiles
// n_qt - 1 - r and r of one (b, h) back to back: with causal masking the pair always
// totals the same number of key tiles (balanced workgroups, no tail of short tiles) and
// the second tile's first K/V tile (keys 0..63, shared by both) is prefetched during the
// first one.  Workgroups are dispatched round-robin over the 8 XCDs (id % 8);
// renumbering so each XCD receives a contiguous range keeps the K/V of a (b, h) in that
// XCD's L2.
__device__ __forceinline__ void fwd_tile_coords(const FwdParams& p, int& b, int& h, int& qa, int& qb_, int& n_items) {
  const int n = gridDim.x;
  int id = blockIdx.x;
  if ((n & 7) == 0) id = (id & 7) * (n >> 3) + (id >> 3);
  const int n_pairs = (p.n_qt + 1) >> 1;
  const int bh = id / n_pairs;
  const int r = id - bh * n_pairs;
  qa = p.n_qt - 1 - r;  // the longer tile first
  qb_ = r;
  n_items = qa == qb_ ? 1 : 2;
  b = bh / p.H;
  h = bh - b * p.H;
}

typedef __attribute__((address_space(3))) void lds_void;

// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSgMfma = 0x008, kSgDsRead = 0x100;
#ifndef S_AHEAD
#define S_AHEAD 4  // S^T A fragments in flight ahead of their MFMA
#endif
#ifndef PV_AHEAD
#define PV_AHEAD 3  // V^T fragments (two transpose reads each) in flight ahead of their MFMA
#endif

// x, with the compiler unable to see its value (keeps address arithmetic in the loop)
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// One 1 KiB direct-to-LDS load: lane l's 16 bytes land at lds + 16 l.
__device__ __forceinline__ void dma16(buf_rsrc r, uint32_t voff, lds_void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, (int)voff, 0, 0, 0);
}

template <int DN>
__global__ __launch_bounds__(256, 2) void prefill_fwd_kernel(FwdParams p) {
  using C = FwdCfg<DN>;
  // the two stages are separate objects so the compiler sees that reads of one do not
  // wait for loads into the other
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[C::STAGE];

  int b, h, qt_first, qt_second, n_items;
  fwd_tile_coords(p, b, h, qt_first, qt_second, n_items);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int q_off = (int)p.q_offset;  // the host keeps q_offset < 2^30
  const bf16* kn_b = p.kn + (int64_t)b * p.kn_s.b + (int64_t)h * p.kn_s.h;
  const bf16* kr_b = p.kr + (int64_t)b * p.kr_s.b + (int64_t)h * p.kr_s.h;
  const bf16* v_b = p.v + (int64_t)b * p.v_s.b + (int64_t)h * p.v_s.h;

  // Zero both stages once: rows past Tk are never loaded, and what they hold must be finite
  // (their scores are masked; their V rows meet p = 0).
  {
    const u32x4 z{0u, 0u, 0u, 0u};
    for (int i = tid; i < C::STAGE / 16; i += 256) {
      sts16(stage0 + 16 * i, z);
      sts16(stage1 + 16 * i, z);
    }
  }

  // Global byte offsets of this lane's 16 bytes for each of the wave's loads.  Load I of a
  // region covers rows RPI I .. RPI I + RPI - 1 (RPI = 1024 / row bytes) and is based at
  // its first row; lane l writes LDS position l % (row chunks) of row RPI I + l / (row
  // chunks), which holds logical chunk position ^ f(row).
  // With 256-byte rows, load I = w + 4 k covers rows 4 I + [0, 4): row mod 16 = 4 w + lane / 16
  // for every k.  With 128-byte rows, load I covers rows 8 I + [0, 8): f = (lane / 8) ^ (I mod 8).
  const uint32_t vo_kn256 = (uint32_t)((lane >> 4) * p.kn_s.t * 2 + ((lane & 15) ^ (4 * w + (lane >> 4))) * 16);
  uint32_t vo_r128[2][2];  // [operand: K_nope (DN = 64), K_rope][k]
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int c = (lane & 7) ^ (((lane >> 3) ^ (w + 4 * k)) & 7);
    vo_r128[0][k] = (uint32_t)((lane >> 3) * p.kn_s.t * 2 + c * 16);
    vo_r128[1][k] = (uint32_t)((lane >> 3) * p.kr_s.t * 2 + c * 16);
  }
  const uint32_t vo_v = (uint32_t)((lane >> 4) * p.v_s.t * 2 + ((lane & 15) ^ swzv(lane >> 4)) * 16);
  // Issue the loads of the 64-key tile at kv0 into a stage.  Each load's descriptor ends
  // at the last valid key of its rows: lanes past Tk load nothing.
  auto load_tile = [&](int kv0, unsigned char* st) {
    constexpr int RPI_KN = 1024 / C::KN_RB;
#pragma unroll
    for (int k = 0; k < C::N_KN; ++k) {
      const int r0 = kv0 + RPI_KN * (w + 4 * k);
      dma16(make_rsrc(kn_b + (int64_t)r0 * p.kn_s.t, rows_bytes(min(p.Tk - r0, RPI_KN), p.kn_s.t, C::KN_RB)),
            DN == 128 ? vo_kn256 : vo_r128[0][k], (lds_void*)(st + 1024 * (w + 4 * k)));
    }
#pragma unroll
    for (int k = 0; k < C::N_KR; ++k) {
      const int r0 = kv0 + 8 * (w + 4 * k);
      dma16(make_rsrc(kr_b + (int64_t)r0 * p.kr_s.t, rows_bytes(min(p.Tk - r0, 8), p.kr_s.t, 128)), vo_r128[1][k],
            (lds_void*)(st + C::OFF_KR + 1024 * (w + 4 * k)));
    }
#pragma unroll
    for (int k = 0; k < C::N_V; ++k) {
      const int r0 = kv0 + 4 * (w + 4 * k);
      dma16(make_rsrc(v_b + (int64_t)r0 * p.v_s.t, rows_bytes(min(p.Tk - r0, 4), p.v_s.t, 256)), vo_v,
            (lds_void*)(st + C::OFF_V + 1024 * (w + 4 * k)));
    }
  };

  // LDS byte offsets (within a stage) of this lane's operands.
  // S^T A operand, k-step ks, key block jb: row 32 jb + l32, chunk 2 ks' + g of its region.
  // With power-of-two rows, row * RB + 16 (c ^ f) = (row * RB + 16 f) ^ 16 c.
  // (128-byte rows: rows l32 and 32 + l32 differ in f, so each key block has its own base)
  const int a_kn = DN == 128 ? (l32 * 256 + 16 * (g ^ swz256(l32))) : (l32 * 128 + 16 * (g ^ swz128(l32)));
  const int a_kn1 = DN == 128 ? a_kn + 32 * 256 : ((32 + l32) * 128 + 16 * (g ^ swz128(32 + l32)));
  const int a_kr0 = C::OFF_KR + l32 * 128 + 16 * (g ^ swz128(l32));
  const int a_kr1 = C::OFF_KR + (32 + l32) * 128 + 16 * (g ^ swz128(32 + l32));
  // V^T operand through ds_read_b64_tr_b16: lane r of a 16-lane group addresses key
  // (block start) + 4 g + r / 4, dv columns 32 mb + 16 ((lane >> 4) & 1) + 4 (r % 4).
  const int l16 = lane & 15;
  const int vt_row = 4 * g + (l16 >> 2);
  const int vt_base = C::OFF_V + vt_row * 256 + 16 * ((2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1)) ^ swzv(vt_row)) +
                      8 * (l16 & 1);

  __syncthreads();  // the zeros are in place before any load lands
  bool tile0_ready = false;  // tile 0 of the current q-tile is already in stage 0
  for (int item = 0; item < n_items; ++item) {
  const int qt = item == 0 ? qt_first : qt_second;
  const int q0 = qt * C::BM;
  const int qw0 = q0 + 32 * w;                       // first query row of this wave
  const int q_row = qw0 + l32;                        // this lane's query
  const int q_ld = q_row < p.Tq ? q_row : p.Tq - 1;  // clamped row for loads

  // ---- Q^T fragment (B operand of S^T = K Q^T): dims 16 ks + 8 g + [0, 8)
  bf16x8 qf[C::KS];
  {
    const bf16* qn = p.qn + (int64_t)b * p.qn_s.b + (int64_t)q_ld * p.qn_s.t + (int64_t)h * p.qn_s.h;
    const bf16* qr = p.qr + (int64_t)b * p.qr_s.b + (int64_t)q_ld * p.qr_s.t + (int64_t)h * p.qr_s.h;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const int d = 16 * ks + 8 * g;
      qf[ks] = as_bf16x8(d < DN ? ldg16(qn + d) : ldg16(qr + (d - DN)));
    }
  }

  // ---- key range of the workgroup and of this wave
  int kv_end = p.Tk;
  int wave_last = p.Tk - 1;  // last key any row of this wave can see
  if (p.causal) {
    const int64_t lim = (int64_t)q0 + C::BM + p.q_offset;  // exclusive bound for the tile's last row
    if (lim < kv_end) kv_end = lim < 0 ? 0 : (int)lim;
    const int64_t wl = (int64_t)qw0 + 31 + p.q_offset;
    if (wl < wave_last) wave_last = (int)wl;
  }
  const int n_tiles = (kv_end + C::BN - 1) / C::BN;
  // the next q-tile's first K/V tile is prefetched into stage 0 during the last tile when
  // that tile runs from stage 1 (an even tile count)
  const bool prefetch_next = item + 1 < n_items && (n_tiles & 1) == 0;

  f32x16 oacc[4];
  float m_run, l_run;  // log2-domain reference max of this lane's row; its share of the row sum

  // Tile loop.  Fast form (SAFE = false): the reference max is the first tile's row max
  // (key 0 is visible to every row) and never moves, so later tiles need no max, no
  // rescale and no branch on the scores.  p = 2^(s - m) stays finite unless a later score
  // exceeds the first tile's max by more than ~127 (log2); the workgroup then votes and
  // recomputes the q-tile with the safe form, which moves the reference max lazily (when it
  // grows by more than kFwdRescale) and rescales O and l.
  // Tiles [1, n_hot) are fully visible to every row of the workgroup: they skip the mask
  // and the max.  Tile j runs from stage j % 2.
  int n_full = p.Tk / C::BN;
  if (p.causal) n_full = min(n_full, (q0 + q_off + 1) / C::BN);
  const int n_hot = min(n_full, n_tiles - 1);

  auto run_tiles = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) oacc[mb] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;

    auto tile = [&](int j, auto stage_tag) {
      constexpr int ST = decltype(stage_tag)::value;
      unsigned char* cur = ST == 0 ? stage0 : stage1;
      unsigned char* nxt = ST == 0 ? stage1 : stage0;
      const int kv0 = j * C::BN;
      // masking and the max are needed only on the first tile and on the tiles past n_hot
      const bool gen = SAFE || j == 0 || j >= n_hot;
      // tile j has landed once every wave's own loads have (wait, then barrier); past the
      // barrier every wave is also done with tile j - 1, whose stage is reloaded next
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (j + 1 < n_tiles) {
        load_tile(kv0 + C::BN, nxt);
      } else if (ST == 1 && prefetch_next) {
        load_tile(0, stage0);  // the next q-tile of this (b, h) starts at key 0
      }
      if (kv0 > wave_last) return;  // every key of the tile is masked for this wave

      // the per-k-step addresses are recomputed in every tile (one XOR each) rather than
      // held in registers across the loop
      const int b_kn0 = opaque(a_kn), b_kr0 = opaque(a_kr0), b_kr1 = opaque(a_kr1), b_vt = opaque(vt_base);
      const int b_kn1 = DN == 128 ? b_kn0 + 32 * 256 : opaque(a_kn1);
      // S^T: 2 x KS MFMAs alternating between the two key blocks, the A fragments read
      // S_AHEAD MFMAs ahead of their use (the schedule is pinned by the group barriers)
      f32x16 sacc[2];
      sacc[0] = f32x16{};
      sacc[1] = f32x16{};
      {
        constexpr int NS = 2 * C::KS;  // step n: key block n % 2, k-step n / 2
        bf16x8 a[NS];
#pragma unroll
        for (int n = 0; n < NS; ++n) {
          const int ks = n >> 1, jb = n & 1;
          const int off = ks < C::KNS ? (jb ? b_kn1 : b_kn0) ^ (32 * ks) : (jb ? b_kr1 : b_kr0) ^ (32 * (ks - C::KNS));
          a[n] = as_bf16x8(lds16(cur + off));
        }
#pragma unroll
        for (int n = 0; n < NS; ++n) sacc[n & 1] = mfma32(a[n], qf[n >> 1], sacc[n & 1]);
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, S_AHEAD, 0);
#pragma unroll
        for (int n = 0; n < NS - S_AHEAD; ++n) {
          __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, S_AHEAD, 0);
      }

      if (gen) {
        // mask only the tiles that cross the causal diagonal or the end of the keys
        const bool need_mask = (p.causal && kv0 + C::BN - 1 > qw0 + q_off) || kv0 + C::BN > p.Tk;
        if (need_mask) {
          // key kv is visible to this lane's row iff kv < lim (lim <= Tk)
          const int lim = p.causal ? min(p.Tk, q_row + q_off + 1) : p.Tk;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kv = kv0 + 32 * jb + 8 * (r >> 2) + 4 * g + (r & 3);
              sacc[jb][r] = kv < lim ? sacc[jb][r] : -INFINITY;
            }
          }
        }
        if (SAFE || j == 0) {
          float mx0 = max3f(sacc[0][0], sacc[0][1], sacc[0][2]);
          float mx1 = max3f(sacc[1][0], sacc[1][1], sacc[1][2]);
#pragma unroll
          for (int r = 3; r < 15; r += 2) {
            mx0 = max3f(mx0, sacc[0][r], sacc[0][r + 1]);
            mx1 = max3f(mx1, sacc[1][r], sacc[1][r + 1]);
          }
          float mloc = max3f(mx0, sacc[0][15], fmaxf(mx1, sacc[1][15]));
          mloc = fmaxf(mloc, wave_shfl_xor(mloc, 32)) * p.scale_log2;  // scale > 0 commutes with max
          if (!SAFE) {
            m_run = mloc;
          } else if (__any(mloc > m_run + kFwdRescale)) {
            const float m_new = mloc > m_run + kFwdRescale ? mloc : m_run;
            const float alpha = fast_exp2(m_run - m_new);  // 1 for rows that keep m_run (incl. -inf)
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) oacc[mb] *= alpha;
          }
        }
      }
      const float neg_m = m_run == -INFINITY ? 0.f : -m_run;

      bf16x8 pb[2][2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          u32x4 pk;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = fast_exp2(__builtin_fmaf(sacc[jb][8 * s + 2 * e], p.scale_log2, neg_m));
            const float p1 = fast_exp2(__builtin_fmaf(sacc[jb][8 * s + 2 * e + 1], p.scale_log2, neg_m));
            l_run += p0 + p1;
            pk[e] = pack_bf16x2(p0, p1);
          }
          pb[jb][s] = as_bf16x8(pk);
        }
      }

      // O^T (128 x 32) += V^T (128 x 64) P^T (64 x 32); K slot (g, e) <-> key
      // 32 jb + 16 s + 8 (e / 4) + 4 g + e % 4, matching the S^T accumulator rows.
      // Rows 32 jb + 16 s (+ 8) keep row % 4, so only the dv block mb changes the swizzle.
      {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        bf16x8 vt[16];  // step n = 4 (2 jb + s) + mb
#pragma unroll
        for (int n = 0; n < 16; ++n) {
          const int mb = n & 3, kb = 16 * (n >> 2);  // kb = 32 jb + 16 s
          const int off = (b_vt ^ (64 * mb)) + kb * 256;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + off));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + off + 8 * 256));
          const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
          vt[n] = as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]});
        }
#pragma unroll
        for (int n = 0; n < 16; ++n) oacc[n & 3] = mfma32(vt[n], pb[n >> 3][(n >> 2) & 1], oacc[n & 3]);
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2 * PV_AHEAD, 0);
#pragma unroll
        for (int n = 0; n < 16 - PV_AHEAD; ++n) {
          __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, PV_AHEAD, 0);
      }
    };

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    for (int j = 0; j < n_tiles; j += 2) {
      tile(j, S0{});
      if (j + 1 < n_tiles) tile(j + 1, S1{});
    }
  };

  if (!tile0_ready) load_tile(0, stage0);
  run_tiles(std::false_type{});
  {
    // workgroup vote: did any row's sum leave the finite range of the fixed reference?
    // The vote slots sit in stage 1, idle between the last tile's reads (first barrier)
    // and the next q-tile's second tile.
    int* vote = reinterpret_cast<int*>(stage1);
    const float lt = l_run + wave_shfl_xor(l_run, 32);
    const bool any_bad = __any(!(lt <= kFwdSumLimit));  // a wave-wide vote: every lane takes part
    __syncthreads();
    if (lane == 0) vote[w] = any_bad ? 1 : 0;
    __syncthreads();
    const bool redo = (vote[0] | vote[1] | vote[2] | vote[3]) != 0;
    if (redo) {
      // a prefetch of the next q-tile may still be landing in stage 0: let it finish
      // before the same bytes are loaded again
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      load_tile(0, stage0);
      run_tiles(std::true_type{});
    }
  }
  tile0_ready = prefetch_next;

  // ---- epilogue: normalise and store O [q][d] and LSE
  const float l_tot = l_run + wave_shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (q_row < p.Tq) {
    bf16* op = p.o + (int64_t)b * p.o_s.b + (int64_t)q_row * p.o_s.t + (int64_t)h * p.o_s.h;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x2 v2{pack_bf16x2(oacc[mb][4 * i + 0] * inv, oacc[mb][4 * i + 1] * inv),
                 pack_bf16x2(oacc[mb][4 * i + 2] * inv, oacc[mb][4 * i + 3] * inv)};
        stg8(op + 32 * mb + 8 * i + 4 * g, v2);
      }
    }
    if (g == 0) {
      const float lse = l_tot > 0.f ? (m_run + fast_log2(l_tot)) * kLn2 : -INFINITY;
      p.lse[((int64_t)b * p.H + h) * p.Tq + q_row] = lse;
    }
  }
  }  // item
}

template <int DN>
static int launch_fwd(const FwdParams& prm, hipStream_t s) {
  const int64_t n = (int64_t)prm.B * prm.H * ((prm.n_qt + 1) / 2);
  MLA_CHECK(n < (1ll << 31), MLA_ERR_INVALID_ARG, "mla_prefill_fwd: grid too large");
  prefill_fwd_kernel<DN><<<dim3((unsigned)n), dim3(256), 0, s>>>(prm);
  return launch_status("mla_prefill_fwd");
}

}  // namespace mla

using namespace mla;

extern "C" int mla_prefill_fwd(const mla_prefill_fwd_args* a, void* stream) {
  const char* op = "mla_prefill_fwd";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->d_rope == 64 && a->d_v == 128 && (a->d_nope == 128 || a->d_nope == 64), MLA_ERR_UNSUPPORTED,
            "%s: head dims (nope %lld, rope %lld, v %lld) not built; supported nope in {64,128}, rope 64, v 128",
            op, (long long)a->d_nope, (long long)a->d_rope, (long long)a->d_v);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->Tq >= 0 && a->Tk >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->B < (1 << 20) && a->H < (1 << 16) && a->Tq < (1 << 30) && a->Tk < (1 << 30), MLA_ERR_INVALID_ARG,
            "%s: size out of range", op);
  if (a->B == 0 || a->H == 0 || a->Tq == 0) return MLA_OK;
  MLA_CHECK(a->Tk > 0, MLA_ERR_INVALID_ARG, "%s: Tk must be positive", op);
  MLA_CHECK(!a->causal || a->q_offset >= 0, MLA_ERR_INVALID_ARG, "%s: q_offset must be >= 0", op);
  MLA_CHECK(a->q_offset < (1 << 30), MLA_ERR_INVALID_ARG, "%s: q_offset out of range", op);
  MLA_CHECK(a->k_nope_stride.t < (1 << 24) && a->k_rope_stride.t < (1 << 24) && a->v_stride.t < (1 << 24),
            MLA_ERR_INVALID_ARG, "%s: key/value row strides must be below 2^24 elements", op);
  MLA_TRY(check_operand(op, "q_nope", a->q_nope, a->q_nope_stride));
  MLA_TRY(check_operand(op, "q_rope", a->q_rope, a->q_rope_stride));
  MLA_TRY(check_operand(op, "k_nope", a->k_nope, a->k_nope_stride));
  MLA_TRY(check_operand(op, "k_rope", a->k_rope, a->k_rope_stride));
  MLA_TRY(check_operand(op, "v", a->v, a->v_stride));
  MLA_TRY(check_operand(op, "o", a->o, a->o_stride));
  MLA_CHECK(a->lse, MLA_ERR_INVALID_ARG, "%s: lse is null", op);

  FwdParams prm;
  prm.qn = (const bf16*)a->q_nope;
  prm.qr = (const bf16*)a->q_rope;
  prm.kn = (const bf16*)a->k_nope;
  prm.kr = (const bf16*)a->k_rope;
  prm.v = (const bf16*)a->v;
  prm.o = (bf16*)a->o;
  prm.lse = a->lse;
  prm.B = (int)a->B;
  prm.H = (int)a->H;
  prm.Tq = (int)a->Tq;
  prm.Tk = (int)a->Tk;
  prm.n_qt = (int)((a->Tq + 127) / 128);
  prm.qn_s = a->q_nope_stride;
  prm.qr_s = a->q_rope_stride;
  prm.kn_s = a->k_nope_stride;
  prm.kr_s = a->k_rope_stride;
  prm.v_s = a->v_stride;
  prm.o_s = a->o_stride;
  prm.scale_log2 = a->scale * kLog2e;
  prm.causal = a->causal ? 1 : 0;
  prm.q_offset = a->q_offset;
  hipStream_t s = (hipStream_t)stream;
  return a->d_nope == 128 ? launch_fwd<128>(prm, s) : launch_fwd<64>(prm, s);
}
