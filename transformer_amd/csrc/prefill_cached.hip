// Absorbed latent attention for a chunk of T query tokens per sequence over a cache
// (gfx950): the prefill with a cache in the reference's absorbed form.
//   s[t][j] = (q_lat[t] . c_kv[j] + q_rope[t] . k_rope[j]) * scale,   j <= L0 + t
//   ctx[t]  = softmax_j(s[t]) c_kv,   lse[t] = logsumexp_j(s[t])
// q_lat = q_nope W_UK is absorbed by the caller (transformer.py:252-254) and W_UV applied
// after (:290-291); the mask is the bottom-right causal mask of :273-281 (query t of the
// chunk sits at position L0 + t and sees every key up to it).
//
// Up-projecting the whole cache into per-head K and V (what T > 1 otherwise costs) is
// 2 B L d_latent H (d_nope + d_v) FLOP per chunk; here the cache is read in its latent form
// and each (query, head) pays (d_latent + 64) + d_latent multiply-adds per key: for a 64-token
// chunk over 4000 cached tokens at 16 heads, 285 GFLOP of attention against 546 GFLOP of
// up-projections plus 85 of attention.
//
// Work decomposition.  A workgroup owns one sequence, one group of 16 heads and NW queries of
// the chunk, one per wave (NW = 8, or 4 when 8 would leave CUs idle); it walks the 32-token
// tiles of the keys its last query sees.  Each tile is loaded once for the NW waves by
// direct-to-LDS loads into one of three tile buffers (two tiles in flight while one is
// computed; one barrier per tile).  For its query and 16 heads each wave runs
//   * S^T [16 tok][16 heads] = C [16 tok][KW] . Q^T    (v_mfma_f32_16x16x32_bf16, two 16-token
//     halves), the shared k_rope being 64 more columns of the row (KW = d_latent + 64); Q^T
//     stays in registers;
//   * an online softmax per head (lane = head, registers = tokens), with the reference max
//     moved lazily;
//   * O^T [d_latent][16 heads] += C^T [d_latent][32 tok] . P^T    (v_mfma_f32_16x16x32_bf16),
//     C^T from two ds_read_b64_tr_b16 (one per half tile; K slot 8 G + e holds token 4 G + e of
//     the first half for e < 4 and 16 + 4 G + e - 4 of the second), P^T from the S^T
//     accumulators in the same order; a lane then owns 4 consecutive latent columns of its
//     head, so the ctx stores are vectors.
// LDS fragments are read two products ahead of the MFMA that takes them.  When the grid would
// not fill the chip (a few sequences), each workgroup takes one of S ranges of key tiles and
// writes fp32 partials (O relative to its reference max, the max, the sum), which
// prefill_cached_merge_kernel combines in range order; otherwise every (query, head) has one
// writer.  Both ways are deterministic.
//
// What bounds it: every wave reads the whole tile from LDS twice (36 KiB of score fragments,
// 32 KiB of transpose fragments per 32 tokens at d_latent 512) for 68 MFMAs, so 8 waves per
// CU need about as many LDS cycles (at 128 bytes per clock) as the MFMAs take on two waves per
// SIMD; more queries per wave would halve that but do not fit the 256 registers of two waves
// per SIMD (Q and O of one query take 200).
//
// LDS tile layout: the latent part of row t (LCH 16-byte chunks) at stride RSL chunks with
// RSL * 16 = 128 mod 256 bytes, chunk c at position c ^ sw(t); the k_rope part of the 32 rows
// in a separate region of 128-byte rows with the same swizzle.  A latent row is one
// direct-to-LDS load of LCH lanes (lane p fetches the chunk that belongs at position p); the
// k_rope rows of a wave are one load.
#include "mla_common.h"

namespace mla {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct PcParams {
  const bf16 *q_lat, *q_rope, *c_kv, *k_rope;
  bf16* ctx;
  float* lse;
  float* part_o;   // S > 1: [unit][split][NW][16 heads][DL] unnormalised O (relative to part_ml.x)
  float2* part_ml; // S > 1: [unit][split][NW][16 heads] (log2-domain reference max, sum)
  int B, T, H, L0, n_hg, n_qb, S, chunk_tiles, nw;
  mla_strides ql_s, qr_s, ctx_s;
  int64_t c_kv_sb, c_kv_st, k_rope_sb, k_rope_st;
  float scale_log2;
};

template <int DL, int NW_>
struct PcCfg {
  static constexpr int TT = 32;                              // tokens per tile
  static constexpr int NW = NW_;                             // waves (= queries) per workgroup
  static constexpr int NBUF = 3;                             // tile buffers (two tiles in flight)
  static constexpr int LCH = DL / 8;                         // latent chunks per row
  static constexpr int RSL = (LCH % 16 == 8) ? LCH : LCH + 8;  // latent row stride in chunks
  static constexpr int NKS = (DL + 64) / 32;                 // score k-steps
  static constexpr int NKL = DL / 32;                        // of which over the latent part
  static constexpr int NB = DL / 16;                         // P V column blocks
  static constexpr int HALF = 16 * RSL * 16;                 // bytes of 16 latent rows
  static constexpr int ROPE = 2 * HALF;                      // offset of the k_rope region
  static constexpr int TILE = ROPE + TT * 128;               // bytes per tile buffer
  static constexpr int PF = 2;                               // LDS fragments read ahead of their MFMA
  static constexpr int ROWS_W = TT / NW;                     // latent rows (and k_rope rows) per wave
  static constexpr int LOADS = ROWS_W + 1;                   // direct-to-LDS loads per wave per tile
  static_assert(LCH % 8 == 0 && LCH <= 64, "a latent row is one load of at most 64 lanes");
  static_assert(TT % NW == 0 && ROWS_W * 8 <= 64, "a wave's k_rope rows are one load");
  static_assert(NBUF == 3, "the waits below assume at most one later tile in flight");
  static_assert(NBUF * TILE <= 160 * 1024, "LDS");
};

// s_waitcnt vmcnt(N) with N an immediate
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// growth of a head's running max (log2 units) that triggers a rescale of O
constexpr float kPcRescale = 8.0f;

// swizzle of token t's chunk index: bits (3, 1, 2) of t as bits (0, 1, 2).  With rows 128 bytes
// past a multiple of 256 (64 banks of 4 bytes), the 16 rows of a score read land on 16 distinct
// 16-byte bank groups, and in a transpose read the pair index (bits 1, 2) differs between the 4
// rows of equal parity that 32 lanes touch, so those 32 lanes cover all 64 banks once.
__device__ __forceinline__ int pc_swz(int t) { return ((t >> 3) & 1) | (((t >> 1) & 1) << 1) | (((t >> 2) & 1) << 2); }

template <int DL, int NW>
__global__ __launch_bounds__(64 * NW, 1) void prefill_cached_kernel(PcParams p) {
  using C = PcCfg<DL, NW>;
  __shared__ __attribute__((aligned(1024))) unsigned char tiles[C::NBUF * C::TILE];

  // workgroup id -> (b, head group, key range, query block), id = ((b n_hg + hg) S + split)
  // n_qb + qb.  The query blocks of one key range are consecutive ids and consecutive ids share
  // an XCD (hardware places id on XCD id % 8), so the workgroups that read the same cache rows
  // meet in one L2.
  const int n_wg = gridDim.x;
  int id = blockIdx.x;
  if ((n_wg & 7) == 0) id = (id & 7) * (n_wg >> 3) + (id >> 3);
  const int qb = id % p.n_qb;
  const int us = id / p.n_qb;
  const int split = us % p.S;
  const int bh = us / p.S;
  const int hg = bh % p.n_hg;
  const int b = bh / p.n_hg;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, G = lane >> 4;
  const int h = hg * 16 + l16;  // this lane's head (S^T column, softmax, O^T column)
  const bool h_ok = h < p.H;
  const int t = qb * NW + w;    // this wave's query
  const int lim = t < p.T ? p.L0 + t + 1 : 0;  // keys [0, lim) are visible to it (0: no query)
  const int n_keys = p.L0 + min(qb * NW + NW, p.T);  // keys the workgroup's last query sees
  // this workgroup's key tiles [j_begin, j_end) (all of them when S = 1; possibly none)
  const int j_begin = split * p.chunk_tiles;
  const int j_end = min(j_begin + p.chunk_tiles, (n_keys + C::TT - 1) / C::TT);

  // Q^T fragments (B operand of S^T = C . Q^T): lane (l16, G), k-step ks holds dims
  // 32 ks + 8 G + [0, 8) of head l16: latent dims from q_lat, the last 64 from q_rope
  bf16x8 qf[C::NKS];
  {
    const bool ok = lim > 0 && h_ok;
    const int tq = ok ? t : 0, hq = ok ? h : 0;
    const bf16* ql = p.q_lat + (int64_t)b * p.ql_s.b + (int64_t)tq * p.ql_s.t + (int64_t)hq * p.ql_s.h;
    const bf16* qr = p.q_rope + (int64_t)b * p.qr_s.b + (int64_t)tq * p.qr_s.t + (int64_t)hq * p.qr_s.h;
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
      const int d = 32 * ks + 8 * G;
      const u32x4 v = ks < C::NKL ? ldg16(ql + d) : ldg16(qr + (d - DL));
      qf[ks] = as_bf16x8(ok ? v : u32x4{0u, 0u, 0u, 0u});
    }
  }

  // Direct-to-LDS tile loads.  Wave w fetches latent rows w, w + NW, ..., one load per row
  // (lanes p < LCH: position p of row r holds chunk p ^ sw(r)), and the k_rope of rows
  // ROWS_W w .. ROWS_W (w + 1) - 1 in one load (lane l: row ROWS_W w + l / 8, position l % 8).
  // Rows past the workgroup's last key repeat that key: finite data, masked to p = 0.  The
  // descriptors start at the tile's first row, so the offsets stay small for any cache length.
  const bf16* ckv_b = p.c_kv + (int64_t)b * p.c_kv_sb;
  const bf16* kr_b = p.k_rope + (int64_t)b * p.k_rope_sb;
  const uint32_t lds0 = lds_addr(tiles);
  // row strides in bytes (below 2^24: the host bounds them), 24-bit multiplies for the offsets
  const uint32_t c_st = (uint32_t)p.c_kv_st * 2u, r_st = (uint32_t)p.k_rope_st * 2u;
  auto issue_tile = [&](int j, int slot) {
    const int t0 = j * C::TT;
    const int nv = min(C::TT, n_keys - t0);  // rows of the tile inside the visible keys (>= 1)
    const buf_rsrc rc = make_rsrc(ckv_b + (int64_t)t0 * p.c_kv_st, rows_bytes(nv, p.c_kv_st, DL * 2));
    const buf_rsrc rr = make_rsrc(kr_b + (int64_t)t0 * p.k_rope_st, rows_bytes(nv, p.k_rope_st, 128));
    const uint32_t base = lds0 + (uint32_t)(slot * C::TILE);
#pragma unroll
    for (int n = 0; n < C::ROWS_W; ++n) {
      const int r = w + NW * n;
      const int rc_row = min(r, nv - 1);
      if (lane < C::LCH) {
        const uint32_t voff = __umul24((uint32_t)rc_row, c_st) + (uint32_t)((lane ^ pc_swz(r)) << 4);
        dma16(rc, voff, base + (uint32_t)(r * C::RSL * 16));
      }
    }
    if (lane < 8 * C::ROWS_W) {
      const int r = C::ROWS_W * w + (lane >> 3);
      const int rr_row = min(r, nv - 1);
      const uint32_t voff = __umul24((uint32_t)rr_row, r_st) + (uint32_t)(((lane & 7) ^ pc_swz(r)) << 4);
      dma16(rr, voff, base + (uint32_t)(C::ROPE + C::ROWS_W * w * 128));
    }
  };

  // LDS read offsets (within a tile buffer).  Scores (A operand): row l16 (+ 16 for the
  // second half), chunk 4 ks + G.
  const int swA = pc_swz(l16);
  const int offA0 = l16 * C::RSL * 16 + ((0 + G) ^ swA) * 16;
  const int offA1 = l16 * C::RSL * 16 + ((4 + G) ^ swA) * 16;
  const int offR0 = C::ROPE + l16 * 128 + ((0 + G) ^ swA) * 16;
  const int offR1 = C::ROPE + l16 * 128 + ((4 + G) ^ swA) * 16;
  // P V (transpose read): lane r of group G reads row 4 G + r / 4, columns 16 nb + 4 (r % 4)
  // + [0, 4), so lane (i, G) receives C[4 G + j][16 nb + i], j = 0..3 (and from row + 16 the
  // second half's tokens)
  const int rowB = 4 * G + (l16 >> 2);
  const int swB = pc_swz(rowB);
  const int qB = (l16 & 3) >> 1, halfB = l16 & 1;
  int offB[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) offB[j] = rowB * C::RSL * 16 + (((2 * j) ^ (swB & 6)) + ((qB ^ swB) & 1)) * 16 + halfB * 8;
  // byte offsets (first half) of the score fragment of k-step ks and of the P V fragment of
  // column block nb; a_half: distance to the second half's fragment
  auto a_off = [&](int ks) {
    return ks < C::NKL ? ((ks & 1) ? offA1 : offA0) + (ks >> 1) * 128 : (((ks - C::NKL) & 1) ? offR1 : offR0);
  };
  auto a_half = [&](int ks) { return ks < C::NKL ? C::HALF : 16 * 128; };
  auto b_off = [&](int nb) { return offB[nb & 3] + (nb >> 2) * 128; };

  f32x4 oacc[C::NB];
#pragma unroll
  for (int nb = 0; nb < C::NB; ++nb) oacc[nb] = f32x4{};
  float m_run = -INFINITY;  // log2-domain running max of head h (the same in the 4 lane groups)
  float l_part = 0.f;       // this lane's share of the running sum

  // prologue: tiles j_begin .. j_begin + NBUF - 2 in flight, wait for the first
#pragma unroll
  for (int k = 0; k < C::NBUF - 1; ++k)
    if (j_begin + k < j_end) issue_tile(j_begin + k, k);
  if (j_begin + 1 < j_end) wait_vmem_n<C::LOADS>();
  else wait_vmem_n<0>();
  __syncthreads();

  int slot = 0;  // buffer of tile j
  for (int j = j_begin; j < j_end; ++j) {
    // tile j + NBUF - 1 goes to the buffer tile j - 1 used (its readers passed the barrier)
    if (j + C::NBUF - 1 < j_end) {
      int s_new = slot + C::NBUF - 1;
      s_new -= s_new >= C::NBUF ? C::NBUF : 0;
      issue_tile(j + C::NBUF - 1, s_new);
    }
    const unsigned char* cur = tiles + slot * C::TILE;
    const int t0 = j * C::TT;
    if (t0 < lim) {  // wave-uniform: a tile wholly past the query's keys adds nothing
      // S^T of both halves: sacc[hh][r] = S[token 16 hh + 4 G + r][head l16]
      f32x4 sacc[2] = {f32x4{}, f32x4{}};
      bf16x8 fa[C::PF][2];
#pragma unroll
      for (int k = 0; k < C::PF; ++k) {
        fa[k][0] = as_bf16x8(lds16(cur + a_off(k)));
        fa[k][1] = as_bf16x8(lds16(cur + a_off(k) + a_half(k)));
      }
#pragma unroll
      for (int ks = 0; ks < C::NKS; ++ks) {
        const int f = ks % C::PF;
        sacc[0] = mfma16(fa[f][0], qf[ks], sacc[0]);
        sacc[1] = mfma16(fa[f][1], qf[ks], sacc[1]);
        if (ks + C::PF < C::NKS) {
          fa[f][0] = as_bf16x8(lds16(cur + a_off(ks + C::PF)));
          fa[f][1] = as_bf16x8(lds16(cur + a_off(ks + C::PF) + a_half(ks + C::PF)));
        }
      }
      // online softmax of each head over the tile's 32 tokens
      float x[8];
      float mloc = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = t0 + 16 * (e >> 2) + 4 * G + (e & 3);
        x[e] = key < lim ? sacc[e >> 2][e & 3] * p.scale_log2 : -INFINITY;
        mloc = fmaxf(mloc, x[e]);
      }
      mloc = xor16_max(mloc);
      mloc = xor32_max(mloc);
      // lazy rescaling: the reference max moves only when a head's tile max exceeds it by more
      // than kPcRescale (log2 units), so p <= 2^kPcRescale and O, l and the LSE share m_run
      if (__any(mloc > m_run + kPcRescale)) {
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
        m_run = m_new;
        l_part *= alpha;
#pragma unroll
        for (int nb = 0; nb < C::NB; ++nb) oacc[nb] *= alpha;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      float pr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pr[e] = fast_exp2(x[e] - m_use);
        l_part += pr[e];
      }
      // P^T as the B operand: column = head l16, K slot 8 G + e = token 16 (e / 4) + 4 G + e % 4
      const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                                                         pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7])});
      // C^T fragments of column block nb (both halves), read PF blocks ahead of their products
      s16x4 fb[C::PF][2];
#pragma unroll
      for (int k = 0; k < C::PF; ++k) {
        fb[k][0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + b_off(k)));
        fb[k][1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + b_off(k) + C::HALF));
      }
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) {
        const int f = nb % C::PF;
        const s16x8 v = __builtin_shufflevector(fb[f][0], fb[f][1], 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[nb] = mfma16(__builtin_bit_cast(bf16x8, v), pb, oacc[nb]);
        if (nb + C::PF < C::NB) {
          fb[f][0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + b_off(nb + C::PF)));
          fb[f][1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + b_off(nb + C::PF) + C::HALF));
        }
      }
    }
    // tile j + 1 must have landed; those of tile j + 2 may still be in flight
    if (j + 2 < j_end) wait_vmem_n<C::LOADS>();
    else wait_vmem_n<0>();
    __syncthreads();
    slot = slot + 1 == C::NBUF ? 0 : slot + 1;
  }

  // ---- ctx and LSE of this wave's query: lane (l16, G) holds columns 16 nb + 4 G + [0, 4)
  float lsum = l_part;
  lsum = xor16_sum(lsum);
  lsum = xor32_sum(lsum);
  if (p.S > 1) {  // this key range's partials, merged by prefill_cached_merge_kernel
    if (lim > 0 && h_ok) {
      const int64_t rec = ((int64_t)(bh * p.S + split) * p.n_qb + qb) * NW + w;  // this wave's record
      float* po = p.part_o + (rec * 16 + l16) * DL;
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) stg16(po + 16 * nb + 4 * G, __builtin_bit_cast(u32x4, oacc[nb]));
      if (G == 0) p.part_ml[rec * 16 + l16] = float2{m_run, lsum};
    }
    return;
  }
  if (lim > 0 && h_ok) {
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    bf16* cp = p.ctx + (int64_t)b * p.ctx_s.b + (int64_t)t * p.ctx_s.t + (int64_t)h * p.ctx_s.h;
#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb) {
      const f32x4 o = oacc[nb] * inv;
      stg8(cp + 16 * nb + 4 * G, u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])});
    }
    if (p.lse && G == 0)
      p.lse[((int64_t)b * p.H + h) * p.T + t] = lsum > 0.f ? (m_run + fast_log2(lsum)) * kLn2 : -INFINITY;
  }
}

// Merge of the S key ranges of one (b, t, h) per wave, in range order: M = max_s m_s,
// ctx = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, lse = (M + log2 L) ln 2.  Lane l owns
// latent columns 8 l .. 8 l + 7.
template <int DL>
__global__ __launch_bounds__(256) void prefill_cached_merge_kernel(PcParams p) {
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wid >= (int64_t)p.B * p.T * p.H) return;  // wave-uniform; no barrier follows
  const int h = (int)(wid % p.H);
  const int64_t bt = wid / p.H;
  const int t = (int)(bt % p.T), b = (int)(bt / p.T);
  const int l16 = h & 15, qb = t / p.nw, w = t - qb * p.nw;
  const int64_t bh = (int64_t)b * p.n_hg + (h >> 4);
  auto rec = [&](int s) { return (((bh * p.S + s) * p.n_qb + qb) * p.nw + w) * 16 + l16; };
  // Both passes take the ranges 8 at a time with every load of the 8 issued first (clamped
  // indices, results past S unused), one memory round trip per 8 ranges instead of per range;
  // the sums are added in range order.
  float M = -INFINITY;
  for (int s0 = 0; s0 < p.S; s0 += 8) {
    float mx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) mx[j] = p.part_ml[rec(min(s0 + j, p.S - 1))].x;
#pragma unroll
    for (int j = 0; j < 8; ++j) M = fmaxf(M, mx[j]);  // a repeated last range leaves the max as it is
  }
  const bool col_ok = 8 * lane < DL;
  float L = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < p.S; s0 += 8) {
    float2 ml[8];
    f32x4 v0[8], v1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t r = rec(min(s0 + j, p.S - 1));
      ml[j] = p.part_ml[r];
      if (col_ok) {
        const float* po = p.part_o + r * DL + 8 * lane;
        v0[j] = __builtin_bit_cast(f32x4, ldg16(po));
        v1[j] = __builtin_bit_cast(f32x4, ldg16(po + 4));
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // past S, or no visible key in the range (the same for the wave): nothing to add
      if (s0 + j >= p.S || ml[j].x == -INFINITY) continue;
      const float f = fast_exp2(ml[j].x - M);
      L += ml[j].y * f;
      if (col_ok) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] += f * v0[j][e];
          acc[4 + e] += f * v1[j][e];
        }
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (col_ok) {
    bf16* cp = p.ctx + (int64_t)b * p.ctx_s.b + (int64_t)t * p.ctx_s.t + (int64_t)h * p.ctx_s.h + 8 * lane;
    stg8(cp, u32x2{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)});
    stg8(cp + 4, u32x2{pack_bf16x2(acc[4] * inv, acc[5] * inv), pack_bf16x2(acc[6] * inv, acc[7] * inv)});
  }
  if (p.lse && lane == 0) p.lse[((int64_t)b * p.H + h) * p.T + t] = L > 0.f ? (M + fast_log2(L)) * kLn2 : -INFINITY;
}

// The merge for more than 8 ranges (a few sequences over a long cache, up to 256 ranges): one
// workgroup per (b, t, h), wave v taking the chunks of 8 ranges v, v + 4, ... (at B = 1 the
// one-wave merge left 64 of the 256 CUs busy, 32 round trips per pass).  The waves' maxima
// meet through LDS (the max is exact in any order); each wave then sums its own ranges in
// range order against that max, and wave 0 adds the four sums in wave order (deterministic).
template <int DL>
__global__ __launch_bounds__(256) void prefill_cached_merge_wide_kernel(PcParams p) {
  __shared__ float vm[4], vl[4];
  __shared__ f32x4 va[4][2][64];
  const int64_t item = blockIdx.x;  // (b, t, h)
  const int lane = threadIdx.x & 63;
  const int v = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = (int)(item % p.H);
  const int64_t bt = item / p.H;
  const int t = (int)(bt % p.T), b = (int)(bt / p.T);
  const int l16 = h & 15, qb = t / p.nw, w = t - qb * p.nw;
  const int64_t bh = (int64_t)b * p.n_hg + (h >> 4);
  auto rec = [&](int s) { return (((bh * p.S + s) * p.n_qb + qb) * p.nw + w) * 16 + l16; };
  float M = -INFINITY;
  for (int s0 = 8 * v; s0 < p.S; s0 += 32) {
    float mx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) mx[j] = p.part_ml[rec(min(s0 + j, p.S - 1))].x;
#pragma unroll
    for (int j = 0; j < 8; ++j) M = fmaxf(M, mx[j]);
  }
  if (lane == 0) vm[v] = M;
  __syncthreads();
  M = fmaxf(fmaxf(vm[0], vm[1]), fmaxf(vm[2], vm[3]));
  const bool col_ok = 8 * lane < DL;
  float L = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 8 * v; s0 < p.S; s0 += 32) {
    float2 ml[8];
    f32x4 v0[8], v1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t r = rec(min(s0 + j, p.S - 1));
      ml[j] = p.part_ml[r];
      if (col_ok) {
        const float* po = p.part_o + r * DL + 8 * lane;
        v0[j] = __builtin_bit_cast(f32x4, ldg16(po));
        v1[j] = __builtin_bit_cast(f32x4, ldg16(po + 4));
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j >= p.S || ml[j].x == -INFINITY) continue;
      const float f = fast_exp2(ml[j].x - M);
      L += ml[j].y * f;
      if (col_ok) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] += f * v0[j][e];
          acc[4 + e] += f * v1[j][e];
        }
      }
    }
  }
  if (lane == 0) vl[v] = L;
  va[v][0][lane] = f32x4{acc[0], acc[1], acc[2], acc[3]};
  va[v][1][lane] = f32x4{acc[4], acc[5], acc[6], acc[7]};
  __syncthreads();
  if (v != 0) return;
  L = ((vl[0] + vl[1]) + vl[2]) + vl[3];
  const f32x4 a0 = ((va[0][0][lane] + va[1][0][lane]) + va[2][0][lane]) + va[3][0][lane];
  const f32x4 a1 = ((va[0][1][lane] + va[1][1][lane]) + va[2][1][lane]) + va[3][1][lane];
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (col_ok) {
    bf16* cp = p.ctx + (int64_t)b * p.ctx_s.b + (int64_t)t * p.ctx_s.t + (int64_t)h * p.ctx_s.h + 8 * lane;
    stg8(cp, u32x2{pack_bf16x2(a0[0] * inv, a0[1] * inv), pack_bf16x2(a0[2] * inv, a0[3] * inv)});
    stg8(cp + 4, u32x2{pack_bf16x2(a1[0] * inv, a1[1] * inv), pack_bf16x2(a1[2] * inv, a1[3] * inv)});
  }
  if (p.lse && lane == 0) p.lse[((int64_t)b * p.H + h) * p.T + t] = L > 0.f ? (M + fast_log2(L)) * kLn2 : -INFINITY;
}

// workgroups of 8 waves (8 queries) share each tile among more queries; when they would not
// fill the chip's 256 CUs, workgroups of 4 waves give twice as many, and if those still do not,
// the keys are split into ranges of at least kPcMinSplitTiles tiles until they do
constexpr int kPcBigNW = 8, kPcSmallNW = 4, kPcFillWgs = 256, kPcMinSplitTiles = 4, kPcMaxSplits = 256;

struct PcLayout {
  int nw = 0, n_hg = 0, n_qb = 0, S = 1, chunk_tiles = 0;
  int64_t n_wg = 0;  // workgroups per key range
  size_t o_bytes = 0, total = 0;
};

static PcLayout pc_layout(const mla_prefill_cached_args* a) {
  PcLayout d;
  d.n_hg = (int)((a->H + 15) / 16);
  const int64_t n_wg_big = a->B * (int64_t)d.n_hg * ((a->T + kPcBigNW - 1) / kPcBigNW);
  d.nw = n_wg_big < kPcFillWgs ? kPcSmallNW : kPcBigNW;
  d.n_qb = (int)((a->T + d.nw - 1) / d.nw);
  d.n_wg = a->B * (int64_t)d.n_hg * d.n_qb;
  const int64_t n_tiles = (a->L0 + a->T + 31) / 32;  // tiles of the workgroup that sees the most keys
  int64_t S = a->num_splits;
  if (S <= 0)
    S = d.n_wg >= kPcFillWgs ? 1
                             : std::min<int64_t>((kPcFillWgs + d.n_wg - 1) / d.n_wg,
                                                 std::max<int64_t>(1, n_tiles / kPcMinSplitTiles));
  S = std::max<int64_t>(1, std::min<int64_t>({S, n_tiles, (int64_t)kPcMaxSplits}));
  const int64_t chunk = (n_tiles + S - 1) / S;
  d.S = (int)((n_tiles + chunk - 1) / chunk);  // no empty trailing range
  d.chunk_tiles = (int)chunk;
  if (d.S > 1) {
    const size_t recs = (size_t)d.n_wg * d.S * d.nw * 16;
    d.o_bytes = (recs * (size_t)a->d_latent * sizeof(float) + 255) / 256 * 256;
    d.total = d.o_bytes + recs * sizeof(float2);
  }
  return d;
}

template <int NW>
void launch_prefill_cached(const PcParams& prm, int d_latent, dim3 grid, hipStream_t s) {
  const dim3 block(64 * NW);
  switch (d_latent) {
    case 128: prefill_cached_kernel<128, NW><<<grid, block, 0, s>>>(prm); break;
    case 256: prefill_cached_kernel<256, NW><<<grid, block, 0, s>>>(prm); break;
    case 384: prefill_cached_kernel<384, NW><<<grid, block, 0, s>>>(prm); break;
    default: prefill_cached_kernel<512, NW><<<grid, block, 0, s>>>(prm); break;
  }
}

}  // namespace mla

using namespace mla;

// The sizes mla_prefill_cached accepts (without its pointer and stride checks), tested before the
// layout's arithmetic: the workspace query answers 0 for anything else.
static bool pc_sizes_ok(const mla_prefill_cached_args* a) {
  if (a->d_rope != 64 || (a->d_latent != 128 && a->d_latent != 256 && a->d_latent != 384 && a->d_latent != 512))
    return false;
  if (a->B <= 0 || a->T <= 0 || a->H <= 0 || a->L0 < 0 || a->num_splits < 0 || a->B >= 65536 || a->H >= 65536 ||
      a->T >= (1 << 20) || a->L0 >= (1ll << 30) || a->L >= (1ll << 31) || a->L < a->L0 + a->T)
    return false;
  const PcLayout d = pc_layout(a);
  return d.n_wg * d.S < (1ll << 31) && a->B * a->T * a->H < (d.S > 8 ? (1ll << 31) : (1ll << 33));
}

extern "C" size_t mla_prefill_cached_workspace_bytes(const mla_prefill_cached_args* a) {
  if (!a || !pc_sizes_ok(a)) return 0;
  return pc_layout(a).total;
}

extern "C" int mla_prefill_cached(const mla_prefill_cached_args* a, void* stream) {
  const char* op = "mla_prefill_cached";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_TRY(check_scale(op, a->scale));
  MLA_CHECK(a->d_rope == 64, MLA_ERR_UNSUPPORTED, "%s: d_rope must be 64", op);
  MLA_CHECK(a->d_latent == 128 || a->d_latent == 256 || a->d_latent == 384 || a->d_latent == 512,
            MLA_ERR_UNSUPPORTED, "%s: d_latent %lld not built (128, 256, 384, 512)", op, (long long)a->d_latent);
  MLA_CHECK(a->B >= 0 && a->T >= 0 && a->H >= 0 && a->L0 >= 0 && a->num_splits >= 0, MLA_ERR_INVALID_ARG,
            "%s: negative size or split count", op);
  MLA_CHECK(a->B < 65536 && a->H < 65536 && a->T < (1 << 20) && a->L0 < (1ll << 30) && a->L < (1ll << 31),
            MLA_ERR_INVALID_ARG, "%s: size out of range", op);
  if (a->B == 0 || a->T == 0 || a->H == 0) return MLA_OK;
  MLA_CHECK(a->L >= a->L0 + a->T, MLA_ERR_INVALID_ARG,
            "%s: the cache (L = %lld) must hold the L0 + T = %lld positions the chunk sees", op, (long long)a->L,
            (long long)(a->L0 + a->T));
  MLA_CHECK(a->q_lat && a->q_rope && a->c_kv && a->k_rope && a->ctx, MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  const void* ptrs[] = {a->q_lat, a->q_rope, a->c_kv, a->k_rope};
  for (const void* q : ptrs)
    MLA_CHECK(((uintptr_t)q & 15) == 0, MLA_ERR_INVALID_ARG, "%s: inputs must be 16-byte aligned", op);
  const int64_t st[] = {a->q_lat_stride.b, a->q_lat_stride.t, a->q_lat_stride.h, a->q_rope_stride.b,
                        a->q_rope_stride.t, a->q_rope_stride.h, a->c_kv_sb, a->c_kv_st, a->k_rope_sb, a->k_rope_st};
  for (int64_t s : st)
    MLA_CHECK(s >= 0 && (s & 7) == 0, MLA_ERR_INVALID_ARG, "%s: strides must be non-negative multiples of 8", op);
  // a tile's descriptors start at its first row and span 32 rows; the kernel forms the offsets
  // with 24-bit multiplies of the byte strides
  MLA_CHECK(a->c_kv_st < (1 << 23) && a->k_rope_st < (1 << 23), MLA_ERR_INVALID_ARG, "%s: row stride too large", op);
  MLA_CHECK(((uintptr_t)a->ctx & 7) == 0 && a->ctx_stride.b >= 0 && a->ctx_stride.t >= 0 && a->ctx_stride.h >= 0 &&
                (a->ctx_stride.b & 3) == 0 && (a->ctx_stride.t & 3) == 0 && (a->ctx_stride.h & 3) == 0,
            MLA_ERR_INVALID_ARG, "%s: ctx must be 8-byte aligned with strides multiples of 4", op);
  const PcLayout d = pc_layout(a);
  MLA_CHECK(d.n_wg * d.S < (1ll << 31) && a->B * a->T * a->H < (d.S > 8 ? (1ll << 31) : (1ll << 33)),
            MLA_ERR_INVALID_ARG, "%s: grid too large",
            op);
  if (d.S > 1) {
    MLA_CHECK(a->workspace && a->workspace_bytes >= d.total, MLA_ERR_WORKSPACE,
              "%s: workspace of %zu bytes required (got %zu)", op, d.total, a->workspace_bytes);
    MLA_CHECK(((uintptr_t)a->workspace & 255) == 0, MLA_ERR_WORKSPACE, "%s: workspace must be 256-byte aligned", op);
  }
  PcParams prm;
  prm.q_lat = (const bf16*)a->q_lat;
  prm.q_rope = (const bf16*)a->q_rope;
  prm.c_kv = (const bf16*)a->c_kv;
  prm.k_rope = (const bf16*)a->k_rope;
  prm.ctx = (bf16*)a->ctx;
  prm.lse = a->lse;
  prm.part_o = d.S > 1 ? (float*)a->workspace : nullptr;
  prm.part_ml = d.S > 1 ? (float2*)((char*)a->workspace + d.o_bytes) : nullptr;
  prm.B = (int)a->B;
  prm.T = (int)a->T;
  prm.H = (int)a->H;
  prm.L0 = (int)a->L0;
  prm.n_hg = d.n_hg;
  prm.n_qb = d.n_qb;
  prm.S = d.S;
  prm.chunk_tiles = d.chunk_tiles;
  prm.nw = d.nw;
  prm.ql_s = a->q_lat_stride;
  prm.qr_s = a->q_rope_stride;
  prm.ctx_s = a->ctx_stride;
  prm.c_kv_sb = a->c_kv_sb;
  prm.c_kv_st = a->c_kv_st;
  prm.k_rope_sb = a->k_rope_sb;
  prm.k_rope_st = a->k_rope_st;
  prm.scale_log2 = a->scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(d.n_wg * d.S));
  if (d.nw == kPcBigNW) launch_prefill_cached<kPcBigNW>(prm, (int)a->d_latent, grid, s);
  else launch_prefill_cached<kPcSmallNW>(prm, (int)a->d_latent, grid, s);
  if (d.S > 8) {  // the wide merge: one workgroup per (b, t, h)
    MLA_TRY(launch_status(op));
    const dim3 mgrid((unsigned)(a->B * a->T * a->H));
    switch (a->d_latent) {
      case 128: prefill_cached_merge_wide_kernel<128><<<mgrid, 256, 0, s>>>(prm); break;
      case 256: prefill_cached_merge_wide_kernel<256><<<mgrid, 256, 0, s>>>(prm); break;
      case 384: prefill_cached_merge_wide_kernel<384><<<mgrid, 256, 0, s>>>(prm); break;
      default: prefill_cached_merge_wide_kernel<512><<<mgrid, 256, 0, s>>>(prm); break;
    }
  } else if (d.S > 1) {
    MLA_TRY(launch_status(op));
    const dim3 mgrid((unsigned)((a->B * a->T * a->H + 3) / 4));
    switch (a->d_latent) {
      case 128: prefill_cached_merge_kernel<128><<<mgrid, 256, 0, s>>>(prm); break;
      case 256: prefill_cached_merge_kernel<256><<<mgrid, 256, 0, s>>>(prm); break;
      case 384: prefill_cached_merge_kernel<384><<<mgrid, 256, 0, s>>>(prm); break;
      default: prefill_cached_merge_kernel<512><<<mgrid, 256, 0, s>>>(prm); break;
    }
  }
  return launch_status(op);
}
