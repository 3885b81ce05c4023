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
// and each (query, head) pays (d_latent + 64) + d_latent per key: for a 64-token chunk over
// 4000 cached tokens at 16 heads, 285 GFLOP of attention against 546 GFLOP of up-projections
// plus 85 of attention.
//
// Work decomposition.  A workgroup owns one sequence, one group of 16 heads and 4 queries
// of the chunk, one per wave; it walks the 16-token tiles of the keys its last query sees.
// Every tile is loaded once for the 4 waves (each thread stages a few 16-byte chunks through
// registers into one of two LDS tile buffers, one barrier per tile), and each wave runs, for
// its own query and 16 heads:
//   * S^T [16 tok][16 heads] = C [16 tok][KW] . Q^T    v_mfma_f32_16x16x32_bf16, the shared
//     k_rope being 64 more columns of the row (KW = d_latent + 64); Q^T stays in registers;
//   * an online softmax per head (lane = head, registers = tokens), with the reference max
//     moved lazily;
//   * O^T [d_latent][16 heads] += C^T [d_latent][16 tok] . P^T    v_mfma_f32_16x16x16_bf16,
//     C^T from ds_read_b64_tr_b16, P^T from the S^T accumulators; a lane then owns 4
//     consecutive latent columns of its head, so the ctx stores are vectors.
// No split over the keys: every (query, head) has one writer (deterministic).
//
// LDS tile layout (as the decode's): row t holds KW bf16 as 16-byte chunks, chunk c at
// position c ^ sw(t) (sw(t) a permutation of bits 1..3 of t), row stride RS chunks with
// RS * 16 = 128 mod 256 bytes, so the score reads (16 tokens x one chunk) and the
// transpose reads (4 tokens x 2 chunks per 16 lanes) are free of bank conflicts.
#include "mla_common.h"

namespace mla {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct PcParams {
  const bf16 *q_lat, *q_rope, *c_kv, *k_rope;
  bf16* ctx;
  float* lse;
  int B, T, H, L0, n_hg, n_qb;
  mla_strides ql_s, qr_s, ctx_s;
  int64_t c_kv_sb, c_kv_st, k_rope_sb, k_rope_st;
  float scale_log2;
};

template <int DL>
struct PcCfg {
  static constexpr int TT = 16;                          // tokens per tile
  static constexpr int NQ = 4;                           // queries (waves) per workgroup
  static constexpr int KW = DL + 64;                     // columns of a staged row
  static constexpr int NCH = KW / 8;                     // 16-byte chunks per row
  static constexpr int RS = (NCH % 16 == 8) ? NCH : NCH + 8;  // row stride in chunks
  static constexpr int NKS = KW / 32;                    // score k-steps
  static constexpr int NB = DL / 16;                     // P V column blocks
  static constexpr int LCH = DL / 8;                     // latent chunks per row
  static constexpr int PRE_L = TT * LCH / 256;           // latent chunks per thread per tile
  static constexpr int TILE = TT * RS * 16;              // bytes per tile buffer
  static_assert((TT * LCH) % 256 == 0, "the latent part of a tile splits evenly over 256 threads");
  static_assert(NCH % 8 == 0, "the swizzle works on groups of 8 chunks");
};

// growth of a head's running max (log2 units) that triggers a rescale of O
constexpr float kPcRescale = 8.0f;

// swizzle of token t's chunk index: a permutation of bits (1, 2, 3) of t
__device__ __forceinline__ int pc_swz(int t) { return ((t >> 2) & 1) | (((t >> 3) & 1) << 1) | (((t >> 1) & 1) << 2); }

template <int DL>
__global__ __launch_bounds__(256, 2) void prefill_cached_kernel(PcParams p) {
  using C = PcCfg<DL>;
  __shared__ __attribute__((aligned(16))) unsigned char tiles[2 * C::TILE];

  // workgroup id -> (b, head group, query block); the query blocks of one sequence are
  // consecutive, so they run together and share its cache rows in L2
  const int id = blockIdx.x;
  const int qb = id % p.n_qb;
  const int bh = id / p.n_qb;
  const int hg = bh % p.n_hg;
  const int b = bh / p.n_hg;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, G = lane >> 4;
  const int t = qb * C::NQ + w;               // this wave's query of the chunk
  const bool active = t < p.T;                 // wave-uniform
  const int h = hg * 16 + l16;                 // this lane's head (S^T column, softmax, O^T column)
  const bool h_ok = h < p.H;
  const int lim = p.L0 + t + 1;                // keys [0, lim) are visible to the query
  const int n_keys = p.L0 + min(qb * C::NQ + C::NQ, p.T);  // keys the workgroup's last query sees
  const int n_tiles = (n_keys + C::TT - 1) / C::TT;

  // Q^T fragments (B operand of S^T = C . Q^T): lane (l16, G), k-step ks holds dims
  // 32 ks + 8 G + [0, 8) of head l16: latent dims from q_lat, the last 64 from q_rope
  bf16x8 qf[C::NKS];
  {
    const bool ok = active && h_ok;
    const int tq = active ? t : 0, hq = h_ok ? h : 0;
    const bf16* ql = p.q_lat + (int64_t)b * p.ql_s.b + (int64_t)tq * p.ql_s.t + (int64_t)hq * p.ql_s.h;
    const bf16* qr = p.q_rope + (int64_t)b * p.qr_s.b + (int64_t)tq * p.qr_s.t + (int64_t)hq * p.qr_s.h;
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
      const int d = 32 * ks + 8 * G;
      const u32x4 v = d < DL ? ldg16(ql + d) : ldg16(qr + (d - DL));
      qf[ks] = as_bf16x8(ok ? v : u32x4{0u, 0u, 0u, 0u});
    }
  }

  // tile staging through registers: thread tid holds latent chunks q = tid + 256 i of the
  // tile (row q / LCH) and, for tid < 128, k_rope chunk tid (row tid / 8); rows past the
  // workgroup's last key repeat that key (finite data, masked to p = 0)
  const bf16* ckv_b = p.c_kv + (int64_t)b * p.c_kv_sb;
  const bf16* kr_b = p.k_rope + (int64_t)b * p.k_rope_sb;
  u32x4 pre[C::PRE_L + 1];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < C::PRE_L; ++i) {
      const int q = tid + 256 * i;
      const int row = q / C::LCH;
      const int key = min(t0 + row, n_keys - 1);
      pre[i] = ldg16(ckv_b + (int64_t)key * p.c_kv_st + 8 * (q - row * C::LCH));
    }
    if (tid < 128) {
      const int key = min(t0 + (tid >> 3), n_keys - 1);
      pre[C::PRE_L] = ldg16(kr_b + (int64_t)key * p.k_rope_st + 8 * (tid & 7));
    }
  };
  auto store_tile = [&](unsigned char* buf) {
#pragma unroll
    for (int i = 0; i < C::PRE_L; ++i) {
      const int q = tid + 256 * i;
      const int row = q / C::LCH;
      const int c = q - row * C::LCH;
      sts16(buf + (row * C::RS + (c ^ pc_swz(row))) * 16, pre[i]);
    }
    if (tid < 128) {
      const int row = tid >> 3;
      const int c = C::LCH + (tid & 7);
      sts16(buf + (row * C::RS + (c ^ pc_swz(row))) * 16, pre[C::PRE_L]);
    }
  };

  // LDS read offsets.  Scores (A operand): row l16, chunk 4 ks + G.
  const int swA = pc_swz(l16);
  const int offA0 = l16 * C::RS * 16 + ((0 + G) ^ swA) * 16;
  const int offA1 = l16 * C::RS * 16 + ((4 + G) ^ swA) * 16;
  // P V (transpose read): lane r of group G reads row 4 G + r / 4, columns 16 nb + 4 (r % 4)
  // + [0, 4), so lane (i, G) receives C[4 G + j][16 nb + i], j = 0..3: the A operand of O^T
  // (row = latent column 16 nb + i, K slots = tokens 4 G + j)
  const int rowB = 4 * G + (l16 >> 2);
  const int swB = pc_swz(rowB);
  const int qB = (l16 & 3) >> 1, halfB = l16 & 1;
  int offB[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) offB[j] = rowB * C::RS * 16 + (((2 * j) ^ (swB & 6)) + ((qB ^ swB) & 1)) * 16 + halfB * 8;

  f32x4 oacc[C::NB];
#pragma unroll
  for (int nb = 0; nb < C::NB; ++nb) oacc[nb] = f32x4{};
  float m_run = -INFINITY;  // log2-domain running max of head h (the same in the 4 lane groups)
  float l_part = 0.f;       // this lane's share of the running sum (its 4 tokens per tile)

  load_tile(0);
  store_tile(tiles);
  if (n_tiles > 1) load_tile(C::TT);
  __syncthreads();

  for (int j = 0; j < n_tiles; ++j) {
    unsigned char* cur = tiles + (j & 1) * C::TILE;
    // tile j + 1 goes to the other buffer, whose last readers (tile j - 1) passed the barrier
    if (j + 1 < n_tiles) {
      store_tile(tiles + ((j + 1) & 1) * C::TILE);
      if (j + 2 < n_tiles) load_tile((j + 2) * C::TT);
    }
    const int t0 = j * C::TT;
    if (active && t0 < lim) {  // a tile wholly past the query's keys adds nothing
      // S^T: acc[r] = S[token 4 G + r][head l16]
      f32x4 sacc = f32x4{};
#pragma unroll
      for (int ks = 0; ks < C::NKS; ++ks) {
        const int off = ((ks & 1) ? offA1 : offA0) + (ks >> 1) * 128;
        sacc = mfma16(as_bf16x8(lds16(cur + off)), qf[ks], sacc);
      }
      float x[4];
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = t0 + 4 * G + r;
        x[r] = key < lim ? sacc[r] * p.scale_log2 : -INFINITY;
        mloc = fmaxf(mloc, x[r]);
      }
      mloc = fmaxf(mloc, wave_shfl_xor(mloc, 16));
      mloc = fmaxf(mloc, wave_shfl_xor(mloc, 32));
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
      float pr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = fast_exp2(x[r] - m_use);
        l_part += pr[r];
      }
      // P^T as the B operand of the 16x16x16 MFMA: column = head l16, K slots = tokens 4 G + e
      const s16x4 pa = __builtin_bit_cast(s16x4, u32x2{pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3])});
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) {
        const int off = offB[nb & 3] + (nb >> 2) * 128;
        const s16x4 bv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(cur + off));
        oacc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bv, pa, oacc[nb], 0, 0, 0);
      }
    }
    __syncthreads();  // tile j is consumed; tile j + 1 is in place
  }

  // ---- ctx and LSE of this wave's query: lane (l16, G) holds columns 16 nb + 4 G + [0, 4)
  float lsum = l_part;
  lsum += wave_shfl_xor(lsum, 16);
  lsum += wave_shfl_xor(lsum, 32);
  if (active && h_ok) {
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

}  // namespace mla

using namespace mla;

extern "C" int mla_prefill_cached(const mla_prefill_cached_args* a, void* stream) {
  const char* op = "mla_prefill_cached";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_TRY(check_scale(op, a->scale));
  MLA_CHECK(a->d_rope == 64, MLA_ERR_UNSUPPORTED, "%s: d_rope must be 64", op);
  MLA_CHECK(a->d_latent == 128 || a->d_latent == 256 || a->d_latent == 384 || a->d_latent == 512,
            MLA_ERR_UNSUPPORTED, "%s: d_latent %lld not built (128, 256, 384, 512)", op, (long long)a->d_latent);
  MLA_CHECK(a->B >= 0 && a->T >= 0 && a->H >= 0 && a->L0 >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
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
  MLA_CHECK(((uintptr_t)a->ctx & 7) == 0 && a->ctx_stride.b >= 0 && a->ctx_stride.t >= 0 && a->ctx_stride.h >= 0 &&
                (a->ctx_stride.b & 3) == 0 && (a->ctx_stride.t & 3) == 0 && (a->ctx_stride.h & 3) == 0,
            MLA_ERR_INVALID_ARG, "%s: ctx must be 8-byte aligned with strides multiples of 4", op);
  const int n_hg = (int)((a->H + 15) / 16);
  const int n_qb = (int)((a->T + PcCfg<512>::NQ - 1) / PcCfg<512>::NQ);
  const int64_t n_wg = a->B * (int64_t)n_hg * n_qb;
  MLA_CHECK(n_wg < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: grid too large", op);
  PcParams prm;
  prm.q_lat = (const bf16*)a->q_lat;
  prm.q_rope = (const bf16*)a->q_rope;
  prm.c_kv = (const bf16*)a->c_kv;
  prm.k_rope = (const bf16*)a->k_rope;
  prm.ctx = (bf16*)a->ctx;
  prm.lse = a->lse;
  prm.B = (int)a->B;
  prm.T = (int)a->T;
  prm.H = (int)a->H;
  prm.L0 = (int)a->L0;
  prm.n_hg = n_hg;
  prm.n_qb = n_qb;
  prm.ql_s = a->q_lat_stride;
  prm.qr_s = a->q_rope_stride;
  prm.ctx_s = a->ctx_stride;
  prm.c_kv_sb = a->c_kv_sb;
  prm.c_kv_st = a->c_kv_st;
  prm.k_rope_sb = a->k_rope_sb;
  prm.k_rope_st = a->k_rope_st;
  prm.scale_log2 = a->scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)n_wg), block(256);
  switch (a->d_latent) {
    case 128: prefill_cached_kernel<128><<<grid, block, 0, s>>>(prm); break;
    case 256: prefill_cached_kernel<256><<<grid, block, 0, s>>>(prm); break;
    case 384: prefill_cached_kernel<384><<<grid, block, 0, s>>>(prm); break;
    default: prefill_cached_kernel<512><<<grid, block, 0, s>>>(prm); break;
  }
  return launch_status(op);
}
