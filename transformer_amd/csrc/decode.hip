// Absorbed latent-KV decode for MLA (one query token per sequence), gfx950.
//
// Restates the T == 1 absorbed branch of transformer.py:249-286:
//   s_j = (q_lat . c_kv[j] + q_rope . k_rope[j]) * scale      (:259-269)
//   p   = softmax(s)                                          (:283)
//   ctx = sum_j p_j c_kv[j]                                   (:286)
// with q_lat = q_nope W_UK computed by the caller (:252-254) and W_UV applied
// after (:290-291).
//
// HBM-bound: the cache (c_kv [L][DL] + k_rope [L][64] per sequence) is the only
// large operand and is read exactly once for all heads.  Work decomposition:
//   grid = (split, batch, head-group of 16 heads); a split is a contiguous token
//   range; one workgroup (4 waves) walks it in 64-token tiles:
//     1. stage the tile [64][DL (+64)] in LDS (register prefetch of the next tile
//        is issued before the math of the current one);
//     2. S^T [64 tok][16 heads] = Ck [64][DL+64] . Q^T   (MFMA 16x16x32, wave w owns
//        tokens 16w..16w+15; the shared k_rope is simply 64 more columns of the row);
//     3. online softmax per head (max across the 4 waves through LDS);
//     4. O [16 heads][DL] += P [16][64] . Ck [64][DL]     (MFMA 16x16x32, wave w owns
//        DL/4 columns).
//   Splits write normalised partials and log2-domain LSEs; a second kernel merges
//   them in split order (deterministic, no atomics).
#include "mla_common.h"

namespace mla {

struct DecParams {
  const bf16 *q_lat, *q_rope, *c_kv, *k_rope;
  const int32_t* seq_lens;
  bf16* ctx;
  float* lse;
  float* part_o;    // [B][n_hg*16][S][DL] (normalised), used when S > 1
  float* part_lse;  // [B][n_hg*16][S] log2 domain
  int B, H, L, S, chunk;
  int64_t q_lat_sb, q_lat_sh, q_rope_sb, q_rope_sh;
  int64_t c_kv_sb, c_kv_st;
  int64_t k_rope_sb, k_rope_sh, k_rope_st;
  int64_t ctx_sb, ctx_sh;
  float scale_log2;
};

template <int DL, bool SHARED>
struct DecCfg {
  static constexpr int TT = 64;                      // tokens per tile
  static constexpr int KW = DL + (SHARED ? 64 : 0);  // width of a key row used by the QK MFMA
  static constexpr int KROW = KW + 8;                // LDS row stride (elements)
  static constexpr int NKS = KW / 32;                // QK k-steps
  static constexpr int CH_ROW = KW / 8;              // 16-byte chunks per key row
  static constexpr int CH_PER_THREAD = TT * CH_ROW / 256;
  static constexpr int NB = DL / 64;                 // 16-wide d blocks per wave in PV
  static constexpr int PS_LD = TT + 8;
  static_assert((TT * CH_ROW) % 256 == 0, "tile chunks must divide the workgroup");
};

// wide latents keep Q and the next-tile prefetch in registers: one workgroup per CU
// (512 VGPRs per lane) instead of two.
template <int DL, bool SHARED>
__global__ __launch_bounds__(256, DL >= 384 ? 1 : 2) void decode_kernel(DecParams p) {
  using C = DecCfg<DL, SHARED>;
  __shared__ __attribute__((aligned(16))) bf16 Ck[C::TT * C::KROW];
  __shared__ __attribute__((aligned(16))) bf16 Ps[16 * C::PS_LD];
  __shared__ float red[4][16];
  __shared__ float alpha_s[16];
  __shared__ float qr_s[SHARED ? 1 : 16 * 64];

  const int split = blockIdx.x;
  const int b = blockIdx.y;
  const int hg = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int h = hg * 16 + l16;  // head of this lane in the QK / softmax phase
  const bool h_ok = h < p.H;

  int Lb = p.L;
  if (p.seq_lens) {
    const int sl = p.seq_lens[b];
    Lb = sl < 0 ? 0 : (sl < p.L ? sl : p.L);
  }
  const int t_begin = split * p.chunk;
  const int t_end = min(Lb, t_begin + p.chunk);

  // ---- Q fragment: B operand of S^T = Ck . Q^T (column = head, K slot = dim 32 ks + 8 g + e)
  bf16x8 qf[C::NKS];
  {
    const bf16* ql = p.q_lat + (int64_t)b * p.q_lat_sb + (int64_t)(h_ok ? h : 0) * p.q_lat_sh;
    const bf16* qr = p.q_rope + (int64_t)b * p.q_rope_sb + (int64_t)(h_ok ? h : 0) * p.q_rope_sh;
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
      const int d = 32 * ks + 8 * g;
      u32x4 v = d < DL ? ldg16(ql + d) : ldg16(qr + (d - DL));
      if (!h_ok) v = u32x4{0u, 0u, 0u, 0u};
      qf[ks] = as_bf16x8(v);
    }
    if (!SHARED) {
      // per-head k_rope: the rope score is a 64-wide dot per (token, head) done on the VALU
      for (int i = tid; i < 16 * 64; i += 256) {
        const int hh = hg * 16 + i / 64;
        qr_s[i] = hh < p.H ? (float)p.q_rope[(int64_t)b * p.q_rope_sb + (int64_t)hh * p.q_rope_sh + (i & 63)] : 0.f;
      }
    }
  }

  const bf16* ckv_b = p.c_kv + (int64_t)b * p.c_kv_sb;
  const bf16* kr_b = p.k_rope + (int64_t)b * p.k_rope_sb;

  u32x4 pre[C::CH_PER_THREAD];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < C::CH_PER_THREAD; ++i) {
      const int c = tid + 256 * i;
      const int row = c / C::CH_ROW;
      const int col = (c - row * C::CH_ROW) * 8;
      int t = t0 + row;
      t = t < p.L ? t : p.L - 1;
      pre[i] = col < DL ? ldg16(ckv_b + (int64_t)t * p.c_kv_st + col)
                        : ldg16(kr_b + (int64_t)t * p.k_rope_st + (col - DL));
    }
  };

  f32x4 oacc[C::NB];
#pragma unroll
  for (int nb = 0; nb < C::NB; ++nb) oacc[nb] = f32x4{};
  float m_run = -INFINITY;  // per head l16 (log2 domain), identical in every wave
  float l_part = 0.f;       // this lane's share of the row sum of head l16

  const int n_tiles = t_end > t_begin ? (t_end - t_begin + C::TT - 1) / C::TT : 0;
  if (n_tiles > 0) load_tile(t_begin);
  for (int it = 0; it < n_tiles; ++it) {
    const int t0 = t_begin + it * C::TT;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < C::CH_PER_THREAD; ++i) {
      const int c = tid + 256 * i;
      const int row = c / C::CH_ROW;
      const int col = (c - row * C::CH_ROW) * 8;
      sts16(&Ck[row * C::KROW + col], pre[i]);
    }
    __syncthreads();
    if (it + 1 < n_tiles) load_tile(t0 + C::TT);

    // ---- S^T for tokens 16 w + [0, 16): acc[r] = S[tok = 16 w + 4 g + r][head l16]
    f32x4 sacc = f32x4{};
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
      const bf16x8 a = as_bf16x8(lds16(&Ck[(16 * w + l16) * C::KROW + 32 * ks + 8 * g]));
      sacc = mfma16(a, qf[ks], sacc);
    }
    float x[4];
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = t0 + 16 * w + 4 * g + r;
      float s = sacc[r];
      if (!SHARED) {
        const int tl = tok < p.L ? tok : p.L - 1;
        const bf16* kr = kr_b + (int64_t)(h_ok ? h : 0) * p.k_rope_sh + (int64_t)tl * p.k_rope_st;
        float acc = 0.f;
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) {
          const u32x4 v = ldg16(kr + 8 * c8);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc += lo_bf16(v[q]) * qr_s[l16 * 64 + 8 * c8 + 2 * q];
            acc += hi_bf16(v[q]) * qr_s[l16 * 64 + 8 * c8 + 2 * q + 1];
          }
        }
        s += acc;
      }
      x[r] = tok < t_end ? s * p.scale_log2 : -INFINITY;
      mloc = fmaxf(mloc, x[r]);
    }
    mloc = fmaxf(mloc, wave_shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, wave_shfl_xor(mloc, 32));
    if (g == 0) red[w][l16] = mloc;
    __syncthreads();
    const float tmax = fmaxf(fmaxf(red[0][l16], red[1][l16]), fmaxf(red[2][l16], red[3][l16]));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    if (w == 0 && g == 0) alpha_s[l16] = alpha;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = fast_exp2(x[r] - m_use);
      ps += pr;
      // PV k-step kk holds tokens 32 kk + [0, 32); K slot (g', e) <-> token 32 kk + g' + 4 e,
      // stored at Ps[h][32 kk + 8 g' + e]
      const int tl = 16 * w + 4 * g + r;
      const int kk = tl >> 5, tq = tl & 31;
      Ps[l16 * C::PS_LD + 32 * kk + 8 * (tq & 3) + (tq >> 2)] = (bf16)pr;
    }
    l_part = l_part * alpha + ps;
    __syncthreads();

    // ---- O[h][d] += P[h][tok] C[tok][d]; lane: column d = base + 16 nb + l16, rows h = 4 g + r
    float al[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) al[r] = alpha_s[4 * g + r];
#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) oacc[nb][r] *= al[r];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const bf16x8 a = as_bf16x8(lds16(&Ps[l16 * C::PS_LD + 32 * kk + 8 * g]));
      const unsigned short* cbase =
          reinterpret_cast<const unsigned short*>(&Ck[(32 * kk + g) * C::KROW + w * (DL / 4) + l16]);
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) {
        u32x4 bv;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const uint32_t lo = cbase[(8 * e2) * C::KROW + 16 * nb];
          const uint32_t hi = cbase[(8 * e2 + 4) * C::KROW + 16 * nb];
          bv[e2] = lo | (hi << 16);
        }
        oacc[nb] = mfma16(a, as_bf16x8(bv), oacc[nb]);
      }
    }
  }

  // ---- row sums: reduce the per-lane partials over g and over the waves
  float lsum = l_part;
  lsum += wave_shfl_xor(lsum, 16);
  lsum += wave_shfl_xor(lsum, 32);
  __syncthreads();
  if (g == 0) red[w][l16] = lsum;
  __syncthreads();
  float lh[4], mh[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * g + r;
    lh[r] = red[0][hh] + red[1][hh] + red[2][hh] + red[3][hh];
  }
  // m_run of head (4 g + r) lives in lanes with l16 == 4 g + r: fetch it through LDS
  __syncthreads();
  if (w == 0 && g == 0) alpha_s[l16] = m_run;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) mh[r] = alpha_s[4 * g + r];

  if (p.S == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hh = hg * 16 + 4 * g + r;
      if (hh >= p.H) continue;
      const float inv = lh[r] > 0.f ? 1.f / lh[r] : 0.f;
      bf16* cp = p.ctx + (int64_t)b * p.ctx_sb + (int64_t)hh * p.ctx_sh + w * (DL / 4) + l16;
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) cp[16 * nb] = (bf16)(oacc[nb][r] * inv);
      if (w == 0 && l16 == 0)
        p.lse[(int64_t)b * p.H + hh] = lh[r] > 0.f ? (mh[r] + fast_log2(lh[r])) * kLn2 : -INFINITY;
    }
  } else {
    const int HP = gridDim.z * 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hh = hg * 16 + 4 * g + r;
      const float inv = lh[r] > 0.f ? 1.f / lh[r] : 0.f;
      float* po = p.part_o + (((int64_t)b * HP + hh) * p.S + split) * DL + w * (DL / 4) + l16;
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) po[16 * nb] = oacc[nb][r] * inv;
      if (w == 0 && l16 == 0)
        p.part_lse[((int64_t)b * HP + hh) * p.S + split] = lh[r] > 0.f ? mh[r] + fast_log2(lh[r]) : -INFINITY;
    }
  }
}

// Merge split partials in split order: lse = log2 sum 2^lse_s, ctx = sum 2^(lse_s - lse) o_s.
template <int DL>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecParams p) {
  const int b = blockIdx.x / p.H;
  const int h = blockIdx.x - b * p.H;
  const int HP = ((p.H + 15) / 16) * 16;
  const float* pl = p.part_lse + ((int64_t)b * HP + h) * p.S;
  float m = -INFINITY;
  for (int s = 0; s < p.S; ++s) m = fmaxf(m, pl[s]);
  float tot = 0.f;
  for (int s = 0; s < p.S; ++s) tot += pl[s] == -INFINITY ? 0.f : fast_exp2(pl[s] - m);
  const float inv = tot > 0.f ? 1.f / tot : 0.f;
  const float* po = p.part_o + ((int64_t)b * HP + h) * p.S * DL;
  bf16* cp = p.ctx + (int64_t)b * p.ctx_sb + (int64_t)h * p.ctx_sh;
  for (int d = threadIdx.x; d < DL; d += 128) {
    float acc = 0.f;
    for (int s = 0; s < p.S; ++s) {
      const float ws = pl[s] == -INFINITY ? 0.f : fast_exp2(pl[s] - m);
      acc += ws * po[(int64_t)s * DL + d];
    }
    cp[d] = (bf16)(acc * inv);
  }
  if (threadIdx.x == 0) p.lse[(int64_t)b * p.H + h] = tot > 0.f ? (m + fast_log2(tot)) * kLn2 : -INFINITY;
}

static int pick_splits(const mla_decode_args* a, int n_hg) {
  const int64_t tiles = (a->L + 63) / 64;
  if (a->num_splits > 0) return (int)std::min<int64_t>(a->num_splits, std::max<int64_t>(tiles, 1));
  const int64_t wgs = a->B * n_hg;
  int64_t s = (512 + wgs - 1) / wgs;  // aim at ~2 workgroups per CU on 256 CUs
  s = std::min<int64_t>(s, std::max<int64_t>(tiles / 2, 1));  // keep >= 2 tiles per split
  return (int)std::max<int64_t>(s, 1);
}

static void dec_layout(const mla_decode_args* a, int& n_hg, int& S, int& chunk, size_t& ws_o, size_t& ws_l) {
  n_hg = (int)((a->H + 15) / 16);
  S = pick_splits(a, n_hg);
  const int64_t per = (a->L + S - 1) / S;
  chunk = (int)(((per + 63) / 64) * 64);
  S = (int)((a->L + chunk - 1) / chunk);  // drop splits that would start past L
  if (S < 1) S = 1;
  const size_t HP = (size_t)n_hg * 16;
  ws_o = S > 1 ? (size_t)a->B * HP * S * a->d_latent * sizeof(float) : 0;
  ws_l = S > 1 ? (size_t)a->B * HP * S * sizeof(float) : 0;
}

template <int DL, bool SHARED>
static void launch_dec(const DecParams& prm, int n_hg, hipStream_t s) {
  decode_kernel<DL, SHARED><<<dim3(prm.S, prm.B, n_hg), dim3(256), 0, s>>>(prm);
  if (prm.S > 1) decode_combine_kernel<DL><<<dim3(prm.B * prm.H), dim3(128), 0, s>>>(prm);
}

template <bool SHARED>
static int dispatch_dec(int DL, const DecParams& prm, int n_hg, hipStream_t s) {
  switch (DL) {
    case 64: launch_dec<64, SHARED>(prm, n_hg, s); break;
    case 128: launch_dec<128, SHARED>(prm, n_hg, s); break;
    case 256: launch_dec<256, SHARED>(prm, n_hg, s); break;
    case 384: launch_dec<384, SHARED>(prm, n_hg, s); break;
    case 512: launch_dec<512, SHARED>(prm, n_hg, s); break;
    default: set_error("mla_decode: d_latent %d not built", DL); return MLA_ERR_UNSUPPORTED;
  }
  return launch_status("mla_decode");
}

}  // namespace mla

using namespace mla;

extern "C" size_t mla_decode_workspace_bytes(const mla_decode_args* a) {
  if (!a || a->B <= 0 || a->H <= 0 || a->L <= 0 || a->d_latent <= 0) return 0;
  int n_hg, S, chunk;
  size_t wo, wl;
  dec_layout(a, n_hg, S, chunk, wo, wl);
  return wo + wl + (wo ? 256 : 0);
}

extern "C" int mla_decode(const mla_decode_args* a, void* stream) {
  const char* op = "mla_decode";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->d_rope == 64, MLA_ERR_UNSUPPORTED, "%s: d_rope must be 64", op);
  MLA_CHECK(a->d_latent == 64 || a->d_latent == 128 || a->d_latent == 256 || a->d_latent == 384 ||
                a->d_latent == 512,
            MLA_ERR_UNSUPPORTED, "%s: d_latent %lld not built (64, 128, 256, 384, 512)", op, (long long)a->d_latent);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->L >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->B < 65536 && a->H < 65536 && a->L < (1ll << 30), MLA_ERR_INVALID_ARG, "%s: size out of range", op);
  if (a->B == 0 || a->H == 0) return MLA_OK;
  MLA_CHECK(a->L > 0, MLA_ERR_INVALID_ARG, "%s: empty cache (L = 0)", op);
  MLA_CHECK(a->n_k_rope_heads == 1 || a->n_k_rope_heads == a->H, MLA_ERR_INVALID_ARG,
            "%s: n_k_rope_heads must be 1 or H", op);
  MLA_CHECK(a->q_lat && a->q_rope && a->c_kv && a->k_rope && a->ctx && a->lse, MLA_ERR_INVALID_ARG,
            "%s: null pointer", op);
  const void* ptrs[] = {a->q_lat, a->q_rope, a->c_kv, a->k_rope};
  for (const void* q : ptrs) MLA_CHECK(((uintptr_t)q & 15) == 0, MLA_ERR_INVALID_ARG, "%s: inputs must be 16-byte aligned", op);
  const int64_t strides[] = {a->q_lat_sb, a->q_lat_sh, a->q_rope_sb, a->q_rope_sh, a->c_kv_sb,
                             a->c_kv_st,  a->k_rope_sb, a->k_rope_sh, a->k_rope_st};
  for (int64_t st : strides)
    MLA_CHECK(st >= 0 && (st & 7) == 0, MLA_ERR_INVALID_ARG, "%s: strides must be non-negative multiples of 8", op);
  MLA_CHECK(a->n_k_rope_heads != 1 || a->k_rope_sh == 0, MLA_ERR_INVALID_ARG,
            "%s: a shared k_rope head needs head stride 0", op);
  MLA_CHECK(a->ctx_sb >= 0 && a->ctx_sh >= 0, MLA_ERR_INVALID_ARG, "%s: negative ctx strides", op);

  int n_hg, S, chunk;
  size_t wo, wl;
  dec_layout(a, n_hg, S, chunk, wo, wl);
  if (S > 1) {
    MLA_CHECK(a->workspace && a->workspace_bytes >= wo + wl, MLA_ERR_WORKSPACE,
              "%s: workspace of %zu bytes required (got %zu)", op, wo + wl, a->workspace_bytes);
    MLA_CHECK(((uintptr_t)a->workspace & 15) == 0, MLA_ERR_WORKSPACE, "%s: workspace must be 16-byte aligned", op);
  }
  DecParams prm;
  prm.q_lat = (const bf16*)a->q_lat;
  prm.q_rope = (const bf16*)a->q_rope;
  prm.c_kv = (const bf16*)a->c_kv;
  prm.k_rope = (const bf16*)a->k_rope;
  prm.seq_lens = a->seq_lens;
  prm.ctx = (bf16*)a->ctx;
  prm.lse = a->lse;
  prm.part_o = S > 1 ? (float*)a->workspace : nullptr;
  prm.part_lse = S > 1 ? (float*)((char*)a->workspace + wo) : nullptr;
  prm.B = (int)a->B;
  prm.H = (int)a->H;
  prm.L = (int)a->L;
  prm.S = S;
  prm.chunk = chunk;
  prm.q_lat_sb = a->q_lat_sb;
  prm.q_lat_sh = a->q_lat_sh;
  prm.q_rope_sb = a->q_rope_sb;
  prm.q_rope_sh = a->q_rope_sh;
  prm.c_kv_sb = a->c_kv_sb;
  prm.c_kv_st = a->c_kv_st;
  prm.k_rope_sb = a->k_rope_sb;
  prm.k_rope_sh = a->k_rope_sh;
  prm.k_rope_st = a->k_rope_st;
  prm.ctx_sb = a->ctx_sb;
  prm.ctx_sh = a->ctx_sh;
  prm.scale_log2 = a->scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  return a->n_k_rope_heads == 1 ? dispatch_dec<true>((int)a->d_latent, prm, n_hg, s)
                                : dispatch_dec<false>((int)a->d_latent, prm, n_hg, s);
}
