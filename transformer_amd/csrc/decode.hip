// Absorbed latent-KV decode for MLA (one query token per sequence), gfx950.
//
// Restates the T == 1 absorbed branch of transformer.py:249-286:
//   s_j = (q_lat . c_kv[j] + q_rope . k_rope[j]) * scale      (:259-269)
//   p   = softmax(s)                                          (:283)
//   ctx = sum_j p_j c_kv[j]                                   (:286)
// with q_lat = q_nope W_UK computed by the caller (:252-254) and W_UV applied
// after (:290-291).
//
// HBM-bound: the cache (c_kv [L][DL] + k_rope [L][64] per sequence) is the only large
// operand and is read exactly once for all 16 heads of a head group.
//
// Work decomposition.  A workgroup (4 waves) owns one (batch, head group, context
// split).  Inside it every wave streams its own 16-token tiles (tiles w, w+4, ...):
//   * the next tile is prefetched into registers while the current one is in the
//     wave's private LDS buffer (no workgroup barrier in the loop);
//   * S^T [16 tok][16 heads] = C [16 tok][KW] . Q^T     v_mfma_f32_16x16x32_bf16, the
//     shared k_rope being 64 more columns of the row (KW = DL + 64);
//   * online softmax per head inside the wave (lane = head, registers = tokens);
//   * O^T [DL][16 heads] += C^T [DL][16 tok] . P^T [16 tok][16 heads]
//     (v_mfma_f32_16x16x16_bf16): C^T comes from ds_read_b64_tr_b16 (the LDS transpose
//     read) of the same row-major tile the QK step used, P^T straight from the S^T
//     accumulators; a lane then owns 4 consecutive columns of its own head, so the
//     softmax rescale is per lane and the stores are vectors.
// The 4 waves then merge (m, l, O) through LDS in a fixed order and the workgroup
// stores its rows with coalesced 16-byte stores.  With several splits each workgroup
// writes a normalised bf16 partial and its log2-domain LSE, and decode_merge_kernel
// combines the splits in split order (deterministic, no atomics).  Splits of one
// (batch, head group) are placed on one XCD so the partials stay in that XCD's L2.
//
// LDS tile layout: row t of a tile holds KW bf16 as 16-byte chunks; chunk c sits at
// position c ^ sw(t) (sw(t) in [0, 8), a permutation of bits 1..3 of t) with a row
// stride of RS chunks (RS * 16 bytes = 128 mod 256), which keeps both the QK reads
// (16 tokens x one chunk) and the transpose reads (4 tokens x 2 chunks per 16 lanes)
// free of bank conflicts.
#include <mutex>

#include "mla_common.h"

namespace mla {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct DecParams {
  const bf16 *q_lat, *q_rope, *c_kv, *k_rope;
  const int32_t* seq_lens;
  bf16* ctx;
  float* lse;
  float* part_lse;     // [B * n_hg][S][16] log2 domain (S > 1)
  bf16* part_o;        // [B * n_hg][S][16][DL] normalised (S > 1)
  int B, H, L, S, chunk, n_hg;
  int64_t q_lat_sb, q_lat_sh, q_rope_sb, q_rope_sh;
  int64_t c_kv_sb, c_kv_st;
  int64_t k_rope_sb, k_rope_sh, k_rope_st;
  int64_t ctx_sb, ctx_sh;
  float scale_log2;
};

template <int DL, bool SHARED>
struct DecCfg {
  static constexpr int TT = 16;                          // tokens per wave tile
  static constexpr int KW = DL + (SHARED ? 64 : 0);      // columns of a staged row
  static constexpr int NCH = KW / 8;                     // 16-byte chunks per row
  static constexpr int RS = (NCH % 16 == 8) ? NCH : NCH + 8;  // row stride in chunks
  static constexpr int NKS = KW / 32;                    // QK k-steps
  static constexpr int NB = DL / 16;                     // PV column blocks
  static constexpr int PRE = TT * NCH / 64;              // prefetch chunks per lane
  static constexpr int WAVE_LDS = TT * RS * 16;          // bytes per wave buffer
  static_assert((TT * NCH) % 64 == 0, "tile chunks must divide the wave");
  static_assert(NCH % 8 == 0, "swizzle works on groups of 8 chunks");
  static constexpr int O_LDS = 4 * NB * 64 * 16;         // the four waves' O^T for the end merge
  static constexpr int LDS = O_LDS > 4 * WAVE_LDS ? O_LDS : 4 * WAVE_LDS;  // tile buffers, then O^T
};

// growth of a head's running max (log2 units) that triggers a rescale of O
constexpr float kRescale = 8.0f;

// swizzle of token t's chunk index: a permutation of bits (1, 2, 3) of t
__device__ __forceinline__ int tok_swz(int t) { return ((t >> 2) & 1) | (((t >> 3) & 1) << 1) | (((t >> 1) & 1) << 2); }

// linear workgroup id -> (unit = b * n_hg + hg, split), splits of one unit on one XCD
__device__ __forceinline__ void dec_coords(const DecParams& p, int& unit, int& split) {
  const int n = gridDim.x;
  int id = blockIdx.x;
  if ((n & 7) == 0) id = (id & 7) * (n >> 3) + (id >> 3);
  unit = id / p.S;
  split = id - unit * p.S;
}

template <int DL, bool SHARED>
__global__ __launch_bounds__(256, 1) void decode_kernel(DecParams p) {
  using C = DecCfg<DL, SHARED>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[C::LDS];
  __shared__ __attribute__((aligned(16))) unsigned char qs[16 * C::RS * 16];
  __shared__ __attribute__((aligned(16))) unsigned char qrs[SHARED ? 16 : 16 * 9 * 16];
  __shared__ float m_s[4][16], l_s[4][16];

  int unit, split;
  dec_coords(p, unit, split);
  const int b = unit / p.n_hg;
  const int hg = unit - b * p.n_hg;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: tile addresses stay scalar
  const int l16 = lane & 15, G = lane >> 4;
  const int h = hg * 16 + l16;  // head of this lane in S^T (column) and softmax
  const bool h_ok = h < p.H;

  int Lb = p.L;
  if (p.seq_lens) {
    const int sl = p.seq_lens[b];
    Lb = sl < 0 ? 0 : (sl < p.L ? sl : p.L);
  }
  // with per-sequence lengths each sequence splits its own length (the host's chunk covers L):
  // whole 16-token tiles for each of the 4 waves
  const int chunk = p.seq_lens ? ((Lb + p.S - 1) / p.S + 63) / 64 * 64 : p.chunk;
  const int t_begin = split * chunk;
  const int t_end = min(Lb, t_begin + chunk);
  const int n_tiles = t_end > t_begin ? (t_end - t_begin + C::TT - 1) / C::TT : 0;

  const bf16* ckv_b = p.c_kv + (int64_t)b * p.c_kv_sb;
  const bf16* kr_b = p.k_rope + (int64_t)b * p.k_rope_sb;
  unsigned char* buf = lds + w * C::WAVE_LDS;

  // prefetch, in two uniform loops: latent chunk q = 64 i + lane of the tile (row q / (DL/8)),
  // then the shared k_rope chunks (2 per lane, 8 per row).  Rows past the sequence's length
  // repeat its last row: a capacity-sized cache may hold anything (even NaN) there, and a
  // masked score's p = 0 must not meet it in the PV product.  (n_tiles > 0 implies Lb > 0.)
  constexpr int LCH = DL / 8;            // latent chunks per row
  constexpr int PRE_L = C::TT * LCH / 64;
  constexpr int PRE_R = SHARED ? C::TT * 8 / 64 : 0;
  static_assert(PRE_L + PRE_R == C::PRE, "prefetch split");
  u32x4 pre[C::PRE];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < PRE_L; ++i) {
      const int q = 64 * i + lane;
      const int row = q / LCH;
      int t = t0 + row;
      t = t < Lb ? t : Lb - 1;
      pre[i] = ldg16(ckv_b + (int64_t)t * p.c_kv_st + 8 * (q - row * LCH));
    }
#pragma unroll
    for (int i = 0; i < PRE_R; ++i) {
      const int q = 64 * i + lane;
      int t = t0 + (q >> 3);
      t = t < Lb ? t : Lb - 1;
      pre[PRE_L + i] = ldg16(kr_b + (int64_t)t * p.k_rope_st + 8 * (q & 7));
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < PRE_L; ++i) {
      const int q = 64 * i + lane;
      const int row = q / LCH;
      const int c = q - row * LCH;
      sts16(buf + (row * C::RS + (c ^ tok_swz(row))) * 16, pre[i]);
    }
#pragma unroll
    for (int i = 0; i < PRE_R; ++i) {
      const int q = 64 * i + lane;
      const int row = q >> 3;
      const int c = LCH + (q & 7);
      sts16(buf + (row * C::RS + (c ^ tok_swz(row))) * 16, pre[PRE_L + i]);
    }
  };

  // the first tile is in flight while Q is staged
  int k = w;
  if (k < n_tiles) load_tile(t_begin + k * C::TT);

  // ---- Q^T (B operand of S^T = C . Q^T: column = head, K slot = dim 32 ks + 8 G + e) is
  // staged once in LDS with the tile swizzle (row = head); per-head q_rope rows too.
  // Order: tile k is in flight, Q is loaded, tile k goes to LDS and tile k + 4 is issued,
  // then Q is written: Q's latency overlaps the second tile's.
  constexpr int QCH = (16 * C::NCH + 255) / 256;  // Q chunks per thread
  u32x4 qreg[QCH];
#pragma unroll
  for (int i = 0; i < QCH; ++i) {
    const int q = tid + 256 * i;
    qreg[i] = u32x4{0u, 0u, 0u, 0u};
    if (q < 16 * C::NCH) {
      const int hr = q / C::NCH;
      const int c = q - hr * C::NCH;
      const int hh = hg * 16 + hr;
      if (hh < p.H) {
        const bf16* ql = p.q_lat + (int64_t)b * p.q_lat_sb + (int64_t)hh * p.q_lat_sh;
        const bf16* qr = p.q_rope + (int64_t)b * p.q_rope_sb + (int64_t)hh * p.q_rope_sh;
        qreg[i] = c < DL / 8 ? ldg16(ql + 8 * c) : ldg16(qr + 8 * (c - DL / 8));
      }
    }
  }
  bool staged = false;  // tile k already in LDS
  if (k < n_tiles) {
    store_tile();
    staged = true;
    if (k + 4 < n_tiles) load_tile(t_begin + (k + 4) * C::TT);
  }
#pragma unroll
  for (int i = 0; i < QCH; ++i) {
    const int q = tid + 256 * i;
    if (q < 16 * C::NCH) {
      const int hr = q / C::NCH;
      const int c = q - hr * C::NCH;
      sts16(qs + (hr * C::RS + (c ^ tok_swz(hr))) * 16, qreg[i]);
    }
  }
  if (!SHARED) {
    for (int q = tid; q < 16 * 8; q += 256) {
      const int hr = q >> 3, c = q & 7;
      const int hh = hg * 16 + hr;
      const u32x4 v = hh < p.H ? ldg16(p.q_rope + (int64_t)b * p.q_rope_sb + (int64_t)hh * p.q_rope_sh + 8 * c)
                               : u32x4{0u, 0u, 0u, 0u};
      sts16(qrs + (hr * 9 + c) * 16, v);
    }
  }
  __syncthreads();

  // LDS read offsets.  QK (A operand): row l16, chunk 4 ks + G.
  const int swA = tok_swz(l16);
  const int offA0 = l16 * C::RS * 16 + ((0 + G) ^ swA) * 16;
  const int offA1 = l16 * C::RS * 16 + ((4 + G) ^ swA) * 16;
  // PV (transpose read): lane r of group G reads row 4 G + r / 4, columns 16 nb + 4 (r % 4) + [0, 4),
  // so lane (i, G) receives C[4 G + j][16 nb + i], j = 0..3: the A operand of O^T (row = column
  // 16 nb + i, K slots = tokens 4 G + j)
  const int rowB = 4 * G + (l16 >> 2);
  const int swB = tok_swz(rowB);
  const int qB = (l16 & 3) >> 1, halfB = l16 & 1;
  int offB[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) offB[j] = rowB * C::RS * 16 + (((2 * j) ^ (swB & 6)) + ((qB ^ swB) & 1)) * 16 + halfB * 8;

  f32x4 oacc[C::NB];
#pragma unroll
  for (int nb = 0; nb < C::NB; ++nb) oacc[nb] = f32x4{};
  float m_run = -INFINITY;  // log2-domain running max of head h (same in the 4 lane groups)
  float l_part = 0.f;       // this lane's share of the running sum (its 4 tokens per tile)

  for (; k < n_tiles; k += 4) {
    const int t0 = t_begin + k * C::TT;
    if (!staged) {
      store_tile();
      if (k + 4 < n_tiles) load_tile(t0 + 4 * C::TT);
    }
    staged = false;

    // S^T: acc[r] = S[token 4 G + r][head l16]
    f32x4 sacc = f32x4{};
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
      const int off = ((ks & 1) ? offA1 : offA0) + (ks >> 1) * 128;
      sacc = mfma16(as_bf16x8(lds16(buf + off)), as_bf16x8(lds16(qs + off)), sacc);
    }
    if (!SHARED) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int t = t0 + 4 * G + r;
        t = t < Lb ? t : Lb - 1;
        const bf16* kr = kr_b + (int64_t)(h_ok ? h : 0) * p.k_rope_sh + (int64_t)t * p.k_rope_st;
        float acc = 0.f;
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) {
          const u32x4 v = ldg16(kr + 8 * c8);
          const u32x4 qv = lds16(qrs + (l16 * 9 + c8) * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc += lo_bf16(v[e]) * lo_bf16(qv[e]);
            acc += hi_bf16(v[e]) * hi_bf16(qv[e]);
          }
        }
        sacc[r] += acc;
      }
    }

    // online softmax of head l16 over this tile's 16 tokens
    float x[4];
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * G + r;
      x[r] = t < t_end ? sacc[r] * p.scale_log2 : -INFINITY;
      mloc = fmaxf(mloc, x[r]);
    }
    mloc = xor16_max(mloc);
    mloc = xor32_max(mloc);
    // Lazy rescaling: the reference max m_run only moves when a head's tile max exceeds it
    // by more than kRescale (log2 units), so p <= 2^kRescale and O, l and the final LSE all
    // use the same m_run; the O rescale (a pass over every accumulator) is then rare.
    if (__any(mloc > m_run + kRescale)) {
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
#pragma unroll
      for (int nb = 0; nb < C::NB; ++nb) oacc[nb] *= alpha;  // O^T columns are head l16
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = fast_exp2(x[r] - m_use);
      l_part += pr[r];
    }
    // P^T as the B operand of the 16x16x16 MFMA: column = head l16, K slots = tokens 4 G + e
    const uint32_t p01 = pack_bf16x2(pr[0], pr[1]);
    const uint32_t p23 = pack_bf16x2(pr[2], pr[3]);
    const s16x4 pa = __builtin_bit_cast(s16x4, u32x2{p01, p23});

#pragma unroll
    for (int nb = 0; nb < C::NB; ++nb) {
      const int off = offB[nb & 3] + (nb >> 2) * 128;
      const s16x4 bv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(buf + off));
      oacc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bv, pa, oacc[nb], 0, 0, 0);
    }
  }

  // ---- merge the 4 waves: M = max_w m_w, O = sum_w 2^(m_w - M) O_w, L likewise
  float lsum = l_part;
  lsum = xor16_sum(lsum);
  lsum = xor32_sum(lsum);
  if (G == 0) {
    m_s[w][l16] = m_run;
    l_s[w][l16] = lsum;
  }
  __syncthreads();  // every wave is done with its tiles: the buffers take the O^T slots
  // every wave's unscaled O^T in a lane-major slot [NB][64] f32x4 of its own; each wave then
  // scales and sums the four slots of its column blocks (one pass, two barriers in all)
  f32x4* xo = reinterpret_cast<f32x4*>(lds);
#pragma unroll
  for (int nb = 0; nb < C::NB; ++nb) xo[(w * C::NB + nb) * 64 + lane] = oacc[nb];
  __syncthreads();
  // this lane's head l16: M = max_w m_w, f_w = 2^(m_w - M), L = sum_w f_w l_w
  float Mh, Lh = 0.f, fv[4];
  {
    Mh = fmaxf(fmaxf(m_s[0][l16], m_s[1][l16]), fmaxf(m_s[2][l16], m_s[3][l16]));
    const float Mu = Mh == -INFINITY ? 0.f : Mh;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      fv[v] = fast_exp2(m_s[v][l16] - Mu);
      Lh += l_s[v][l16] * fv[v];
    }
  }

  // wave w stores column blocks nb = w, w + 4, ...: lane (l16, G) holds columns
  // 16 nb + 4 G + [0, 4) of head l16
  const int hh = hg * 16 + l16;
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  const float lse2 = Lh > 0.f ? Mh + fast_log2(Lh) : -INFINITY;
  for (int nb = w; nb < C::NB; nb += 4) {
#pragma clang fp contract(off)
    // fixed order (f_0 O_0 + f_2 O_2) + (f_1 O_1 + f_3 O_3), each product rounded on its own
    const f32x4 o0 = xo[nb * 64 + lane] * fv[0], o1 = xo[(C::NB + nb) * 64 + lane] * fv[1];
    const f32x4 o2 = xo[(2 * C::NB + nb) * 64 + lane] * fv[2], o3 = xo[(3 * C::NB + nb) * 64 + lane] * fv[3];
    const f32x4 o = ((o0 + o2) + (o1 + o3)) * inv;
    const int col = 16 * nb + 4 * G;
    if (p.S == 1) {
      if (hh < p.H)
        stg8(p.ctx + (int64_t)b * p.ctx_sb + (int64_t)hh * p.ctx_sh + col,
             u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])});
    } else {
      stg8(p.part_o + (((int64_t)unit * p.S + split) * 16 + l16) * DL + col,
           u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])});
    }
  }
  if (w == 0 && G == 0) {
    if (p.S == 1) {
      if (hh < p.H) p.lse[(int64_t)b * p.H + hh] = lse2 * kLn2;
    } else {
      p.part_lse[((int64_t)unit * p.S + split) * 16 + l16] = lse2;
    }
  }
}

// Merge the S split partials of every (batch, head) in split order:
//   lse = log2 sum_s 2^lse_s,  ctx = sum_s 2^(lse_s - lse) o_s.
// One thread per 4 consecutive columns of one head; every partial element is read once.
// Splits are taken in chunks of 8 whose loads are all issued before any is used (the
// index is clamped and the value masked, so no branch stands between them): up to 8
// splits cost one memory round trip.  Within a chunk the max is taken first and the
// terms are added in split order; a later chunk rescales the running sums.
// Merge of the S split partials of one (b, head hh) for columns 4 c4 .. 4 c4 + 3, in split
// order: returns the bf16 ctx values (packed) and writes them to ctx when it is given;
// c4 == 0 also writes the head's LSE.
// Chunks c0, c0 + cstep, ... of 8 splits (splits 8 c .. 8 c + 7 below S), in that order:
// M is their running max, tot and acc their weighted sums relative to M.  pl and po point at
// split 0's LSE and partial columns of one (unit, head).
template <int DL>
__device__ __forceinline__ void merge_span(const float* pl, const bf16* po, int S, int c0, int cstep, float& M,
                                           float& tot, float (&acc)[4]) {
  M = -INFINITY;
  tot = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = 0.f;
  for (int s0 = 8 * c0; s0 < S; s0 += 8 * cstep) {
    float ls[8];
    u32x2 ov[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int sj = min(s0 + j, S - 1);
      ls[j] = pl[sj * 16];
      ov[j] = ldg8(po + (int64_t)sj * 16 * DL);
    }
    float mc = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ls[j] = s0 + j < S ? ls[j] : -INFINITY;
      mc = fmaxf(mc, ls[j]);
    }
    const float m_new = fmaxf(M, mc);
    const float mu = m_new == -INFINITY ? 0.f : m_new;
    const float a = M == -INFINITY ? 0.f : fast_exp2(M - mu);  // the running sums are 0 while M is -inf
    tot *= a;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= a;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float ws = fast_exp2(ls[j] - mu);  // 0 for masked and empty splits
      tot += ws;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        acc[2 * e] += ws * lo_bf16(ov[j][e]);
        acc[2 * e + 1] += ws * hi_bf16(ov[j][e]);
      }
    }
    M = m_new;
  }
}

template <int DL>
__device__ __forceinline__ u32x2 merge_c4(const DecParams& p, int b, int hh, int c4) {
  const int64_t unit = (int64_t)b * p.n_hg + (hh >> 4);
  const int hr = hh & 15;
  const float* pl = p.part_lse + unit * p.S * 16 + hr;
  const bf16* po = p.part_o + (unit * p.S * 16 + hr) * DL + 4 * c4;
  float M, tot, acc[4];
  merge_span<DL>(pl, po, p.S, 0, 1, M, tot, acc);
  const float inv = tot > 0.f ? 1.f / tot : 0.f;
  const u32x2 v{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
  if (p.ctx) stg8(p.ctx + (int64_t)b * p.ctx_sb + (int64_t)hh * p.ctx_sh + 4 * c4, v);
  if (c4 == 0) p.lse[(int64_t)b * p.H + hh] = tot > 0.f ? (M + fast_log2(tot)) * kLn2 : -INFINITY;
  return v;
}

template <int DL>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecParams p) {
  constexpr int C4 = DL / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = (int64_t)p.B * p.n_hg * 16 * C4;
  if (idx >= n) return;
  const int c4 = (int)(idx % C4);
  const int64_t uh = idx / C4;  // unit * 16 + hr
  const int hr = (int)(uh & 15);
  const int64_t unit = uh >> 4;
  const int b = (int)(unit / p.n_hg);
  const int hh = (int)(unit - (int64_t)b * p.n_hg) * 16 + hr;
  if (hh >= p.H) return;
  merge_c4<DL>(p, b, hh, c4);
}

// Whether the split merge runs as decode_merge_wide_kernel.  Otherwise one thread per output
// quad walks the splits 8 at a time (ceil(S / 8) dependent memory round trips), in
// decode_merge_kernel or, with W_UV, inside decode_merge_uv_kernel (no launch of its own).  The
// rule is the same with and without W_UV, so mla_decode_out's ctx stays mla_decode's bit for bit.
// Measured (graph-timed calls, d_latent 512, 16 heads), up to 32 splits the in-thread walk wins:
// with W_UV 17.5 -> 16.1 us at B = 1 over 1000 of 1536 positions (12 splits) and 26.0 -> 22.5 us
// at B = 16 over 2000 (15 splits); without it 22.8 -> 20.1 us at B = 16 and 19.5 -> 18.3 us at
// B = 8 over 3000 (23 splits), while at B <= 4 the few merge workgroups lose 0.3-0.6 us to the
// wide kernel.  Past 32 splits (one sequence over long contexts: up to 256) the wide merge runs.
__host__ __device__ __forceinline__ bool dec_wide(int S) { return S > 32; }

// The merge for many splits.  One thread per output quad walks its splits 8 at a time,
// a memory round trip per 8 (at B = 1 the automatic 256 splits took 22.7 us, as long as the
// main kernel over 65536 positions).  Here a workgroup owns kWideQ quads of one (b, head)
// and spreads the chunks of 8 splits over kWideG thread groups (group k takes chunks k,
// k + kWideG, ...); the groups' maxima and sums then meet through LDS, added in group order
// (deterministic).
constexpr int kWideQ = 8, kWideG = 32;
static_assert(kWideQ * kWideG == 256, "one thread per (quad, group)");

template <int DL>
__global__ __launch_bounds__(256) void decode_merge_wide_kernel(DecParams p) {
  constexpr int C4 = DL / 4;
  constexpr int NCB = C4 / kWideQ;  // quad blocks per head
  static_assert(C4 % kWideQ == 0, "whole quad blocks");
  __shared__ float gm[kWideG][kWideQ], gt[kWideG][kWideQ];
  __shared__ f32x4 ga[kWideG][kWideQ];
  const int qd = threadIdx.x % kWideQ, k = threadIdx.x / kWideQ;
  const int64_t blk = blockIdx.x;
  const int cb = (int)(blk % NCB);
  const int64_t uh = blk / NCB;  // unit * 16 + hr
  const int hr = (int)(uh & 15);
  const int64_t unit = uh >> 4;
  const int b = (int)(unit / p.n_hg);
  const int hh = (int)(unit - (int64_t)b * p.n_hg) * 16 + hr;
  if (hh >= p.H) return;  // the whole workgroup (hh is the workgroup's)
  const int c4 = cb * kWideQ + qd;
  float M, tot, acc[4];
  merge_span<DL>(p.part_lse + unit * p.S * 16 + hr, p.part_o + (unit * p.S * 16 + hr) * DL + 4 * c4, p.S, k,
                 kWideG, M, tot, acc);
  gm[k][qd] = M;
  gt[k][qd] = tot;
  ga[k][qd] = f32x4{acc[0], acc[1], acc[2], acc[3]};
  __syncthreads();
  if (k != 0) return;
  const int ng = min(kWideG, (p.S + 7) / 8);  // groups that took a chunk
  float Mx = -INFINITY;
  for (int g = 0; g < ng; ++g) Mx = fmaxf(Mx, gm[g][qd]);
  const float mu = Mx == -INFINITY ? 0.f : Mx;
  float T = 0.f;
  f32x4 A = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < ng; ++g) {
    const float wg = gm[g][qd] == -INFINITY ? 0.f : fast_exp2(gm[g][qd] - mu);  // empty groups weigh 0
    T += wg * gt[g][qd];
    A += wg * ga[g][qd];
  }
  const float inv = T > 0.f ? 1.f / T : 0.f;
  if (p.ctx)
    stg8(p.ctx + (int64_t)b * p.ctx_sb + (int64_t)hh * p.ctx_sh + 4 * c4,
         u32x2{pack_bf16x2(A[0] * inv, A[1] * inv), pack_bf16x2(A[2] * inv, A[3] * inv)});
  if (c4 == 0) p.lse[(int64_t)b * p.H + hh] = T > 0.f ? (Mx + fast_log2(T)) * kLn2 : -INFINITY;
}

// The merge with the W_UV product (transformer.py:286-291):
//   out[b][h][d] = sum_c bf16(ctx[b][h][c]) W_UV[h][d][c],  d < 128.
// A workgroup owns one head, kUvBB sequences and one half of the 128 output rows d:
//   * its 64 rows of W_UV[h] (64 x DL bf16) go to LDS by direct-to-LDS loads of 1 KiB runs,
//     chunk c of row r stored at position c ^ (r mod 16);
//   * meanwhile it merges the kUvBB sequences' ctx rows (or, with one split, reads back what
//     the main kernel wrote) into an LDS tile of 16 rows (the rest zero), with the same swizzle;
//   * wave w then computes C^T [16 d][16 b] = W_UV[16 w + .., :] ctx^T on
//     v_mfma_f32_16x16x32_bf16 (DL / 32 k-steps): a lane holds 4 consecutive d of one sequence.
// Every output has one writer (deterministic).
constexpr int kUvBB = 4;   // sequences per workgroup
constexpr int kUvRows = 64;  // output rows d per workgroup (two workgroups per 128)

struct UvParams {
  const bf16* w;
  bf16* out;
  const bf16* ctx_src;  // one split: the ctx the main kernel wrote; otherwise null
  int64_t w_sh, w_sd, out_sb, out_sh;
};

template <int DL>
__global__ __launch_bounds__(256) void decode_merge_uv_kernel(DecParams p, UvParams u) {
  constexpr int C4 = DL / 4;
  constexpr int RC = DL / 8;                    // 16-byte chunks per row
  constexpr int SWM = RC < 16 ? RC - 1 : 15;    // swizzle mask (rows of fewer than 16 chunks)
  extern __shared__ __attribute__((aligned(1024))) unsigned char wl[];  // [kUvRows][DL] bf16, swizzled
  __shared__ __attribute__((aligned(16))) unsigned char cs[16 * DL * 2];  // ctx rows [16][DL], swizzled
  const int h = blockIdx.x % p.H;
  const int rest = blockIdx.x / p.H;
  const int dh = rest & 1;                      // which half of the output rows
  const int b0 = (rest >> 1) * kUvBB;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // W_UV[h] rows kUvRows dh .. + kUvRows: the descriptor covers exactly them
  {
    const bf16* wb = u.w + (int64_t)h * u.w_sh + (int64_t)(kUvRows * dh) * u.w_sd;
    const buf_rsrc r = make_rsrc(wb, rows_bytes(kUvRows, u.w_sd, DL * 2));
    const uint32_t base = lds_addr(wl);
    constexpr int NI = kUvRows * RC / 64;  // 1 KiB loads
    for (int i = w; i < NI; i += 4) {
      const int fq = 64 * i + lane;
      const int row = fq / RC, pos = fq - row * RC;
      dma16(r, (uint32_t)(row * u.w_sd * 2 + ((pos ^ (row & SWM)) << 4)), base + 1024u * (uint32_t)i);
    }
  }
  // ctx rows of the kUvBB sequences (rows kUvBB .. 15 of the tile are zero)
  for (int i = threadIdx.x; i < (16 - kUvBB) * RC; i += 256)
    sts16(cs + (kUvBB * RC + i) * 16, u32x4{0u, 0u, 0u, 0u});
  for (int i = threadIdx.x; i < kUvBB * C4; i += 256) {
    const int sq = i / C4, c4 = i - sq * C4;
    const int b = b0 + sq;
    u32x2 v{0u, 0u};
    if (b < p.B) {
      if (u.ctx_src) v = ldg8(u.ctx_src + (int64_t)b * p.ctx_sb + (int64_t)h * p.ctx_sh + 4 * c4);
      else v = merge_c4<DL>(p, b, h, c4);
    }
    const int c = c4 >> 1;
    sts8(cs + sq * DL * 2 + ((c ^ (sq & SWM)) << 4) + (c4 & 1) * 8, v);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's W_UV loads have landed
  __syncthreads();

  // C^T [16 d][16 b]: wave w takes rows d = 16 w + (l % 16); k-step ks covers chunks 4 ks + l / 16
  const int l16 = lane & 15, q = lane >> 4;
  const int dr = 16 * w + l16;  // this lane's W_UV row within the workgroup's 64
  f32x4 acc = f32x4{};
#pragma unroll
  for (int ks = 0; ks < DL / 32; ++ks) {
    const int c = 4 * ks + q;
    const bf16x8 a = as_bf16x8(lds16(wl + dr * DL * 2 + ((c ^ (dr & SWM)) << 4)));
    const bf16x8 bv = as_bf16x8(lds16(cs + l16 * DL * 2 + ((c ^ (l16 & SWM)) << 4)));
    acc = mfma16(a, bv, acc);
  }
  // lane (l16, q): sequence b0 + l16, rows d = kUvRows dh + 16 w + 4 q + [0, 4)
  const int b = b0 + l16;
  if (l16 < kUvBB && b < p.B)
    stg8(u.out + (int64_t)b * u.out_sb + (int64_t)h * u.out_sh + kUvRows * dh + 16 * w + 4 * q,
         u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])});
}

// W_UK absorption of the decode queries (transformer.py:252-254):
//   q_lat[b][h][c] = sum_d q_nope[b][h][d] W_UK[h][d][c].
// A workgroup owns one head and kAbBB sequences, so W_UK[h] is read once for them.  Wave w
// takes rows d in [w DN/4, (w + 1) DN/4) and lane l the columns [8 l, 8 l + 8) (d_latent
// <= 512): all of the wave's row loads are issued first, the q values come from LDS
// (broadcast), and the four waves' partial sums are added through LDS in wave order.
constexpr int kAbBB = 2;

struct AbsorbParams {
  const bf16* q;
  const bf16* w;
  bf16* out;
  int B, H, DL;
  int64_t q_sb, q_sh, w_sh, w_sd, o_sb, o_sh;
};

template <int DN>
__global__ __launch_bounds__(256) void absorb_q_kernel(AbsorbParams a) {
  constexpr int RW = DN / 4;
  __shared__ float qs[kAbBB][DN];
  __shared__ f32x4 part[4][kAbBB][128];  // [wave][sequence][2 lane + half]
  const int h = blockIdx.x % a.H;
  const int b0 = (blockIdx.x / a.H) * kAbBB;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool col_ok = 8 * lane < a.DL;
  const bf16* wr = a.w + (int64_t)h * a.w_sh + (int64_t)(w * RW) * a.w_sd + 8 * lane;
  u32x4 wv[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) wv[r] = col_ok ? ldg16(wr + (int64_t)r * a.w_sd) : u32x4{0u, 0u, 0u, 0u};
  for (int i = threadIdx.x; i < kAbBB * DN; i += 256) {
    const int sq = i / DN, d = i - sq * DN;
    const int b = b0 + sq;
    qs[sq][d] = b < a.B ? (float)a.q[(int64_t)b * a.q_sb + (int64_t)h * a.q_sh + d] : 0.f;
  }
  __syncthreads();
  float acc[kAbBB][8];
#pragma unroll
  for (int sq = 0; sq < kAbBB; ++sq)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[sq][e] = 0.f;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    float wf[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wf[2 * e] = lo_bf16(wv[r][e]);
      wf[2 * e + 1] = hi_bf16(wv[r][e]);
    }
#pragma unroll
    for (int sq = 0; sq < kAbBB; ++sq) {
      const float qd = qs[sq][w * RW + r];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[sq][e] = __builtin_fmaf(qd, wf[e], acc[sq][e]);
    }
  }
#pragma unroll
  for (int sq = 0; sq < kAbBB; ++sq) {
    part[w][sq][2 * lane] = f32x4{acc[sq][0], acc[sq][1], acc[sq][2], acc[sq][3]};
    part[w][sq][2 * lane + 1] = f32x4{acc[sq][4], acc[sq][5], acc[sq][6], acc[sq][7]};
  }
  __syncthreads();
  static_assert(kAbBB * 128 == 256, "one thread per output quad of the workgroup");
  const int sq = threadIdx.x >> 7, qd = threadIdx.x & 127;
  const f32x4 t = ((part[0][sq][qd] + part[1][sq][qd]) + part[2][sq][qd]) + part[3][sq][qd];
  const int b = b0 + sq, c = 4 * qd;
  if (b < a.B && c < a.DL)
    stg8(a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + c, u32x2{pack_bf16x2(t[0], t[1]), pack_bf16x2(t[2], t[3])});
}

static int pick_splits(const mla_decode_args* a, int n_hg) {
  const int64_t max_s = std::max<int64_t>(1, a->L / 128);  // >= 2 tiles per wave
  if (a->num_splits > 0) return (int)std::min<int64_t>(a->num_splits, std::max<int64_t>((a->L + 15) / 16, 1));
  const int64_t units = a->B * n_hg;
  int64_t s = (256 + units - 1) / units;  // one workgroup per CU on 256 CUs
  return (int)std::max<int64_t>(1, std::min<int64_t>(s, max_s));
}

struct DecLayout {
  int n_hg, S, chunk;
  size_t off_o, total;  // workspace: part_lse at 0, part_o at off_o
};

static DecLayout dec_layout(const mla_decode_args* a) {
  DecLayout d;
  d.n_hg = (int)((a->H + 15) / 16);
  int S = pick_splits(a, d.n_hg);
  const int64_t per = (a->L + S - 1) / S;
  d.chunk = (int)(((per + 63) / 64) * 64);  // whole 16-token tiles for each of the 4 waves
  S = (int)((a->L + d.chunk - 1) / d.chunk);
  d.S = S < 1 ? 1 : S;
  const size_t units = (size_t)a->B * d.n_hg;
  if (d.S > 1) {
    d.off_o = ((units * d.S * 16 * sizeof(float)) + 255) & ~(size_t)255;
    d.total = d.off_o + units * d.S * 16 * (size_t)a->d_latent * sizeof(uint16_t);
  } else {
    d.off_o = d.total = 0;
  }
  return d;
}

template <int DL, bool SHARED>
static void launch_dec(const DecParams& prm, const UvParams* uv, hipStream_t s) {
  const unsigned n = (unsigned)(prm.B * prm.n_hg * prm.S);
  decode_kernel<DL, SHARED><<<dim3(n), dim3(256), 0, s>>>(prm);
  // many splits: the wide merge (into ctx and lse; with W_UV the product then reads ctx back)
  const bool wide = dec_wide(prm.S);
  if (wide)
    decode_merge_wide_kernel<DL>
        <<<dim3((unsigned)(prm.B * prm.n_hg * 16 * (DL / 4 / kWideQ))), dim3(256), 0, s>>>(prm);
  if (uv) {
    const unsigned nu = (unsigned)(prm.H * 2 * ((prm.B + kUvBB - 1) / kUvBB));
    decode_merge_uv_kernel<DL><<<dim3(nu), dim3(256), (size_t)kUvRows * DL * 2, s>>>(prm, *uv);
  } else if (prm.S > 1 && !wide) {
    const int64_t threads = (int64_t)prm.B * prm.n_hg * 16 * (DL / 4);
    decode_merge_kernel<DL><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s>>>(prm);
  }
}

template <bool SHARED>
static int dispatch_dec(int DL, const DecParams& prm, const UvParams* uv, hipStream_t s, const char* op) {
  switch (DL) {
    case 64: launch_dec<64, SHARED>(prm, uv, s); break;
    case 128: launch_dec<128, SHARED>(prm, uv, s); break;
    case 256: launch_dec<256, SHARED>(prm, uv, s); break;
    case 384: launch_dec<384, SHARED>(prm, uv, s); break;
    case 512: launch_dec<512, SHARED>(prm, uv, s); break;
    default: set_error("%s: d_latent %d not built", op, DL); return MLA_ERR_UNSUPPORTED;
  }
  return launch_status(op);
}

// Validates the decode arguments and fills the kernel parameters; `*empty` is set when
// there is nothing to launch (B == 0 or H == 0).  ctx may be null only if ctx_optional.
static int dec_setup(const mla_decode_args* a, const char* op, bool ctx_optional, DecLayout& d, DecParams& prm,
                     bool* empty) {
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_TRY(check_scale(op, a->scale));
  MLA_CHECK(a->d_rope == 64, MLA_ERR_UNSUPPORTED, "%s: d_rope must be 64", op);
  MLA_CHECK(a->d_latent == 64 || a->d_latent == 128 || a->d_latent == 256 || a->d_latent == 384 ||
                a->d_latent == 512,
            MLA_ERR_UNSUPPORTED, "%s: d_latent %lld not built (64, 128, 256, 384, 512)", op, (long long)a->d_latent);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->L >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->B < 65536 && a->H < 65536 && a->L < (1ll << 30), MLA_ERR_INVALID_ARG, "%s: size out of range", op);
  *empty = a->B == 0 || a->H == 0;
  if (*empty) return MLA_OK;
  MLA_CHECK(a->L > 0, MLA_ERR_INVALID_ARG, "%s: empty cache (L = 0)", op);
  MLA_CHECK(a->n_k_rope_heads == 1 || a->n_k_rope_heads == a->H, MLA_ERR_INVALID_ARG,
            "%s: n_k_rope_heads must be 1 or H", op);
  MLA_CHECK(a->q_lat && a->q_rope && a->c_kv && a->k_rope && (a->ctx || ctx_optional) && a->lse,
            MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  const void* ptrs[] = {a->q_lat, a->q_rope, a->c_kv, a->k_rope};
  for (const void* q : ptrs) MLA_CHECK(((uintptr_t)q & 15) == 0, MLA_ERR_INVALID_ARG, "%s: inputs must be 16-byte aligned", op);
  const int64_t strides[] = {a->q_lat_sb, a->q_lat_sh, a->q_rope_sb, a->q_rope_sh, a->c_kv_sb,
                             a->c_kv_st,  a->k_rope_sb, a->k_rope_sh, a->k_rope_st};
  for (int64_t st : strides)
    MLA_CHECK(st >= 0 && (st & 7) == 0, MLA_ERR_INVALID_ARG, "%s: strides must be non-negative multiples of 8", op);
  MLA_CHECK(a->n_k_rope_heads != 1 || a->k_rope_sh == 0, MLA_ERR_INVALID_ARG,
            "%s: a shared k_rope head needs head stride 0", op);
  MLA_CHECK(a->ctx_sb >= 0 && a->ctx_sh >= 0, MLA_ERR_INVALID_ARG, "%s: negative ctx strides", op);
  MLA_CHECK(!a->ctx || (((uintptr_t)a->ctx & 7) == 0 && (a->ctx_sb & 3) == 0 && (a->ctx_sh & 3) == 0),
            MLA_ERR_INVALID_ARG, "%s: ctx must be 8-byte aligned with strides multiples of 4", op);

  d = dec_layout(a);
  const int64_t n_wg = a->B * (int64_t)d.n_hg * d.S;
  const int64_t n_merge = (a->B * (int64_t)d.n_hg * 16 * (a->d_latent / 4) + 255) / 256;  // merge blocks
  const int64_t n_wide = dec_wide(d.S) ? a->B * (int64_t)d.n_hg * 16 * (a->d_latent / 4 / kWideQ) : 0;
  MLA_CHECK(n_wg < (1ll << 31) && n_merge < (1ll << 31) && n_wide < (1ll << 31), MLA_ERR_INVALID_ARG,
            "%s: grid too large", op);
  prm.q_lat = (const bf16*)a->q_lat;
  prm.q_rope = (const bf16*)a->q_rope;
  prm.c_kv = (const bf16*)a->c_kv;
  prm.k_rope = (const bf16*)a->k_rope;
  prm.seq_lens = a->seq_lens;
  prm.ctx = (bf16*)a->ctx;
  prm.lse = a->lse;
  // the partials' workspace (checked by the caller; mla_decode_static passes none and points
  // these at its scratch afterwards)
  const bool parts = d.S > 1 && a->workspace != nullptr;
  prm.part_lse = parts ? (float*)a->workspace : nullptr;
  prm.part_o = parts ? (bf16*)((char*)a->workspace + d.off_o) : nullptr;
  prm.B = (int)a->B;
  prm.H = (int)a->H;
  prm.L = (int)a->L;
  prm.S = d.S;
  prm.chunk = d.chunk;
  prm.n_hg = d.n_hg;
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
  return MLA_OK;
}

static int check_workspace(const mla_decode_args* a, size_t need, const char* op) {
  if (need == 0) return MLA_OK;
  MLA_CHECK(a->workspace && a->workspace_bytes >= need, MLA_ERR_WORKSPACE, "%s: workspace of %zu bytes required (got %zu)",
            op, need, a->workspace_bytes);
  MLA_CHECK(((uintptr_t)a->workspace & 255) == 0, MLA_ERR_WORKSPACE, "%s: workspace must be 256-byte aligned", op);
  return MLA_OK;
}

// decode_out workspace: the split partials, then (with no caller ctx) a bf16 ctx scratch
// [B, H, d_latent] where the W_UV product reads back the merged ctx: with one split the main
// kernel writes it, with many splits the wide merge
static size_t dec_out_ctx_off(const DecLayout& d) {
  return dec_wide(d.S) ? (d.total + 255) & ~(size_t)255 : 0;
}
static size_t dec_out_ws(const mla_decode_out_args* a, const DecLayout& d) {
  if (a->dec.ctx || (d.S > 1 && !dec_wide(d.S))) return d.total;
  return dec_out_ctx_off(d) + (size_t)a->dec.B * (size_t)a->dec.H * (size_t)a->dec.d_latent * sizeof(uint16_t);
}

// The split partials of mla_decode_static: one file-scope array per GPU, sized for any
// automatic split count at d_latent <= 512 (at most 2 x 256 (unit, split) workgroups of 16
// rows of bf16 plus their LSEs).  In host code `scratch` names a host-side stand-in, never
// the device memory: its device address is looked up once per device (static_scratch)
// and only that address is handed to kernels.  Every launch writes all the partials it
// reads before reading them, so the array needs no clearing between calls.
constexpr size_t kDecodeStaticScratch = MLA_DECODE_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kDecodeStaticScratch];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The device address of `scratch` on the current device (which must be the stream's).
static int static_scratch(const char* op, void* stream, void** out) {
  int dev = -1;
  MLA_CHECK(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, MLA_ERR_LAUNCH,
            "%s: no current HIP device (or device id above %d)", op, kMaxDevices - 1);
  if (stream) {
    int sdev = -1;
    MLA_CHECK(hipStreamGetDevice((hipStream_t)stream, &sdev) == hipSuccess, MLA_ERR_INVALID_ARG,
              "%s: cannot query the stream's device", op);
    MLA_CHECK(sdev == dev, MLA_ERR_INVALID_ARG, "%s: the stream belongs to device %d but device %d is current", op,
              sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    MLA_CHECK(e == hipSuccess && ptr, MLA_ERR_LAUNCH, "%s: hipGetSymbolAddress of the static scratch failed: %s", op,
              hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MLA_OK;
}

}  // namespace mla

using namespace mla;

// The sizes the decode entry points accept (without their pointer and stride checks), tested
// before the layout's arithmetic: the workspace queries answer 0 for anything else.
static bool dec_sizes_ok(const mla_decode_args* a) {
  if (a->d_rope != 64 ||
      !(a->d_latent == 64 || a->d_latent == 128 || a->d_latent == 256 || a->d_latent == 384 || a->d_latent == 512))
    return false;
  if (a->B <= 0 || a->H <= 0 || a->L <= 0 || a->B >= 65536 || a->H >= 65536 || a->L >= (1ll << 30)) return false;
  const DecLayout d = dec_layout(a);
  return a->B * (int64_t)d.n_hg * d.S < (1ll << 31);
}

extern "C" size_t mla_decode_workspace_bytes(const mla_decode_args* a) {
  if (!a || !dec_sizes_ok(a)) return 0;
  return dec_layout(a).total;
}

extern "C" int mla_decode(const mla_decode_args* a, void* stream) {
  const char* op = "mla_decode";
  DecLayout d;
  DecParams prm;
  bool empty = false;
  MLA_TRY(dec_setup(a, op, false, d, prm, &empty));
  if (empty) return MLA_OK;
  MLA_TRY(check_workspace(a, d.S > 1 ? d.total : 0, op));
  hipStream_t s = (hipStream_t)stream;
  return a->n_k_rope_heads == 1 ? dispatch_dec<true>((int)a->d_latent, prm, nullptr, s, op)
                                : dispatch_dec<false>((int)a->d_latent, prm, nullptr, s, op);
}

extern "C" int mla_decode_static(const mla_decode_args* a, void* stream) {
  const char* op = "mla_decode_static";
  DecLayout d;
  DecParams prm;
  bool empty = false;
  MLA_TRY(dec_setup(a, op, false, d, prm, &empty));
  if (empty) return MLA_OK;
  const size_t need = d.S > 1 ? d.total : 0;
  MLA_CHECK(need <= kDecodeStaticScratch, MLA_ERR_WORKSPACE,
            "%s: %d splits need %zu bytes of partials, above the %zu-byte static scratch (use fewer splits, or "
            "mla_decode with a workspace)",
            op, d.S, need, kDecodeStaticScratch);
  if (need) {
    void* ptr = nullptr;
    MLA_TRY(static_scratch(op, stream, &ptr));
    prm.part_lse = (float*)ptr;
    prm.part_o = (bf16*)((char*)ptr + d.off_o);
  }
  hipStream_t s = (hipStream_t)stream;
  return a->n_k_rope_heads == 1 ? dispatch_dec<true>((int)a->d_latent, prm, nullptr, s, op)
                                : dispatch_dec<false>((int)a->d_latent, prm, nullptr, s, op);
}

extern "C" size_t mla_decode_out_workspace_bytes(const mla_decode_out_args* a) {
  if (!a || !dec_sizes_ok(&a->dec)) return 0;
  return dec_out_ws(a, dec_layout(&a->dec));
}

extern "C" int mla_decode_out(const mla_decode_out_args* a, void* stream) {
  const char* op = "mla_decode_out";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  DecLayout d;
  DecParams prm;
  bool empty = false;
  MLA_TRY(dec_setup(&a->dec, op, true, d, prm, &empty));
  if (empty) return MLA_OK;
  MLA_CHECK(a->d_v == 128, MLA_ERR_UNSUPPORTED, "%s: d_v %lld not built (128)", op, (long long)a->d_v);
  MLA_CHECK(a->w_uv && a->out, MLA_ERR_INVALID_ARG, "%s: null w_uv or out", op);
  MLA_CHECK(((uintptr_t)a->w_uv & 15) == 0 && a->w_uv_sh >= 0 && (a->w_uv_sh & 7) == 0 &&
                a->w_uv_sd >= a->dec.d_latent && (a->w_uv_sd & 7) == 0,
            MLA_ERR_INVALID_ARG, "%s: w_uv must be 16-byte aligned with strides multiples of 8 (row stride >= d_latent)",
            op);
  MLA_CHECK(((uintptr_t)a->out & 1) == 0 && a->out_sb >= 0 && a->out_sh >= 0, MLA_ERR_INVALID_ARG,
            "%s: bad out pointer or strides", op);
  MLA_CHECK(a->dec.H * 2 * ((a->dec.B + kUvBB - 1) / kUvBB) < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: grid too large",
            op);
  MLA_CHECK(((uintptr_t)a->out & 7) == 0 && (a->out_sb & 3) == 0 && (a->out_sh & 3) == 0, MLA_ERR_INVALID_ARG,
            "%s: out must be 8-byte aligned with strides multiples of 4", op);
  const size_t need = dec_out_ws(a, d);
  MLA_TRY(check_workspace(&a->dec, need, op));
  UvParams uv;
  uv.w = (const bf16*)a->w_uv;
  uv.out = (bf16*)a->out;
  uv.w_sh = a->w_uv_sh;
  uv.w_sd = a->w_uv_sd;
  uv.out_sb = a->out_sb;
  uv.out_sh = a->out_sh;
  uv.ctx_src = nullptr;
  if (d.S == 1 || dec_wide(d.S)) {
    if (!prm.ctx) {  // scratch ctx [B, H, d_latent] in the workspace, past the partials
      prm.ctx = (bf16*)((char*)a->dec.workspace + dec_out_ctx_off(d));
      prm.ctx_sb = a->dec.H * a->dec.d_latent;
      prm.ctx_sh = a->dec.d_latent;
    }
    uv.ctx_src = prm.ctx;
  }
  hipStream_t s = (hipStream_t)stream;
  return a->dec.n_k_rope_heads == 1 ? dispatch_dec<true>((int)a->dec.d_latent, prm, &uv, s, op)
                                    : dispatch_dec<false>((int)a->dec.d_latent, prm, &uv, s, op);
}

extern "C" int mla_absorb_q(const mla_absorb_q_args* a, void* stream) {
  const char* op = "mla_absorb_q";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->B < 65536 && a->H < 65536, MLA_ERR_INVALID_ARG, "%s: size out of range", op);
  MLA_CHECK(a->d_nope == 64 || a->d_nope == 128, MLA_ERR_UNSUPPORTED, "%s: d_nope %lld not built (64, 128)", op,
            (long long)a->d_nope);
  MLA_CHECK(a->d_latent > 0 && a->d_latent <= 512 && a->d_latent % 8 == 0, MLA_ERR_UNSUPPORTED,
            "%s: d_latent %lld must be a multiple of 8 up to 512", op, (long long)a->d_latent);
  if (a->B == 0 || a->H == 0) return MLA_OK;
  MLA_CHECK(a->q_nope && a->w_uk && a->q_lat, MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  MLA_CHECK(((uintptr_t)a->w_uk & 15) == 0 && a->w_uk_sh >= 0 && (a->w_uk_sh & 7) == 0 && a->w_uk_sd >= a->d_latent &&
                (a->w_uk_sd & 7) == 0,
            MLA_ERR_INVALID_ARG, "%s: w_uk must be 16-byte aligned with strides multiples of 8 (row stride >= d_latent)",
            op);
  MLA_CHECK(((uintptr_t)a->q_lat & 7) == 0 && a->out_sb >= 0 && a->out_sh >= 0 && (a->out_sb & 3) == 0 &&
                (a->out_sh & 3) == 0,
            MLA_ERR_INVALID_ARG, "%s: q_lat must be 8-byte aligned with strides multiples of 4", op);
  MLA_CHECK(((uintptr_t)a->q_nope & 1) == 0 && a->q_sb >= 0 && a->q_sh >= 0, MLA_ERR_INVALID_ARG, "%s: bad q_nope", op);
  AbsorbParams p{(const bf16*)a->q_nope, (const bf16*)a->w_uk, (bf16*)a->q_lat, (int)a->B, (int)a->H, (int)a->d_latent,
                 a->q_sb, a->q_sh, a->w_uk_sh, a->w_uk_sd, a->out_sb, a->out_sh};
  const int64_t grid = a->H * ((a->B + kAbBB - 1) / kAbBB);
  MLA_CHECK(grid < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: grid too large", op);
  hipStream_t s = (hipStream_t)stream;
  if (a->d_nope == 128) absorb_q_kernel<128><<<dim3((unsigned)grid), dim3(256), 0, s>>>(p);
  else absorb_q_kernel<64><<<dim3((unsigned)grid), dim3(256), 0, s>>>(p);
  return launch_status(op);
}
