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
// loop walks 64-key tiles staged through LDS: K row-major [64][DQK + 8] and V
// transposed [128][64 + 4] (the transpose is done in registers while staging).
//
// Per 64-key tile and wave:
//   S^T (64 x 32)  = K (64 x DQK) . Q^T (DQK x 32)     2 x DQK/16 MFMA 32x32x16
//   O^T (128 x 32) += V^T (128 x 64) . P^T (64 x 32)   4 x 4     MFMA 32x32x16
// Computing S^T rather than S puts one query row per lane (column of the MFMA
// output), so the running max / sum / rescale of the online softmax are per-lane
// scalars; the row max needs one cross-lane exchange (lanes l and l ^ 32).
// P^T goes straight from the S^T accumulators into the PV MFMA's B operand.
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

template <int DN>
struct FwdCfg {
  static constexpr int DR = 64, DV = 128, DQK = DN + DR;
  static constexpr int BM = 128, BN = 64;
  static constexpr int KS = DQK / 16;        // MFMA k-steps of S^T
  static constexpr int K_LD = DQK + 8;       // LDS row stride (elements) of K: 16-byte pad
  static constexpr int V_LD = DV + 32;       // LDS row stride of V: 64-byte pad (transpose reads)
  static constexpr int K_CH = DQK / 8;       // 16-byte chunks per K row
  static constexpr int K_PER_THREAD = BN * K_CH / 256;
  static constexpr int V_PER_THREAD = BN * (DV / 8) / 256;
  static_assert((BN * K_CH) % 256 == 0 && (BN * DV / 8) % 256 == 0, "tile chunks must divide the workgroup");
};

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

template <int DN>
__global__ __launch_bounds__(256, 2) void prefill_fwd_kernel(FwdParams p) {
  using C = FwdCfg<DN>;
  __shared__ __attribute__((aligned(16))) bf16 Ks[C::BN * C::K_LD];
  __shared__ __attribute__((aligned(16))) bf16 Vs[C::BN * C::V_LD];
  __shared__ int ovf_s[4];

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
  // Tile staging through registers with buffer loads: per-thread byte offsets inside a
  // tile are fixed; each tile gets descriptors based at its first key whose size ends at
  // the last valid key, so rows past Tk read as zero (and are masked).
  constexpr int NKN = C::BN * (DN / 8) / 256, NKR = C::BN * 8 / 256, NV = C::BN * 16 / 256;
  uint32_t off_kn[NKN], off_kr[NKR], off_v[NV];
#pragma unroll
  for (int i = 0; i < NKN; ++i) {
    const int c = tid + 256 * i;
    off_kn[i] = (uint32_t)((c / (DN / 8)) * p.kn_s.t * 2 + (c % (DN / 8)) * 16);
  }
#pragma unroll
  for (int i = 0; i < NKR; ++i) {
    const int c = tid + 256 * i;
    off_kr[i] = (uint32_t)((c >> 3) * p.kr_s.t * 2 + (c & 7) * 16);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = tid + 256 * i;
    off_v[i] = (uint32_t)((c >> 4) * p.v_s.t * 2 + (c & 15) * 16);
  }
  u32x4 kreg[NKN + NKR];
  u32x4 vreg[NV];
  auto load_tile = [&](int kv0) {
    const int nv = min(p.Tk - kv0, C::BN);
    const buf_rsrc rkn = make_rsrc(kn_b + (int64_t)kv0 * p.kn_s.t, rows_bytes(nv, p.kn_s.t, DN * 2));
    const buf_rsrc rkr = make_rsrc(kr_b + (int64_t)kv0 * p.kr_s.t, rows_bytes(nv, p.kr_s.t, 128));
    const buf_rsrc rv = make_rsrc(v_b + (int64_t)kv0 * p.v_s.t, rows_bytes(nv, p.v_s.t, 256));
#pragma unroll
    for (int i = 0; i < NKN; ++i) kreg[i] = bld16(rkn, off_kn[i]);
#pragma unroll
    for (int i = 0; i < NKR; ++i) kreg[NKN + i] = bld16(rkr, off_kr[i]);
#pragma unroll
    for (int i = 0; i < NV; ++i) vreg[i] = bld16(rv, off_v[i]);
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < NKN; ++i) {
      const int c = tid + 256 * i;
      sts16(&Ks[(c / (DN / 8)) * C::K_LD + (c % (DN / 8)) * 8], kreg[i]);
    }
#pragma unroll
    for (int i = 0; i < NKR; ++i) {
      const int c = tid + 256 * i;
      sts16(&Ks[(c >> 3) * C::K_LD + DN + (c & 7) * 8], kreg[NKN + i]);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = tid + 256 * i;
      sts16(&Vs[(c >> 4) * C::V_LD + 8 * (c & 15)], vreg[i]);
    }
  };

  // V^T operand of O^T += V^T P^T through ds_read_b64_tr_b16: the 16-lane group G16 covers
  // dv columns 16 (G16 % 2) + [0, 16) of a 32-row block; lane r of the group addresses row
  // (first key) + r / 4, column + 4 (r % 4).  Byte offsets relative to key kb = 32 jb + 16 s.
  const int l16 = lane & 15;
  const int vt_off = ((l16 >> 2) + 4 * g) * C::V_LD * 2 + (16 * ((lane >> 4) & 1) + 4 * (l16 & 3)) * 2;

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

  f32x16 oacc[4];
  float m_run, l_run;  // log2-domain reference max of this lane's row; its share of the row sum

  // Tile loop.  Fast form (SAFE = false): the reference max is the first tile's row max
  // (key 0 is visible to every row) and never moves, so later tiles need no max, no
  // rescale and no branch on the scores.  p = 2^(s - m) stays finite unless a later score
  // exceeds the first tile's max by more than ~127 (log2); the workgroup then votes and
  // recomputes the q-tile with the safe form, which moves the reference max lazily (when it
  // grows by more than kFwdRescale) and rescales O and l.
  // Tiles [1, n_hot) are fully visible to every row of the workgroup and have a successor
  // in this q-tile: they run a branch-free body (no mask, no max, unconditional prefetch)
  // that the compiler can schedule as one block.
  int n_full = p.Tk / C::BN;
  if (p.causal) n_full = min(n_full, (q0 + q_off + 1) / C::BN);
  const int n_hot = min(n_full, n_tiles - 1);

  auto run_tiles = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) oacc[mb] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;

    auto tile = [&](int j, auto general_tag) {
      constexpr bool GEN = decltype(general_tag)::value;
      const int kv0 = j * C::BN;
      __syncthreads();
      store_tile();
      __syncthreads();
      if (!GEN || j + 1 < n_tiles) {
        load_tile(kv0 + C::BN);
      } else if (item + 1 < n_items) {
        load_tile(0);  // the next q-tile of this (b, h) starts at key 0
      }
      if (GEN && kv0 > wave_last) return;  // every key of the tile is masked for this wave

      f32x16 sacc[2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        sacc[jb] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
          const bf16x8 a = as_bf16x8(lds16(&Ks[(32 * jb + l32) * C::K_LD + 16 * ks + 8 * g]));
          sacc[jb] = mfma32(a, qf[ks], sacc[jb]);
        }
      }

      if (GEN) {
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
      // 32 jb + 16 s + 8 (e / 4) + 4 g + e % 4, matching the S^T accumulator rows
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const char* vb = reinterpret_cast<const char*>(Vs) + (32 * jb + 16 * s) * C::V_LD * 2 + vt_off;
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) {
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + 64 * mb));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + 64 * mb + 8 * C::V_LD * 2));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            oacc[mb] = mfma32(as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]}), pb[jb][s], oacc[mb]);
          }
        }
      }
    };

    if (SAFE) {
      for (int j = 0; j < n_tiles; ++j) tile(j, std::true_type{});
    } else {
      if (n_tiles > 0) tile(0, std::true_type{});
      for (int j = 1; j < n_hot; ++j) tile(j, std::false_type{});
      for (int j = max(1, n_hot); j < n_tiles; ++j) tile(j, std::true_type{});
    }
  };

  if (item == 0) load_tile(0);  // later items: prefetched during the previous one
  run_tiles(std::false_type{});
  {
    // workgroup vote: did any row's sum leave the finite range of the fixed reference?
    const float lt = l_run + wave_shfl_xor(l_run, 32);
    const bool any_bad = __any(!(lt <= kFwdSumLimit));  // a wave-wide vote: every lane takes part
    if (lane == 0) ovf_s[w] = any_bad ? 1 : 0;
    __syncthreads();
    const bool redo = (ovf_s[0] | ovf_s[1] | ovf_s[2] | ovf_s[3]) != 0;
    __syncthreads();  // ovf_s is rewritten by the next vote
    if (redo) {
      load_tile(0);
      run_tiles(std::true_type{});
    }
  }

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
