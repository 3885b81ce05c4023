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
  static constexpr int K_LD = DQK + 8;       // LDS row stride (elements) of K
  static constexpr int VT_LD = BN + 4;       // LDS row stride of V^T
  static constexpr int K_CHUNKS = BN * DQK / 8;             // 16-byte chunks per K tile
  static constexpr int K_PER_THREAD = K_CHUNKS / 256;
  static constexpr int LDS_K = BN * K_LD;                   // elements
  static constexpr int LDS_VT = DV * VT_LD;
  static_assert(K_CHUNKS % 256 == 0, "K tile chunks must divide the workgroup");
};

// Maps the linear workgroup id to (b, h, q-tile).  Workgroups are dispatched
// round-robin over the 8 XCDs (id % 8); renumbering so each XCD receives a
// contiguous range of tiles keeps the K/V of a (b, h) in that XCD's L2.  Inside a
// (b, h) the q-tiles run longest-first (causal work grows with the tile index).
__device__ __forceinline__ void fwd_tile_coords(const FwdParams& p, int& b, int& h, int& qt) {
  const int n = gridDim.x;
  int id = blockIdx.x;
  if ((n & 7) == 0) id = (id & 7) * (n >> 3) + (id >> 3);
  const int bh = id / p.n_qt;
  const int r = id - bh * p.n_qt;
  qt = p.causal ? (p.n_qt - 1 - r) : r;
  b = bh / p.H;
  h = bh - b * p.H;
}

template <int DN>
__global__ __launch_bounds__(256, 2) void prefill_fwd_kernel(FwdParams p) {
  using C = FwdCfg<DN>;
  __shared__ __attribute__((aligned(16))) bf16 Ks[C::LDS_K];
  __shared__ __attribute__((aligned(16))) bf16 Vt[C::LDS_VT];

  int b, h, qt;
  fwd_tile_coords(p, b, h, qt);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int q0 = qt * C::BM;
  const int q_row = q0 + 32 * w + l32;              // this lane's query
  const int q_ld = q_row < p.Tq ? q_row : p.Tq - 1;  // clamped row for loads

  // ---- Q fragment (B operand of S^T = K Q^T): dims 16 ks + 8 g + [0, 8)
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

  // ---- key range
  int kv_end = p.Tk;
  if (p.causal) {
    const int64_t lim = (int64_t)q0 + C::BM + p.q_offset;  // exclusive bound for the tile's last row
    if (lim < kv_end) kv_end = lim < 0 ? 0 : (int)lim;
  }
  const int n_tiles = (kv_end + C::BN - 1) / C::BN;

  const bf16* kn_b = p.kn + (int64_t)b * p.kn_s.b + (int64_t)h * p.kn_s.h;
  const bf16* kr_b = p.kr + (int64_t)b * p.kr_s.b + (int64_t)h * p.kr_s.h;
  const bf16* v_b = p.v + (int64_t)b * p.v_s.b + (int64_t)h * p.v_s.h;

  // staging registers for the next tile
  u32x4 kreg[C::K_PER_THREAD];
  u32x4 vreg[4];
  const int v_dc = tid & 15;  // 8-wide d chunk
  const int v_kg = tid >> 4;  // group of 4 keys

  auto load_tile = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < C::K_PER_THREAD; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (C::DQK / 8);
      const int col = (c - row * (C::DQK / 8)) * 8;
      int kv = kv0 + row;
      kv = kv < p.Tk ? kv : p.Tk - 1;
      kreg[i] = col < DN ? ldg16(kn_b + (int64_t)kv * p.kn_s.t + col)
                         : ldg16(kr_b + (int64_t)kv * p.kr_s.t + (col - DN));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int kv = kv0 + 4 * v_kg + r;
      kv = kv < p.Tk ? kv : p.Tk - 1;
      vreg[r] = ldg16(v_b + (int64_t)kv * p.v_s.t + 8 * v_dc);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < C::K_PER_THREAD; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (C::DQK / 8);
      const int col = (c - row * (C::DQK / 8)) * 8;
      sts16(&Ks[row * C::K_LD + col], kreg[i]);
    }
    u32x2 tr[8];
    transpose4x8(vreg, tr);
#pragma unroll
    for (int c = 0; c < 8; ++c) sts8(&Vt[(8 * v_dc + c) * C::VT_LD + 4 * v_kg], tr[c]);
  };

  f32x16 oacc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) oacc[mb] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  if (n_tiles > 0) load_tile(0);
  for (int j = 0; j < n_tiles; ++j) {
    const int kv0 = j * C::BN;
    __syncthreads();
    store_tile();
    __syncthreads();
    if (j + 1 < n_tiles) load_tile(kv0 + C::BN);

    // The body is branch-free: the mask is always applied and a tile this wave's rows
    // cannot see yields p = 0, alpha = 1.  Control flow here makes the compiler move the
    // O accumulators between register files every iteration.
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

    // scale into the log2 domain and mask
    float mloc = -INFINITY;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = sacc[jb][r] * p.scale_log2;
        {
          const int kv = kv0 + 32 * jb + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = kv < p.Tk && (!p.causal || (int64_t)kv <= (int64_t)q_row + p.q_offset);
          x = ok ? x : -INFINITY;
        }
        sacc[jb][r] = x;
        mloc = fmaxf(mloc, x);
      }
    }
    mloc = fmaxf(mloc, wave_shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;

    float lsum = 0.f;
    bf16x8 pb[2][2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        u32x4 pk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = fast_exp2(sacc[jb][8 * s + 2 * e] - m_use);
          const float p1 = fast_exp2(sacc[jb][8 * s + 2 * e + 1] - m_use);
          lsum += p0 + p1;
          pk[e] = pack_bf16x2(p0, p1);
        }
        pb[jb][s] = as_bf16x8(pk);
      }
    }
    l_run = l_run * alpha + lsum;

#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      oacc[mb] *= alpha;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16* vp = &Vt[(32 * mb + l32) * C::VT_LD + 32 * jb + 16 * s + 4 * g];
          const u32x2 lo = lds8(vp);
          const u32x2 hi = lds8(vp + 8);
          const bf16x8 a = as_bf16x8(u32x4{lo[0], lo[1], hi[0], hi[1]});
          oacc[mb] = mfma32(a, pb[jb][s], oacc[mb]);
        }
      }
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
}

template <int DN>
static int launch_fwd(const FwdParams& prm, hipStream_t s) {
  const int64_t n = (int64_t)prm.B * prm.H * prm.n_qt;
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
