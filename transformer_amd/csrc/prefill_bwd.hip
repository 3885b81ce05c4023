// Backward of the causal MLA prefill attention (gfx950): dQ, dK, dV.
//
// Given dO, O and the forward's LSE (natural log), with P = exp(S - LSE):
//   D   = rowsum(dO o O)                     (bwd_rowdot_kernel)
//   dV  = P^T dO,    dP = dO V^T,  dS = P o (dP - D)
//   dK  = dS^T Q * scale                     (bwd_dkdv_kernel: one key tile per workgroup)
//   dQ  = dS K * scale                       (bwd_dq_kernel:   one query tile per workgroup)
// which is the autograd backward of SDPA at transformer.py:314 (recomputed under
// activation checkpointing, :330-335).  dK and dQ are produced by separate kernels
// so every output element is written by exactly one workgroup: no atomics, and the
// result is bitwise reproducible.  A shared k_rope head (stride 0 over heads) gets
// sum_h dk_rope[h], accumulated in fp32 per head and reduced in head order
// (bwd_dkrope_reduce_kernel).
//
// MFMA layout (v_mfma_f32_32x32x16_bf16, see mla_common.h):
//   dK/dV kernel, wave = 32 keys, loop over 32-query tiles staged in LDS as Q, Q^T,
//   dO, dO^T (the transposes are made in registers while staging):
//     S  (32q x 32k) = Q . K^T        A = Q rows (LDS),  B = K rows (registers)
//     dP (32q x 32k) = dO . V^T       A = dO rows (LDS), B = V rows (registers)
//       -> lanes own a key column, registers run over queries, so P^T and dS^T
//          feed the next products' A operand directly:
//     dV (32k x 128) += P^T . dO      B = dO^T (LDS)
//     dK (32k x DQK) += dS^T . Q      B = Q^T  (LDS)
//   dQ kernel, wave = 32 queries, loop over 64-key tiles staged as K, K^T, V:
//     S^T (64k x 32q) = K . Q^T,  dP^T = V . dO^T   (lanes own a query)
//     dQ^T (DQK x 32q) += K^T . dS^T
#include "mla_common.h"

namespace mla {

struct BwdParams {
  const bf16 *dout, *qn, *qr, *kn, *kr, *v, *o;
  const float* lse;
  bf16 *dqn, *dqr, *dkn, *dkr, *dv;
  float* dsum;     // D [B][H][Tq]
  float* dkr_ws;   // [B][Tk][H][64] fp32 per-head dk_rope (shared k_rope only)
  int B, H, Tq, Tk;
  int shared_rope;
  mla_strides do_s, qn_s, qr_s, kn_s, kr_s, v_s, o_s;
  mla_strides dqn_s, dqr_s, dkn_s, dkr_s, dv_s;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
  int causal;
  int64_t q_offset;
};

// ---------------------------------------------------------------- D = rowsum(dO o O)
__global__ __launch_bounds__(256) void bwd_rowdot_kernel(BwdParams p) {
  // 16 lanes per (b, q, h) row of 128 values
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int part = threadIdx.x & 15;
  const int64_t n_rows = (int64_t)p.B * p.Tq * p.H;
  float acc = 0.f;
  int64_t b = 0, q = 0, h = 0;
  if (row < n_rows) {
    h = row % p.H;
    const int64_t bq = row / p.H;
    q = bq % p.Tq;
    b = bq / p.Tq;
    const u32x4 a = ldg16(p.dout + b * p.do_s.b + q * p.do_s.t + h * p.do_s.h + 8 * part);
    const u32x4 c = ldg16(p.o + b * p.o_s.b + q * p.o_s.t + h * p.o_s.h + 8 * part);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc += lo_bf16(a[i]) * lo_bf16(c[i]) + hi_bf16(a[i]) * hi_bf16(c[i]);
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) acc += wave_shfl_xor(acc, m);
  if (row < n_rows && part == 0) p.dsum[(b * p.H + h) * p.Tq + q] = acc;
}

// Stage a [ROWS][COLS] bf16 tile of a nope++rope split operand (COLS = DN + 64, or a
// plain operand with DN = COLS) into LDS, row-major and/or transposed.  Work unit: a
// block of 4 rows x 8 columns (four 16-byte loads), transposed in registers.
template <int ROWS, int COLS, int DN, bool ROWMAJ, bool TRANS>
struct Stager {
  static constexpr int CB = COLS / 8;
  static constexpr int NBLK = (ROWS / 4) * CB;
  static constexpr int PER = (NBLK + 255) / 256;
  u32x4 reg[PER][4];

  __device__ void load(int tid, const bf16* pn, int64_t sn, const bf16* pr, int64_t sr, int r0, int nrows) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = tid + 256 * i;
      if (NBLK % 256 != 0 && blk >= NBLK) break;
      const int rg = blk / CB;
      const int col = (blk - rg * CB) * 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row = r0 + 4 * rg + r;
        row = row < nrows ? row : nrows - 1;
        reg[i][r] = col < DN ? ldg16(pn + (int64_t)row * sn + col) : ldg16(pr + (int64_t)row * sr + (col - DN));
      }
    }
  }
  __device__ void store(int tid, bf16* row_lds, int row_ld, bf16* t_lds, int t_ld) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = tid + 256 * i;
      if (NBLK % 256 != 0 && blk >= NBLK) break;
      const int rg = blk / CB;
      const int col = (blk - rg * CB) * 8;
      if (ROWMAJ) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sts16(&row_lds[(4 * rg + r) * row_ld + col], reg[i][r]);
      }
      if (TRANS) {
        u32x2 tr[8];
        transpose4x8(reg[i], tr);
#pragma unroll
        for (int c = 0; c < 8; ++c) sts8(&t_lds[(col + c) * t_ld + 4 * rg], tr[c]);
      }
    }
  }
};

template <int DN>
struct BwdCfg {
  static constexpr int DR = 64, DV = 128, DQK = DN + DR;
  static constexpr int KS = DQK / 16;  // k-steps over the QK dims
  static constexpr int NDQK = DQK / 32;  // 32-wide blocks of the QK dims
  // dK/dV kernel
  static constexpr int BKV = 128, BQ = 32;
  static constexpr int QB = BQ / 32;  // 32-query blocks per tile
  static constexpr int Q_LD = DQK + 8, QT_LD = BQ + 4, DO_LD = DV + 8, DOT_LD = BQ + 4;
  // dQ kernel
  static constexpr int BQQ = 128, BK = 64;
  static constexpr int K_LD = DQK + 8, KT_LD = BK + 4, V_LD = DV + 8;
};

__device__ __forceinline__ bf16x8 lds_pair8(const bf16* p) {
  const u32x2 lo = lds8(p);
  const u32x2 hi = lds8(p + 8);
  return as_bf16x8(u32x4{lo[0], lo[1], hi[0], hi[1]});
}

// ---------------------------------------------------------------- dK, dV
template <int DN>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_kernel(BwdParams p) {
  using C = BwdCfg<DN>;
  __shared__ __attribute__((aligned(16))) bf16 Qs[C::BQ * C::Q_LD];
  __shared__ __attribute__((aligned(16))) bf16 QsT[C::DQK * C::QT_LD];
  __shared__ __attribute__((aligned(16))) bf16 dOs[C::BQ * C::DO_LD];
  __shared__ __attribute__((aligned(16))) bf16 dOT[C::DV * C::DOT_LD];
  __shared__ __attribute__((aligned(16))) float lse_s[C::BQ];
  __shared__ __attribute__((aligned(16))) float dsum_s[C::BQ];

  const int n_kt = (p.Tk + C::BKV - 1) / C::BKV;
  const int bh = blockIdx.x / n_kt;
  // causal: later key tiles see fewer queries; start with the heavy (early) ones
  const int kt = blockIdx.x - bh * n_kt;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int k0 = kt * C::BKV;
  const int key = k0 + 32 * w + l32;
  const int key_ld = key < p.Tk ? key : p.Tk - 1;

  // K and V rows of this lane's key: B operands of S = Q K^T and dP = dO V^T
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
#pragma unroll
    for (int ks = 0; ks < C::DV / 16; ++ks) vf[ks] = as_bf16x8(ldg16(vp + 16 * ks + 8 * g));
  }

  f32x16 dvacc[C::DV / 32], dkacc[C::NDQK];
#pragma unroll
  for (int i = 0; i < C::DV / 32; ++i) dvacc[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::NDQK; ++i) dkacc[i] = f32x16{};

  // query tiles that can see any key of this tile
  int q_first = 0;
  if (p.causal) {
    const int64_t qf = (int64_t)k0 - p.q_offset;
    q_first = qf <= 0 ? 0 : (int)(qf < p.Tq ? qf : p.Tq);
  }
  const int qt_begin = q_first / C::BQ;
  const int n_qt = (p.Tq + C::BQ - 1) / C::BQ;

  const bf16* qn_b = p.qn + (int64_t)b * p.qn_s.b + (int64_t)h * p.qn_s.h;
  const bf16* qr_b = p.qr + (int64_t)b * p.qr_s.b + (int64_t)h * p.qr_s.h;
  const bf16* do_b = p.dout + (int64_t)b * p.do_s.b + (int64_t)h * p.do_s.h;
  const float* lse_b = p.lse + ((int64_t)b * p.H + h) * p.Tq;
  const float* ds_b = p.dsum + ((int64_t)b * p.H + h) * p.Tq;

  Stager<C::BQ, C::DQK, DN, true, true> qst;
  Stager<C::BQ, C::DV, C::DV, true, true> dost;
  float lse_pre = 0.f, ds_pre = 0.f;
  auto load_q = [&](int q0) {
    qst.load(tid, qn_b, p.qn_s.t, qr_b, p.qr_s.t, q0, p.Tq);
    dost.load(tid, do_b, p.do_s.t, do_b, p.do_s.t, q0, p.Tq);
    if (tid < C::BQ) {
      const int q = q0 + tid;
      lse_pre = q < p.Tq ? lse_b[q] * kLog2e : 0.f;
      ds_pre = q < p.Tq ? ds_b[q] : 0.f;
    }
  };

  if (qt_begin < n_qt) load_q(qt_begin * C::BQ);
  for (int qt = qt_begin; qt < n_qt; ++qt) {
    const int q0 = qt * C::BQ;
    __syncthreads();
    qst.store(tid, Qs, C::Q_LD, QsT, C::QT_LD);
    dost.store(tid, dOs, C::DO_LD, dOT, C::DOT_LD);
    if (tid < C::BQ) {
      lse_s[tid] = lse_pre;
      dsum_s[tid] = ds_pre;
    }
    __syncthreads();
    if (qt + 1 < n_qt) load_q(q0 + C::BQ);

    // The loop body is kept branch-free (the mask is always evaluated, fully masked
    // tiles are computed as zeros): control flow here makes the compiler shuttle the
    // dK/dV accumulators between AGPRs and VGPRs every iteration.
    f32x16 sacc[C::QB], dpacc[C::QB];
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb) {
      sacc[qb] = f32x16{};
      dpacc[qb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
        sacc[qb] = mfma32(as_bf16x8(lds16(&Qs[(32 * qb + l32) * C::Q_LD + 16 * ks + 8 * g])), kf[ks], sacc[qb]);
#pragma unroll
      for (int ks = 0; ks < C::DV / 16; ++ks)
        dpacc[qb] = mfma32(as_bf16x8(lds16(&dOs[(32 * qb + l32) * C::DO_LD + 16 * ks + 8 * g])), vf[ks], dpacc[qb]);
    }

    // P and dS (registers r of block qb hold query 32 qb + 8 (r / 4) + 4 g + r % 4)
    bf16x8 pa[C::QB][2], dsa[C::QB][2];
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int ql = 32 * qb + 8 * r4 + 4 * g;  // first of 4 consecutive local queries
        const f32x4 lq = *reinterpret_cast<const f32x4*>(&lse_s[ql]);
        const f32x4 dq = *reinterpret_cast<const f32x4*>(&dsum_s[ql]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * r4 + i;
          float pv = fast_exp2(sacc[qb][r] * p.scale_log2 - lq[i]);
          {
            const int q = q0 + ql + i;
            const bool ok = q < p.Tq && (!p.causal || (int64_t)key <= (int64_t)q + p.q_offset);
            pv = ok ? pv : 0.f;
          }
          sacc[qb][r] = pv;
          dpacc[qb][r] = pv * (dpacc[qb][r] - dq[i]);
        }
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        u32x4 pk, dk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pk[e] = pack_bf16x2(sacc[qb][8 * s + 2 * e], sacc[qb][8 * s + 2 * e + 1]);
          dk[e] = pack_bf16x2(dpacc[qb][8 * s + 2 * e], dpacc[qb][8 * s + 2 * e + 1]);
        }
        pa[qb][s] = as_bf16x8(pk);
        dsa[qb][s] = as_bf16x8(dk);
      }
    }

    // dV += P^T dO ; dK += dS^T Q   (K slot (g, e) <-> query 32 qb + 16 s + 8 (e / 4) + 4 g + e % 4)
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int qo = 32 * qb + 16 * s + 4 * g;
#pragma unroll
        for (int db = 0; db < C::DV / 32; ++db)
          dvacc[db] = mfma32(pa[qb][s], lds_pair8(&dOT[(32 * db + l32) * C::DOT_LD + qo]), dvacc[db]);
#pragma unroll
        for (int nb = 0; nb < C::NDQK; ++nb)
          dkacc[nb] = mfma32(dsa[qb][s], lds_pair8(&QsT[(32 * nb + l32) * C::QT_LD + qo]), dkacc[nb]);
      }
    }
  }

  // ---- store: register r of block n holds row key (8 (r/4) + 4 g + r%4 within the wave), column 32 n + l32
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kk = k0 + 32 * w + 8 * (r >> 2) + 4 * g + (r & 3);
    if (kk >= p.Tk) continue;
    bf16* dvp = p.dv + (int64_t)b * p.dv_s.b + (int64_t)kk * p.dv_s.t + (int64_t)h * p.dv_s.h;
#pragma unroll
    for (int db = 0; db < C::DV / 32; ++db) dvp[32 * db + l32] = (bf16)dvacc[db][r];
    bf16* dkp = p.dkn + (int64_t)b * p.dkn_s.b + (int64_t)kk * p.dkn_s.t + (int64_t)h * p.dkn_s.h;
#pragma unroll
    for (int nb = 0; nb < C::NDQK; ++nb) {
      const int col = 32 * nb + l32;
      const float val = dkacc[nb][r] * p.scale;
      if (col < DN) {
        dkp[col] = (bf16)val;
      } else if (p.shared_rope) {
        p.dkr_ws[(((int64_t)b * p.Tk + kk) * p.H + h) * 64 + (col - DN)] = val;
      } else {
        p.dkr[(int64_t)b * p.dkr_s.b + (int64_t)kk * p.dkr_s.t + (int64_t)h * p.dkr_s.h + (col - DN)] = (bf16)val;
      }
    }
  }
}

// ---------------------------------------------------------------- dQ
template <int DN>
__global__ __launch_bounds__(256, 1) void bwd_dq_kernel(BwdParams p) {
  using C = BwdCfg<DN>;
  __shared__ __attribute__((aligned(16))) bf16 Ks[C::BK * C::K_LD];
  __shared__ __attribute__((aligned(16))) bf16 KsT[C::DQK * C::KT_LD];
  __shared__ __attribute__((aligned(16))) bf16 Vs[C::BK * C::V_LD];

  const int n_qt = (p.Tq + C::BQQ - 1) / C::BQQ;
  const int bh = blockIdx.x / n_qt;
  const int r_ = blockIdx.x - bh * n_qt;
  const int qt = p.causal ? n_qt - 1 - r_ : r_;  // longest first
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l32 = lane & 31, g = lane >> 5;
  const int q0 = qt * C::BQQ;
  const int q_row = q0 + 32 * w + l32;
  const int q_ld = q_row < p.Tq ? q_row : p.Tq - 1;

  bf16x8 qf[C::KS], dof[C::DV / 16];
  float lse2 = 0.f, dsum = 0.f;
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
    lse2 = p.lse[((int64_t)b * p.H + h) * p.Tq + q_ld] * kLog2e;
    dsum = p.dsum[((int64_t)b * p.H + h) * p.Tq + q_ld];
  }

  int kv_end = p.Tk;
  if (p.causal) {
    const int64_t lim = (int64_t)q0 + C::BQQ + p.q_offset;
    if (lim < kv_end) kv_end = lim < 0 ? 0 : (int)lim;
  }
  const int n_tiles = (kv_end + C::BK - 1) / C::BK;

  const bf16* kn_b = p.kn + (int64_t)b * p.kn_s.b + (int64_t)h * p.kn_s.h;
  const bf16* kr_b = p.kr + (int64_t)b * p.kr_s.b + (int64_t)h * p.kr_s.h;
  const bf16* v_b = p.v + (int64_t)b * p.v_s.b + (int64_t)h * p.v_s.h;

  Stager<C::BK, C::DQK, DN, true, true> kst;
  Stager<C::BK, C::DV, C::DV, true, false> vst;

  f32x16 dqacc[C::NDQK];
#pragma unroll
  for (int i = 0; i < C::NDQK; ++i) dqacc[i] = f32x16{};

  if (n_tiles > 0) {
    kst.load(tid, kn_b, p.kn_s.t, kr_b, p.kr_s.t, 0, p.Tk);
    vst.load(tid, v_b, p.v_s.t, v_b, p.v_s.t, 0, p.Tk);
  }
  for (int j = 0; j < n_tiles; ++j) {
    const int kv0 = j * C::BK;
    __syncthreads();
    kst.store(tid, Ks, C::K_LD, KsT, C::KT_LD);
    vst.store(tid, Vs, C::V_LD, nullptr, 0);
    __syncthreads();
    if (j + 1 < n_tiles) {
      kst.load(tid, kn_b, p.kn_s.t, kr_b, p.kr_s.t, kv0 + C::BK, p.Tk);
      vst.load(tid, v_b, p.v_s.t, v_b, p.v_s.t, kv0 + C::BK, p.Tk);
    }
    // branch-free body (see the dK/dV kernel): masked tiles contribute zeros
    f32x16 sacc[2], dpacc[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      sacc[jb] = f32x16{};
      dpacc[jb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
        sacc[jb] = mfma32(as_bf16x8(lds16(&Ks[(32 * jb + l32) * C::K_LD + 16 * ks + 8 * g])), qf[ks], sacc[jb]);
#pragma unroll
      for (int ks = 0; ks < C::DV / 16; ++ks)
        dpacc[jb] = mfma32(as_bf16x8(lds16(&Vs[(32 * jb + l32) * C::V_LD + 16 * ks + 8 * g])), dof[ks], dpacc[jb]);
    }
    bf16x8 dsb[2][2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fast_exp2(sacc[jb][r] * p.scale_log2 - lse2);
        {
          const int kv = kv0 + 32 * jb + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = kv < p.Tk && (!p.causal || (int64_t)kv <= (int64_t)q_row + p.q_offset);
          pv = ok ? pv : 0.f;
        }
        dpacc[jb][r] = pv * (dpacc[jb][r] - dsum);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        u32x4 pk;
#pragma unroll
        for (int e = 0; e < 4; ++e) pk[e] = pack_bf16x2(dpacc[jb][8 * s + 2 * e], dpacc[jb][8 * s + 2 * e + 1]);
        dsb[jb][s] = as_bf16x8(pk);
      }
    }
#pragma unroll
    for (int mb = 0; mb < C::NDQK; ++mb) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 a = lds_pair8(&KsT[(32 * mb + l32) * C::KT_LD + 32 * jb + 16 * s + 4 * g]);
          dqacc[mb] = mfma32(a, dsb[jb][s], dqacc[mb]);
        }
      }
    }
  }

  // ---- store dQ (times scale): lane = query, registers = 4 consecutive dims per (mb, r/4)
  if (q_row < p.Tq) {
    bf16* dqn = p.dqn + (int64_t)b * p.dqn_s.b + (int64_t)q_row * p.dqn_s.t + (int64_t)h * p.dqn_s.h;
    bf16* dqr = p.dqr + (int64_t)b * p.dqr_s.b + (int64_t)q_row * p.dqr_s.t + (int64_t)h * p.dqr_s.h;
#pragma unroll
    for (int mb = 0; mb < C::NDQK; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * mb + 8 * i + 4 * g;
        const u32x2 v2{pack_bf16x2(dqacc[mb][4 * i] * p.scale, dqacc[mb][4 * i + 1] * p.scale),
                       pack_bf16x2(dqacc[mb][4 * i + 2] * p.scale, dqacc[mb][4 * i + 3] * p.scale)};
        if (d < DN)
          stg8(dqn + d, v2);
        else
          stg8(dqr + (d - DN), v2);
      }
    }
  }
}

// ---------------------------------------------------------------- shared dk_rope = sum over heads
__global__ __launch_bounds__(256) void bwd_dkrope_reduce_kernel(BwdParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over B * Tk * 64
  const int64_t n = (int64_t)p.B * p.Tk * 64;
  if (idx >= n) return;
  const int c = (int)(idx & 63);
  const int64_t bt = idx >> 6;
  const int64_t t = bt % p.Tk, b = bt / p.Tk;
  const float* src = p.dkr_ws + (bt * p.H) * 64 + c;
  float acc = 0.f;
  for (int hh = 0; hh < p.H; ++hh) acc += src[hh * 64];
  p.dkr[b * p.dkr_s.b + t * p.dkr_s.t + c] = (bf16)acc;
}

template <int DN>
static int launch_bwd(const BwdParams& prm, hipStream_t s) {
  using C = BwdCfg<DN>;
  const int64_t rows = (int64_t)prm.B * prm.Tq * prm.H;
  if (rows > 0) bwd_rowdot_kernel<<<dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, s>>>(prm);
  const int64_t n_kt = (prm.Tk + C::BKV - 1) / C::BKV;
  const int64_t n_qt = (prm.Tq + C::BQQ - 1) / C::BQQ;
  MLA_CHECK((int64_t)prm.B * prm.H * n_kt < (1ll << 31) && (int64_t)prm.B * prm.H * n_qt < (1ll << 31),
            MLA_ERR_INVALID_ARG, "mla_prefill_bwd: grid too large");
  bwd_dkdv_kernel<DN><<<dim3((unsigned)(prm.B * prm.H * n_kt)), dim3(256), 0, s>>>(prm);
  bwd_dq_kernel<DN><<<dim3((unsigned)(prm.B * prm.H * n_qt)), dim3(256), 0, s>>>(prm);
  if (prm.shared_rope) {
    const int64_t n = (int64_t)prm.B * prm.Tk * 64;
    bwd_dkrope_reduce_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(prm);
  }
  return launch_status("mla_prefill_bwd");
}

static void bwd_ws_layout(const mla_prefill_bwd_args* a, size_t& d_bytes, size_t& ws_rope) {
  d_bytes = (((size_t)a->B * a->H * a->Tq * sizeof(float)) + 255) & ~(size_t)255;
  const bool shared = a->k_rope_stride.h == 0 && a->H > 1;
  ws_rope = shared ? (size_t)a->B * a->Tk * a->H * 64 * sizeof(float) : 0;
}

}  // namespace mla

using namespace mla;

extern "C" size_t mla_prefill_bwd_workspace_bytes(const mla_prefill_bwd_args* a) {
  if (!a || a->B <= 0 || a->H <= 0 || a->Tq < 0 || a->Tk < 0) return 0;
  size_t d, r;
  bwd_ws_layout(a, d, r);
  return d + r;
}

extern "C" int mla_prefill_bwd(const mla_prefill_bwd_args* a, void* stream) {
  const char* op = "mla_prefill_bwd";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->d_rope == 64 && a->d_v == 128 && (a->d_nope == 128 || a->d_nope == 64), MLA_ERR_UNSUPPORTED,
            "%s: head dims (nope %lld, rope %lld, v %lld) not built", op, (long long)a->d_nope,
            (long long)a->d_rope, (long long)a->d_v);
  MLA_CHECK(a->B >= 0 && a->H >= 0 && a->Tq >= 0 && a->Tk >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->B < (1 << 20) && a->H < (1 << 16) && a->Tq < (1 << 30) && a->Tk < (1 << 30), MLA_ERR_INVALID_ARG,
            "%s: size out of range", op);
  if (a->B == 0 || a->H == 0 || (a->Tq == 0 && a->Tk == 0)) return MLA_OK;
  MLA_CHECK(a->Tq > 0 && a->Tk > 0, MLA_ERR_INVALID_ARG, "%s: Tq and Tk must be positive", op);
  MLA_CHECK(!a->causal || a->q_offset >= 0, MLA_ERR_INVALID_ARG, "%s: q_offset must be >= 0", op);
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
  const bool shared = a->k_rope_stride.h == 0 && a->H > 1;
  MLA_CHECK(!shared || a->dk_rope_stride.h == 0, MLA_ERR_INVALID_ARG,
            "%s: a shared k_rope needs a shared dk_rope (head stride 0)", op);
  size_t d_bytes, ws_rope;
  bwd_ws_layout(a, d_bytes, ws_rope);
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
  prm.dsum = (float*)a->workspace;
  prm.dkr_ws = shared ? (float*)((char*)a->workspace + d_bytes) : nullptr;
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
  hipStream_t s = (hipStream_t)stream;
  return a->d_nope == 128 ? launch_bwd<128>(prm, s) : launch_bwd<64>(prm, s);
}
