// RMSNorm fused into the down-projection GEMM (gfx950): the block's norm1 in front of
// q_down / qk_rope / kv_down (transformer.py:16-27 at :338, then :208-213):
//   r[m]    = 1 / sqrt(sum_k x[m][k]^2 / K + eps)
//   xn[m][k] = bf16((x[m][k] r[m]) w[k])                       (fp32 arithmetic)
//   y[m][n] = bf16( sum_k xn[m][k] W[n][k] )                    (fp32 accumulation)
// the reference's fused kernel (fused_mla_triton_kernels.py:105-230) and its numerics: a first
// pass over x forms r (norm_rms_kernel, 4 bytes per row out), the GEMM streams x again and
// normalises each tile in LDS before its products.  The normalised rows never reach memory.
//
// GEMM.  The product runs transposed, C^T [N][M] = W . xn^T, on v_mfma_f32_32x32x16_bf16: a
// lane's accumulators hold 4 consecutive n of one row m (8-byte stores).  A workgroup computes
// 256 (n) x 256 (m) outputs with 8 waves, wave (wn, wm) owning n rows [128 wn, +128) and m
// columns [64 wm, +64): 8 accumulator blocks of 32 x 32, 128 registers, two waves per SIMD
// (4 waves of 128 m columns, one per SIMD with 256 accumulator registers, measured 475 against
// 377 us at M = 24576, K = 2048, N = 2624).  K advances in stages of 32.  Both operand tiles of
// a stage (256 rows x 64 bytes each) arrive by direct-to-LDS loads into a 4-stage ring, three
// stages ahead; while stage s is multiplied, stage s + 1 (landed at the previous barrier) is
// normalised in place by all threads, 16-byte chunks, with r[m] in registers and w from an LDS
// copy; one barrier per stage.  A row's 4 chunks sit at position c ^ ((row / 4) mod 4), so the
// fragment reads (16 rows x one chunk per 16 lanes) are free of bank conflicts.  The finished
// tile goes through LDS as bf16 rows [m][n], so each wave stores 512 contiguous bytes of y.
#include <cmath>

#include "mla_common.h"

namespace mla {

struct NlParams {
  const bf16* x;         // [M][K], row stride xs
  const bf16* w;         // W [N][K], row stride ws (nn.Linear weights, concatenated)
  const float* wn;       // norm weight [K]
  bf16* y;               // [M][N], row stride ys
  float* inv_rms;        // [M]: written by norm_rms_kernel, read by norm_linear_kernel
  int M, N, K, xs, ws, ys;
  float inv_k, eps;
};

constexpr int kNlBM = 256;    // m per workgroup
constexpr int kNlBN = 256;    // n per workgroup
constexpr int kNlBK = 32;     // k per stage
constexpr int kNlStages = 4;  // LDS ring depth
constexpr int kNlMaxK = 4096; // the norm weight's LDS copy (16 KiB at most)
constexpr int kNlStageBytes = (kNlBN + kNlBM) * kNlBK * 2;  // 32 KiB: W tile, then x tile
constexpr int kNlXOff = kNlBN * kNlBK * 2;                  // the x tile within a stage
constexpr int kNlWMC = 64;                                  // m columns per wave

__device__ __forceinline__ int nl_swz(int row) { return (row >> 2) & 3; }

template <int N>
__device__ __forceinline__ void nl_wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// r[m] of 4 rows per workgroup, one wave per row: lane l sums the squares of 16-byte chunks
// l, l + 64, ... of the row in fp32, then a butterfly over the wave
__global__ __launch_bounds__(256) void norm_rms_kernel(NlParams p) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= p.M) return;  // wave-uniform; no barrier follows
  const bf16* xr = p.x + (int64_t)row * p.xs;
  float ss = 0.f;
  for (int c = lane; c < p.K / 8; c += 64) {
    const u32x4 v = ldg16(xr + 8 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf16(v[e]), hi = hi_bf16(v[e]);
      ss += lo * lo;
      ss += hi * hi;
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ss += wave_shfl_xor(ss, s);
  if (lane == 0) p.inv_rms[row] = 1.f / sqrtf(ss * p.inv_k + p.eps);
}

// WMC: m columns per wave (64: 8 waves, two per SIMD; 128: 4 waves, one per SIMD)
template <int WMC>
__global__ __launch_bounds__(64 * 2 * (kNlBM / WMC), 1) void norm_linear_kernel(NlParams p) {
  constexpr int NW = 2 * (kNlBM / WMC);           // waves
  constexpr int NT = 64 * NW;                     // threads
  constexpr int XJ = WMC / 32;                    // x (m) blocks per wave
  constexpr int LOADS = (kNlStageBytes / 1024) / NW;  // direct-to-LDS loads per wave per stage
  constexpr int NCH = (kNlBM * kNlBK / 8) / NT;   // x chunks each thread normalises per stage
  constexpr int ES = kNlBN * 2 + 16;              // epilogue staging row stride (bytes)
  static_assert(kNlStages * kNlStageBytes >= kNlBM * ES - (kNlMaxK * 4), "epilogue staging fits the LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kNlStages * kNlStageBytes + kNlMaxK * 4];
  unsigned char* const ring = lds;
  float* const wls = (float*)(lds + kNlStages * kNlStageBytes);

  // workgroup -> (n tile, m tile); the n tiles of one m tile are consecutive ids, so the x rows
  // they share meet in one XCD's L2 (hardware places id on XCD id % 8)
  const int n_nt = (p.N + kNlBN - 1) / kNlBN;
  const int n_wg = gridDim.x;
  int id = blockIdx.x;
  if ((n_wg & 7) == 0) id = (id & 7) * (n_wg >> 3) + (id >> 3);
  const int nt = id % n_nt, mt = id / n_nt;
  const int n0 = nt * kNlBN, m0 = mt * kNlBM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = w / (NW / 2), wm = w % (NW / 2);  // n rows [128 wn, +128), m columns [WMC wm, +WMC)
  const int l32 = lane & 31, hk = lane >> 5;

  // direct-to-LDS loads: stage tile rows 0..255 are W rows n0 + row, rows 256..511 x rows
  // m0 + row - 256; load i (of 32 per stage) covers rows 16 i .. 16 i + 15, lane q: row 16 i + q / 4,
  // position q % 4, which holds the row's chunk (q % 4) ^ swz(row).  Rows past N or M read zero
  // (the descriptors end at the last valid row) and their outputs are not stored.
  const int nv = min(kNlBN, p.N - n0), mv = min(kNlBM, p.M - m0);
  const buf_rsrc rw = make_rsrc(p.w + (int64_t)n0 * p.ws, rows_bytes(nv, p.ws, p.K * 2));
  const buf_rsrc rx = make_rsrc(p.x + (int64_t)m0 * p.xs, rows_bytes(mv, p.xs, p.K * 2));
  const uint32_t lds0 = lds_addr(ring);
  uint32_t voff[LOADS];  // byte offsets at k = 0 of this lane's chunk in each of the wave's loads
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int i = w + NW * j;  // load index: 0..15 W rows, 16..31 x rows
    const int row = 16 * (i & 15) + (lane >> 2);
    const int c = (lane & 3) ^ nl_swz(row);
    voff[j] = (uint32_t)(row * (i < 16 ? p.ws : p.xs) * 2 + c * 16);
  }
  auto issue_stage = [&](int s, int slot) {
    const uint32_t kb = (uint32_t)(s * kNlBK * 2);
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int i = w + NW * j;
      dma16(i < 16 ? rw : rx, voff[j] + kb, lds0 + (uint32_t)(slot * kNlStageBytes + i * 1024));
    }
  };

  const int n_st = p.K / kNlBK;
#pragma unroll
  for (int s = 0; s < kNlStages - 1; ++s)
    if (s < n_st) issue_stage(s, s);

  // the norm weight to LDS, and r of the x rows this thread normalises: chunk positions
  // q = tid + NT i of the x tile, row q / 4, position q % 4
  for (int k = tid; k < p.K; k += NT) wls[k] = p.wn[k];
  float rn[NCH];
  int noff[NCH], nk[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int q = tid + NT * i;
    const int row = q >> 2, pos = q & 3;
    noff[i] = kNlXOff + row * 64 + pos * 16;
    nk[i] = 8 * (pos ^ nl_swz(row));  // k offset (within a stage) of the chunk held at this position
    rn[i] = m0 + row < p.M ? p.inv_rms[m0 + row] : 0.f;
  }
  // normalise the x tile of stage s (in slot `slot`) in place
  auto normalise = [&](int s, int slot) {
    unsigned char* st = ring + slot * kNlStageBytes;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int k = s * kNlBK + nk[i];
      const u32x4 v = lds16(st + noff[i]);
      const f32x4 w0 = __builtin_bit_cast(f32x4, lds16(wls + k)), w1 = __builtin_bit_cast(f32x4, lds16(wls + k + 4));
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        o[e] = pack_bf16x2((lo_bf16(v[e]) * rn[i]) * w0[2 * e], (hi_bf16(v[e]) * rn[i]) * w0[2 * e + 1]);
        o[2 + e] = pack_bf16x2((lo_bf16(v[2 + e]) * rn[i]) * w1[2 * e], (hi_bf16(v[2 + e]) * rn[i]) * w1[2 * e + 1]);
      }
      sts16(st + noff[i], o);
    }
  };

  // fragment read offsets within a stage: W block i (32 rows), x block j (32 rows), k16 half h:
  // lane (l32, hk) reads row l32 of the block, chunk 2 h + hk
  int offw[2], offx[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rw_ = 128 * wn + l32;  // the block's row within the tile is + 32 i (swz unchanged)
    offw[h] = rw_ * 64 + (((2 * h + hk) ^ nl_swz(rw_)) * 16);
    const int rx_ = kNlBN + WMC * wm + l32;
    offx[h] = rx_ * 64 + (((2 * h + hk) ^ nl_swz(rx_)) * 16);
  }

  f32x16 acc[4][XJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < XJ; ++j) acc[i][j] = f32x16{};

  // stages 0 and 1 have landed when at most stage 2's loads are in flight; stage 0 is normalised
  // before the loop, each later stage one iteration ahead of its products
  if (n_st >= 3) nl_wait_vmem<LOADS>();
  else nl_wait_vmem<0>();
  __syncthreads();  // the landed stages and the norm weight are visible
  normalise(0, 0);
  __syncthreads();

  int slot = 0;
  for (int s = 0; s < n_st; ++s) {
    if (s + kNlStages - 1 < n_st) {
      int sn = slot + kNlStages - 1;
      sn -= sn >= kNlStages ? kNlStages : 0;
      issue_stage(s + kNlStages - 1, sn);  // into the slot stage s - 1 used
    }
    // all fragment reads of stage s first, then the products of its first k16 half, the
    // normalisation of stage s + 1 (its VALU work runs under those MFMAs), the second half
    const unsigned char* st = ring + slot * kNlStageBytes;
    bf16x8 fw[2][4], fx[2][XJ];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < 4; ++i) fw[h][i] = as_bf16x8(lds16(st + offw[h] + i * 32 * 64));
#pragma unroll
      for (int j = 0; j < XJ; ++j) fx[h][j] = as_bf16x8(lds16(st + offx[h] + j * 32 * 64));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < XJ; ++j) acc[i][j] = mfma32(fw[0][i], fx[0][j], acc[i][j]);
    if (s + 1 < n_st) normalise(s + 1, slot + 1 == kNlStages ? 0 : slot + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < XJ; ++j) acc[i][j] = mfma32(fw[1][i], fx[1][j], acc[i][j]);
    // stage s + 2 (normalised next iteration) must have landed; stage s + 3's loads may fly
    if (s + 3 < n_st) nl_wait_vmem<LOADS>();
    else nl_wait_vmem<0>();
    __syncthreads();
    slot = slot + 1 == kNlStages ? 0 : slot + 1;
  }

  // ---- epilogue: the tile as bf16 rows [m][n] in LDS (the ring is free past the last barrier),
  // then whole row segments stored with 8-byte writes, 512 contiguous bytes per wave
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    unsigned char* er = lds + (WMC * wm + 32 * j + l32) * ES;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // accumulator rows 8 g + 4 hk + [0, 4) of block i: n = 128 wn + 32 i + 8 g + 4 hk
        const f32x16& a = acc[i][j];
        sts8(er + (128 * wn + 32 * i + 8 * g + 4 * hk) * 2,
             u32x2{pack_bf16x2(a[4 * g], a[4 * g + 1]), pack_bf16x2(a[4 * g + 2], a[4 * g + 3])});
      }
    }
  }
  __syncthreads();
  for (int c = tid; c < kNlBM * (kNlBN / 4); c += NT) {
    const int row = c / (kNlBN / 4), n = 4 * (c % (kNlBN / 4));
    if (row < mv && n < nv) stg8(p.y + (int64_t)(m0 + row) * p.ys + n0 + n, lds8(lds + row * ES + n * 2));
  }
}

}  // namespace mla

using namespace mla;

extern "C" int mla_norm_linear(const mla_norm_linear_args* a, void* stream) {
  const char* op = "mla_norm_linear";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->M >= 0 && a->N >= 0 && a->K >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->M < (1ll << 31) && a->N < (1 << 20), MLA_ERR_INVALID_ARG, "%s: size out of range", op);
  if (a->M == 0 || a->N == 0) return MLA_OK;
  MLA_CHECK(a->K > 0 && a->K % kNlBK == 0 && a->K <= kNlMaxK, MLA_ERR_UNSUPPORTED,
            "%s: K = %lld must be a positive multiple of %d up to %d", op, (long long)a->K, kNlBK, kNlMaxK);
  MLA_CHECK(a->N % 4 == 0, MLA_ERR_UNSUPPORTED, "%s: N = %lld must be a multiple of 4", op, (long long)a->N);
  MLA_CHECK(a->x && a->w && a->w_norm && a->y && a->inv_rms, MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  MLA_CHECK(((uintptr_t)a->x & 15) == 0 && ((uintptr_t)a->w & 15) == 0 && ((uintptr_t)a->w_norm & 15) == 0 &&
                ((uintptr_t)a->y & 7) == 0 && ((uintptr_t)a->inv_rms & 3) == 0,
            MLA_ERR_INVALID_ARG, "%s: x, w and w_norm must be 16-byte aligned, y 8-byte aligned", op);
  MLA_CHECK(a->x_stride >= a->K && a->w_stride >= a->K && a->y_stride >= a->N && a->x_stride % 8 == 0 &&
                a->w_stride % 8 == 0 && a->y_stride % 4 == 0,
            MLA_ERR_INVALID_ARG, "%s: row strides must cover a row and be multiples of 8 (x, w) and 4 (y)", op);
  // a tile's 256 rows must be addressable with 32-bit offsets from its first row
  MLA_CHECK(a->x_stride < (1 << 22) && a->w_stride < (1 << 22) && a->y_stride < (1ll << 31), MLA_ERR_INVALID_ARG,
            "%s: row stride too large", op);
  MLA_CHECK(std::isfinite(a->eps) && a->eps >= 0.f, MLA_ERR_INVALID_ARG, "%s: eps must be finite and >= 0", op);
  const int64_t n_wg = ((a->M + kNlBM - 1) / kNlBM) * ((a->N + kNlBN - 1) / kNlBN);
  MLA_CHECK(n_wg < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: grid too large", op);
  NlParams p{(const bf16*)a->x, (const bf16*)a->w, a->w_norm, (bf16*)a->y, a->inv_rms, (int)a->M, (int)a->N, (int)a->K,
             (int)a->x_stride, (int)a->w_stride, (int)a->y_stride, 1.f / (float)a->K, a->eps};
  hipStream_t s = (hipStream_t)stream;
  norm_rms_kernel<<<dim3((unsigned)((a->M + 3) / 4)), dim3(256), 0, s>>>(p);
  MLA_TRY(launch_status(op));
  norm_linear_kernel<kNlWMC><<<dim3((unsigned)n_wg), dim3(64 * 2 * (kNlBM / kNlWMC)), 0, s>>>(p);
  return launch_status(op);
}
