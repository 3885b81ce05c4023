// Row RMSNorm, forward and backward, in front of the MLA down-projections (gfx950).
//
//   r[m] = 1 / sqrt(sum_k x[m][k]^2 / K + eps),   y[m][k] = (x[m][k] * r[m]) * w[k]
//
// restates RMSNorm.forward (transformer.py:26-27), x * rsqrt(mean(x^2) + eps) * weight, in
// fp32 and in the same order.  y is stored as bf16 (the rounding autocast applies where the
// down-projection GEMM, transformer.py:208-213, reads the norm's output) or as fp32 (an
// fp32 module outside autocast).
//
// The op moves bytes and does little arithmetic (HBM-bound): one wave per row; lane l owns
// the row's 8-element chunks c = l + 64 i (i < NC), loaded as 16-byte vectors (two for an
// fp32 row) and kept in registers between the sum of squares and the scaling.  A wave
// walks rows row, row + n_waves, ...; it issues the next row's loads before it reduces the
// current row, so two rows per wave are in flight, and keeps w in registers across rows.
// The wave-wide sum is a butterfly of shuffles, which leaves the same total (and r) in
// every lane.
//
// Backward (autograd of the same expression, t = x r, y = t w):
//   g = w dy,  dx = r g - x (r^3 / K) sum_k(g x),  dw = sum_m dy t.
// The row walk computes dx; each lane accumulates dy t for its columns over the wave's
// rows, the workgroup's four waves add theirs through LDS into one row of partials per
// workgroup, and a second kernel sums those rows column by column in a fixed order, so dw
// is bitwise reproducible (no atomics).
#include <type_traits>

#include "mla_common.h"

namespace mla {

constexpr int kRmsMaxK = 4096;  // NC <= 8 chunks per lane keeps the row in registers
constexpr int kRmsFwdMaxGrid = 4096;
constexpr int kRmsBwdMaxGrid = 512;

struct RmsFwdParams {
  const void* x;
  const float* w;
  void* y;
  float* inv;
  int M, K;
  int64_t xs, ys;
  float eps;
};

struct RmsBwdParams {
  const void* dy;
  const void* x;
  const float* w;
  const float* inv;
  void* dx;
  float* part;  // [gridDim.x, K] per-workgroup dw partials
  int M, K;
  int64_t dys, xs, dxs;
};

// 8 consecutive elements of a row as fp32 (bf16 rows: one 16-byte load; fp32: two)
template <bool F32>
struct Chunk {
  typename std::conditional<F32, f32x4, u32x4>::type a, b;
};
template <bool F32>
__device__ __forceinline__ void load_chunk(Chunk<F32>& c, const void* row, int k) {
  if constexpr (F32) {
    const float* p = static_cast<const float*>(row) + k;
    c.a = *reinterpret_cast<const f32x4*>(p);
    c.b = *reinterpret_cast<const f32x4*>(p + 4);
  } else {
    c.a = ldg16(static_cast<const bf16*>(row) + k);
  }
}
template <bool F32>
__device__ __forceinline__ void unpack_chunk(const Chunk<F32>& c, float v[8]) {
  if constexpr (F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = c.a[e];
      v[4 + e] = c.b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = lo_bf16(c.a[e]);
      v[2 * e + 1] = hi_bf16(c.a[e]);
    }
  }
}
template <bool F32>
__device__ __forceinline__ void store_chunk(void* row, int k, const float v[8]) {
  if constexpr (F32) {
    float* p = static_cast<float*>(row) + k;
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    stg16(static_cast<bf16*>(row) + k,
          u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])});
  }
}

__device__ __forceinline__ float wave_sum(float s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  return s;
}

template <bool XF32, bool YF32, int NC>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(RmsFwdParams p) {
  const int lane = threadIdx.x & 63;
  const int n_waves = gridDim.x * 4;
  const int nch = p.K >> 3;
  float w[NC][8];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    Chunk<true> wc;
    if (c < nch) load_chunk(wc, p.w, 8 * c);
    else wc.a = wc.b = f32x4{0.f, 0.f, 0.f, 0.f};
    unpack_chunk(wc, w[i]);
  }
  Chunk<XF32> cur[NC], nxt[NC];
  auto load_row = [&](int row, Chunk<XF32>(&r)[NC]) {
    const void* base = XF32 ? (const void*)((const float*)p.x + (int64_t)row * p.xs)
                            : (const void*)((const bf16*)p.x + (int64_t)row * p.xs);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) load_chunk(r[i], base, 8 * c);
    }
  };
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row < p.M) load_row(row, cur);
  for (; row < p.M; row += n_waves) {
    if (row + n_waves < p.M) load_row(row + n_waves, nxt);
    float v[NC][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        unpack_chunk(cur[i], v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
    }
    ss = wave_sum(ss);
    const float r = 1.f / sqrtf(ss / (float)p.K + p.eps);
    void* yrow = YF32 ? (void*)((float*)p.y + (int64_t)row * p.ys) : (void*)((bf16*)p.y + (int64_t)row * p.ys);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (v[i][e] * r) * w[i][e];
        store_chunk<YF32>(yrow, 8 * c, o);
      }
    }
    if (p.inv && lane == 0) p.inv[row] = r;
#pragma unroll
    for (int i = 0; i < NC; ++i) cur[i] = nxt[i];
  }
}

template <bool XF32, bool DYF32, int NC>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(RmsBwdParams p) {
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int n_waves = gridDim.x * 4;
  const int nch = p.K >> 3;
  const float inv_k = 1.f / (float)p.K;
  float w[NC][8], dw[NC][8];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    Chunk<true> wc;
    if (c < nch) load_chunk(wc, p.w, 8 * c);
    else wc.a = wc.b = f32x4{0.f, 0.f, 0.f, 0.f};
    unpack_chunk(wc, w[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) dw[i][e] = 0.f;
  }
  for (int row = blockIdx.x * 4 + wv; row < p.M; row += n_waves) {
    const void* dyrow = DYF32 ? (const void*)((const float*)p.dy + (int64_t)row * p.dys)
                              : (const void*)((const bf16*)p.dy + (int64_t)row * p.dys);
    const void* xrow = XF32 ? (const void*)((const float*)p.x + (int64_t)row * p.xs)
                            : (const void*)((const bf16*)p.x + (int64_t)row * p.xs);
    Chunk<DYF32> dyc[NC];
    Chunk<XF32> xc[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        load_chunk(dyc[i], dyrow, 8 * c);
        load_chunk(xc[i], xrow, 8 * c);
      }
    }
    const float r = p.inv[row];
    float g[NC][8], xv[NC][8];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      float dyv[8];
      if (c < nch) {
        unpack_chunk(dyc[i], dyv);
        unpack_chunk(xc[i], xv[i]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) dyv[e] = xv[i][e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        g[i][e] = w[i][e] * dyv[e];
        s = __builtin_fmaf(g[i][e], xv[i][e], s);
        dw[i][e] = __builtin_fmaf(dyv[e], xv[i][e] * r, dw[i][e]);
      }
    }
    s = wave_sum(s);
    const float coef = r * r * r * inv_k * s;
    void* dxrow = XF32 ? (void*)((float*)p.dx + (int64_t)row * p.dxs) : (void*)((bf16*)p.dx + (int64_t)row * p.dxs);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = r * g[i][e] - xv[i][e] * coef;
        store_chunk<XF32>(dxrow, 8 * c, o);
      }
    }
  }
  // the four waves' partials -> one row of this workgroup, chunk by chunk through LDS
  __shared__ f32x4 red[4][128];  // [wave][lane * 2 + half]: 8 floats per lane
  float* part = p.part + (int64_t)blockIdx.x * p.K;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    red[wv][2 * lane] = f32x4{dw[i][0], dw[i][1], dw[i][2], dw[i][3]};
    red[wv][2 * lane + 1] = f32x4{dw[i][4], dw[i][5], dw[i][6], dw[i][7]};
    __syncthreads();
    // thread t sums quad t of the 128 quads (lane t / 2, half t % 2) over the waves in order
    const int t = threadIdx.x;
    if (t < 128) {
      const f32x4 a = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
      const int c = (t >> 1) + 64 * i;
      if (c < nch) *reinterpret_cast<f32x4*>(part + 8 * c + 4 * (t & 1)) = a;
    }
    __syncthreads();
  }
}

// dw[k] = sum over the G workgroup rows of part[g][k], in order g = 0, 1, ...: each wave
// takes every fourth row, and the four wave sums are added in wave order.
__global__ __launch_bounds__(256) void rmsnorm_dw_reduce_kernel(const float* part, float* dw, int G, int K) {
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (col < K)
    for (int g = wv; g < G; g += 4) s += part[(int64_t)g * K + col];
  __shared__ float red[4][64];
  red[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && col < K) dw[col] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// chunks per lane for a row of K elements: the smallest built NC >= K / 512
static int rms_nc(int64_t K) {
  const int64_t need = (K / 8 + 63) / 64;
  for (int nc : {1, 2, 3, 4, 6, 8})
    if (nc >= need) return nc;
  return 0;
}

template <bool XF32, bool YF32>
static void launch_rms_fwd(int nc, const RmsFwdParams& prm, int grid, hipStream_t s) {
  switch (nc) {
    case 1: rmsnorm_fwd_kernel<XF32, YF32, 1><<<grid, 256, 0, s>>>(prm); break;
    case 2: rmsnorm_fwd_kernel<XF32, YF32, 2><<<grid, 256, 0, s>>>(prm); break;
    case 3: rmsnorm_fwd_kernel<XF32, YF32, 3><<<grid, 256, 0, s>>>(prm); break;
    case 4: rmsnorm_fwd_kernel<XF32, YF32, 4><<<grid, 256, 0, s>>>(prm); break;
    case 6: rmsnorm_fwd_kernel<XF32, YF32, 6><<<grid, 256, 0, s>>>(prm); break;
    default: rmsnorm_fwd_kernel<XF32, YF32, 8><<<grid, 256, 0, s>>>(prm); break;
  }
}
template <bool XF32, bool DYF32>
static void launch_rms_bwd(int nc, const RmsBwdParams& prm, int grid, hipStream_t s) {
  switch (nc) {
    case 1: rmsnorm_bwd_kernel<XF32, DYF32, 1><<<grid, 256, 0, s>>>(prm); break;
    case 2: rmsnorm_bwd_kernel<XF32, DYF32, 2><<<grid, 256, 0, s>>>(prm); break;
    case 3: rmsnorm_bwd_kernel<XF32, DYF32, 3><<<grid, 256, 0, s>>>(prm); break;
    case 4: rmsnorm_bwd_kernel<XF32, DYF32, 4><<<grid, 256, 0, s>>>(prm); break;
    case 6: rmsnorm_bwd_kernel<XF32, DYF32, 6><<<grid, 256, 0, s>>>(prm); break;
    default: rmsnorm_bwd_kernel<XF32, DYF32, 8><<<grid, 256, 0, s>>>(prm); break;
  }
}

static int rms_check_row_operand(const char* op, const char* name, const void* ptr, int64_t stride, int64_t M,
                                 int64_t K) {
  MLA_CHECK(ptr, MLA_ERR_INVALID_ARG, "%s: %s is null", op, name);
  MLA_CHECK(((uintptr_t)ptr & 15) == 0, MLA_ERR_INVALID_ARG, "%s: %s must be 16-byte aligned", op, name);
  MLA_CHECK(M <= 1 || (stride >= K && (stride & 7) == 0), MLA_ERR_INVALID_ARG,
            "%s: %s row stride %lld must be >= K and a multiple of 8", op, name, (long long)stride);
  return MLA_OK;
}

static int rms_bwd_grid(int64_t M) { return (int)(M <= 0 ? 0 : std::min<int64_t>((M + 3) / 4, kRmsBwdMaxGrid)); }

}  // namespace mla

using namespace mla;

extern "C" int mla_rmsnorm(const mla_rmsnorm_args* a, void* stream) {
  const char* op = "mla_rmsnorm";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->M >= 0 && a->M < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: M out of range", op);
  MLA_CHECK(a->K > 0 && a->K <= kRmsMaxK && (a->K & 7) == 0, MLA_ERR_UNSUPPORTED,
            "%s: K = %lld must be a positive multiple of 8 and at most %d", op, (long long)a->K, kRmsMaxK);
  MLA_CHECK(a->x_dtype == MLA_DTYPE_BF16 || a->x_dtype == MLA_DTYPE_F32, MLA_ERR_UNSUPPORTED, "%s: x dtype", op);
  MLA_CHECK(a->y_dtype == MLA_DTYPE_BF16 || a->y_dtype == MLA_DTYPE_F32, MLA_ERR_UNSUPPORTED, "%s: y dtype", op);
  MLA_CHECK(a->eps >= 0.f, MLA_ERR_INVALID_ARG, "%s: eps must be >= 0", op);
  if (a->M == 0) return MLA_OK;
  MLA_TRY(rms_check_row_operand(op, "x", a->x, a->x_stride, a->M, a->K));
  MLA_TRY(rms_check_row_operand(op, "y", a->y, a->y_stride, a->M, a->K));
  MLA_TRY(rms_check_row_operand(op, "w", a->w, a->K, 1, a->K));
  RmsFwdParams prm{a->x, a->w, a->y, a->inv_rms, (int)a->M, (int)a->K, a->x_stride, a->y_stride, a->eps};
  const int grid = (int)std::min<int64_t>((a->M + 3) / 4, kRmsFwdMaxGrid);
  const int nc = rms_nc(a->K);
  hipStream_t s = (hipStream_t)stream;
  const bool xf = a->x_dtype == MLA_DTYPE_F32, yf = a->y_dtype == MLA_DTYPE_F32;
  if (xf && yf) launch_rms_fwd<true, true>(nc, prm, grid, s);
  else if (xf) launch_rms_fwd<true, false>(nc, prm, grid, s);
  else if (yf) launch_rms_fwd<false, true>(nc, prm, grid, s);
  else launch_rms_fwd<false, false>(nc, prm, grid, s);
  return launch_status(op);
}

extern "C" size_t mla_rmsnorm_bwd_workspace_bytes(const mla_rmsnorm_bwd_args* a) {
  // 0 for the sizes mla_rmsnorm_bwd rejects
  if (!a || a->M <= 0 || a->M >= (1ll << 31) || a->K <= 0 || a->K > kRmsMaxK || (a->K & 7) != 0) return 0;
  return (size_t)rms_bwd_grid(a->M) * (size_t)a->K * sizeof(float);
}

extern "C" int mla_rmsnorm_bwd(const mla_rmsnorm_bwd_args* a, void* stream) {
  const char* op = "mla_rmsnorm_bwd";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->M >= 0 && a->M < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: M out of range", op);
  MLA_CHECK(a->K > 0 && a->K <= kRmsMaxK && (a->K & 7) == 0, MLA_ERR_UNSUPPORTED,
            "%s: K = %lld must be a positive multiple of 8 and at most %d", op, (long long)a->K, kRmsMaxK);
  MLA_CHECK(a->x_dtype == MLA_DTYPE_BF16 || a->x_dtype == MLA_DTYPE_F32, MLA_ERR_UNSUPPORTED, "%s: x dtype", op);
  MLA_CHECK(a->dy_dtype == MLA_DTYPE_BF16 || a->dy_dtype == MLA_DTYPE_F32, MLA_ERR_UNSUPPORTED, "%s: dy dtype", op);
  MLA_TRY(rms_check_row_operand(op, "w", a->w, a->K, 1, a->K));
  MLA_TRY(rms_check_row_operand(op, "dw", a->dw, a->K, 1, a->K));
  const int G = rms_bwd_grid(a->M);
  hipStream_t s = (hipStream_t)stream;
  if (G > 0) {
    MLA_TRY(rms_check_row_operand(op, "dy", a->dy, a->dy_stride, a->M, a->K));
    MLA_TRY(rms_check_row_operand(op, "x", a->x, a->x_stride, a->M, a->K));
    MLA_TRY(rms_check_row_operand(op, "dx", a->dx, a->dx_stride, a->M, a->K));
    MLA_CHECK(a->inv_rms, MLA_ERR_INVALID_ARG, "%s: inv_rms is null", op);
    const size_t need = mla_rmsnorm_bwd_workspace_bytes(a);
    MLA_CHECK(a->workspace && a->workspace_bytes >= need && ((uintptr_t)a->workspace & 15) == 0, MLA_ERR_WORKSPACE,
              "%s: workspace of %zu bytes (16-byte aligned) needed, %zu given", op, need, a->workspace_bytes);
    RmsBwdParams prm{a->dy, a->x, a->w, a->inv_rms, a->dx, (float*)a->workspace,
                     (int)a->M, (int)a->K, a->dy_stride, a->x_stride, a->dx_stride};
    const int nc = rms_nc(a->K);
    const bool xf = a->x_dtype == MLA_DTYPE_F32, df = a->dy_dtype == MLA_DTYPE_F32;
    if (xf && df) launch_rms_bwd<true, true>(nc, prm, G, s);
    else if (xf) launch_rms_bwd<true, false>(nc, prm, G, s);
    else if (df) launch_rms_bwd<false, true>(nc, prm, G, s);
    else launch_rms_bwd<false, false>(nc, prm, G, s);
    MLA_TRY(launch_status(op));
  }
  rmsnorm_dw_reduce_kernel<<<(unsigned)((a->K + 63) / 64), 256, 0, s>>>((const float*)a->workspace, a->dw, G,
                                                                        (int)a->K);
  return launch_status(op);
}
