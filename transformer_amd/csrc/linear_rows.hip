// Products of a few rows with a weight matrix, for the decode step (gfx950):
//   y[g][m][n] = sum_k x[g][m][k] W[g][n][k],   m < M (a few rows), n < N, k < K, g < G
// bf16 inputs, fp32 accumulation, one rounding to bf16.  W is [N, K] with K contiguous (an
// nn.Linear weight, or a per-head slice of one); G > 1 runs G independent products of the
// same shape (the per-head W_UK absorption).
//
// With M = 32 (one token of each of 32 sequences) these products are bound by reading W
// once (10.7 MB for the down-projections at the ModelArgs.mla_baseline dims) and by latency, and a
// vendor GEMM tiles them for large M.  Here a workgroup owns 16 output columns of one
// group.  Its 16 weight rows are staged whole in LDS by direct-to-LDS loads of contiguous
// 1 KiB runs (loads of 16 rows x 64 bytes streamed at a fraction of the rate), while each
// wave loads its x fragments into registers; the four waves split K, run
// v_mfma_f32_16x16x32_bf16 on C^T [16 n][16 m] blocks, and their partial sums are added
// through LDS in wave order (deterministic).  A lane then holds 4 consecutive columns of one
// row: 8-byte stores.  With fewer than 256 column blocks the 16-row passes are split over
// workgroups whose ids differ by 8 (one XCD, so the weights' second read hits its L2): twice
// the workgroups, each reading half of x.
//
// MFMA layout (16x16x32): lane l supplies A row l % 16 (= W row n0 + l % 16) and B column
// l % 16 (= x row m0 + l % 16), K slots 8 (l / 16) + e; accumulator r holds
// C[4 (l / 16) + r][l % 16], i.e. y[m0 + l % 16][n0 + 4 (l / 16) + r].
#include <algorithm>

#include "mla_common.h"
#include "rope_append.h"

namespace mla {

struct RowsParams {
  const bf16* x;
  const bf16* w;
  bf16* y;
  int M, N, K, G;
  int64_t x_sm, x_sg, w_sn, w_sg, y_sm, y_sg;
  int nz;  // row splits: workgroup split mz takes the 16 MB-row passes mz, mz + nz, ...
};

constexpr int kRowsKsMax = 16;  // k-steps of 32 per wave held in flight (K <= 4 * 32 * 16 = 2048 per pass)
constexpr int kRowsAhead = 3;      // weight fragments read ahead of their products
constexpr int kRowsFillWgs = 256;  // workgroups that fill the chip (one per CU)
constexpr int kRowsMaxK = 4096;  // the workgroup's 16 weight rows are staged whole in LDS (<= 128 KiB)

// MB: 16-row blocks of x handled together (M <= 16 MB per pass).  Dynamic LDS: 16 K bf16.
// Workgroup (bx, g) of the product: bx as blockIdx.x of linear_rows_kernel, g the group.
template <int MB>
__device__ __forceinline__ void linear_rows_block(const RowsParams& p, int bx, int g) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char wt[];  // [16 rows][K], chunks swizzled
  const int lane = threadIdx.x & 63;
  // wave-uniform (an SGPR): the k-step guards below must be scalar branches, since an MFMA
  // runs whatever the EXEC mask holds and a lane-masked guard would not skip it
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, q = lane >> 4;
  // bx -> (column block cb, row split mz of p.nz): the p.nz splits of a column block get ids 8
  // apart, so they run on one XCD (id % 8) and the second read of its weights hits L2
  int cb, mz;
  {
    const int blk = bx, nz = p.nz, n_cb = (p.N + 15) / 16;
    const int base = (n_cb / 8) * 8 * nz;
    if (blk < base) {
      cb = (blk / (8 * nz)) * 8 + (blk & 7);
      mz = (blk >> 3) % nz;
    } else {
      cb = (n_cb / 8) * 8 + (blk - base) / nz;
      mz = (blk - base) % nz;
    }
  }
  const int n0 = cb * 16;
  const int C = p.K / 8;  // 16-byte chunks per weight row (a multiple of 16)

  // The workgroup's weight rows n0 .. n0 + 15 go to LDS through direct-to-LDS loads of 1 KiB
  // runs (64 lanes x 16 bytes): load i fills the flattened chunks [64 i, 64 i + 64) of
  // [16 rows][C chunks].  Chunk position pos of row r holds the row's chunk pos ^ r (r < 16 <=
  // C, so the XOR stays inside the row), which keeps the fragment reads below conflict-free.
  // The descriptor covers the valid rows only: rows past N load nothing.
  {
    const int n_valid = min(16, p.N - n0);
    const bf16* wb = p.w + (int64_t)g * p.w_sg + (int64_t)n0 * p.w_sn;
    const buf_rsrc r = make_rsrc(wb, rows_bytes(n_valid, p.w_sn, p.K * 2));
    const uint32_t base = lds_addr(wt);
    for (int i = w; i < C / 4; i += 4) {
      const int fq = 64 * i + lane;
      const int row = fq / C, pos = fq - row * C;
      const uint32_t voff = (uint32_t)(row * p.w_sn * 2 + ((pos ^ row) << 4));
      dma16(r, voff, base + 1024u * (uint32_t)i);
    }
  }
  const bf16* xg = p.x + (int64_t)g * p.x_sg + 8 * q;
  __shared__ f32x4 red[4][MB][64];
  // this lane's fragment row of the staged weights: row l16, chunk c at (c ^ l16)
  const unsigned char* wrow = wt + l16 * C * 16;

  bool first = true;  // the staged weights are awaited once, before the first products
  for (int m0 = 16 * MB * mz; m0 < p.M; m0 += 16 * MB * p.nz) {
    f32x4 acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = f32x4{};
    const bf16* xr[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int m = min(m0 + 16 * i + l16, p.M - 1);  // clamped: rows past M are not stored
      xr[i] = xg + (int64_t)m * p.x_sm;
    }
    // wave w takes the k-steps (of 32) w, w + 4, ...; passes of kRowsKsMax steps (K is a
    // multiple of 128, so every wave has the same number of steps and meets the barrier once)
    const int n_ks = p.K / 32;
    for (int ks0 = w; ks0 < n_ks; ks0 += 4 * kRowsKsMax) {
      const int n_sw = min(kRowsKsMax, (n_ks - ks0 + 3) / 4);  // steps of this pass (>= 1)
      u32x4 xv[kRowsKsMax][MB];
#pragma unroll
      for (int s = 0; s < kRowsKsMax; ++s) {
        if (s < n_sw) {
          const int ks = ks0 + 4 * s;
#pragma unroll
          for (int i = 0; i < MB; ++i) xv[s][i] = ldg16(xr[i] + 32 * ks);
        }
      }
      if (first) {  // the staged weights have landed (every wave's loads)
        first = false;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      }
      // weight fragments are read kRowsAhead k-steps ahead of their products, so that many LDS
      // reads are in flight at each wait (at most kRowsAhead + 1 fragments live)
      auto wfrag = [&](int s) {
        const int c = 4 * (ks0 + 4 * s) + q;  // this lane's chunk of the k-step
        return as_bf16x8(lds16(wrow + ((c ^ l16) << 4)));
      };
      bf16x8 wv[kRowsKsMax];
#pragma unroll
      for (int s = 0; s < kRowsAhead; ++s)
        if (s < n_sw) wv[s] = wfrag(s);
#pragma unroll
      for (int s = 0; s < kRowsKsMax; ++s) {
        if (s < n_sw) {
          if (s + kRowsAhead < kRowsKsMax && s + kRowsAhead < n_sw) wv[s + kRowsAhead] = wfrag(s + kRowsAhead);
#pragma unroll
          for (int i = 0; i < MB; ++i) acc[i] = mfma16(wv[s], as_bf16x8(xv[s][i]), acc[i]);
        }
      }
    }
    // the four waves' partial sums, added in wave order
#pragma unroll
    for (int i = 0; i < MB; ++i) red[w][i][lane] = acc[i];
    __syncthreads();
    for (int i = w; i < MB; i += 4) {
      const f32x4 s = ((red[0][i][lane] + red[1][i][lane]) + red[2][i][lane]) + red[3][i][lane];
      const int m = m0 + 16 * i + l16;
      const int n = n0 + 4 * q;
      if (m < p.M && n < p.N)
        stg8(p.y + (int64_t)g * p.y_sg + (int64_t)m * p.y_sm + n,
             u32x2{pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])});
    }
    __syncthreads();  // red is reused by the next row pass
  }
}

template <int MB>
__global__ __launch_bounds__(256) void linear_rows_kernel(RowsParams p) {
  linear_rows_block<MB>(p, blockIdx.x, blockIdx.y);
}

// The decode step's q_up product and its RoPE + cache append (rope_append_block) in one launch:
// both read only the down-projection's output, so workgroups [0, n_rows) run the product
// (workgroup i as (i % n_rows_x, i / n_rows_x) of linear_rows_kernel's grid) and the rest the
// append blocks.  One launch instead of two in the recorded step; the arithmetic of each part
// is that of its own kernel.
template <int MB>
__global__ __launch_bounds__(256) void linear_rows_rope_append_kernel(RowsParams p, RopeAppendParams r, int n_rows_x,
                                                                      int n_rows) {
  const int blk = blockIdx.x;
  if (blk < n_rows) linear_rows_block<MB>(p, blk % n_rows_x, blk / n_rows_x);
  else rope_append_block(r, (int64_t)(blk - n_rows));
}

}  // namespace mla

using namespace mla;

// Checks the arguments and fills the launch: the kernel's MB, its grid and dynamic LDS bytes; mb = 0
// when there is nothing to launch.
static int rows_setup(const mla_linear_rows_args* a, const char* op, RowsParams& p, int& mb, dim3& grid,
                      size_t& lds) {
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->M >= 0 && a->N >= 0 && a->K >= 0 && a->G >= 0, MLA_ERR_INVALID_ARG, "%s: negative size", op);
  MLA_CHECK(a->M < (1 << 20) && a->N < (1 << 24) && a->K < (1 << 20) && a->G < 65536, MLA_ERR_INVALID_ARG,
            "%s: size out of range", op);
  mb = 0;
  if (a->M == 0 || a->N == 0 || a->G == 0) return MLA_OK;
  MLA_CHECK(a->K > 0 && a->K % 128 == 0 && a->K <= kRowsMaxK, MLA_ERR_UNSUPPORTED,
            "%s: K = %lld must be a positive multiple of 128 up to %d", op, (long long)a->K, kRowsMaxK);
  MLA_CHECK(a->N % 4 == 0, MLA_ERR_UNSUPPORTED, "%s: N = %lld must be a multiple of 4", op, (long long)a->N);
  MLA_CHECK(a->x && a->w && a->y, MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  MLA_CHECK(((uintptr_t)a->x & 15) == 0 && ((uintptr_t)a->w & 15) == 0 && ((uintptr_t)a->y & 7) == 0,
            MLA_ERR_INVALID_ARG, "%s: x and w must be 16-byte aligned, y 8-byte aligned", op);
  const int64_t st[] = {a->x_sm, a->x_sg, a->w_sn, a->w_sg};
  for (int64_t s : st)
    MLA_CHECK(s >= 0 && (s & 7) == 0, MLA_ERR_INVALID_ARG, "%s: x and w strides must be non-negative multiples of 8",
              op);
  MLA_CHECK(a->y_sm >= 0 && a->y_sg >= 0 && (a->y_sm & 3) == 0 && (a->y_sg & 3) == 0, MLA_ERR_INVALID_ARG,
            "%s: y strides must be non-negative multiples of 4", op);
  p = RowsParams{(const bf16*)a->x, (const bf16*)a->w, (bf16*)a->y, (int)a->M, (int)a->N, (int)a->K, (int)a->G,
                 a->x_sm, a->x_sg, a->w_sn, a->w_sg, a->y_sm, a->y_sg, 1};
  const int64_t n_cb = (a->N + 15) / 16;
  lds = (size_t)16 * a->K * 2;
  if (n_cb * a->G < kRowsFillWgs && a->M > 16) {
    // too few column blocks to fill the chip: 16-row passes split over workgroups (each then
    // reads half or less of x, and the weights once more from L2)
    p.nz = (int)std::min<int64_t>((a->M + 15) / 16, (kRowsFillWgs + n_cb * a->G - 1) / (n_cb * a->G));
    mb = 1;
    grid = dim3((unsigned)(n_cb * p.nz), (unsigned)a->G);
    return MLA_OK;
  }
  grid = dim3((unsigned)n_cb, (unsigned)a->G);
  mb = a->M <= 16 ? 1 : a->M <= 32 ? 2 : 4;
  return MLA_OK;
}

extern "C" int mla_linear_rows(const mla_linear_rows_args* a, void* stream) {
  const char* op = "mla_linear_rows";
  RowsParams p;
  int mb = 0;
  dim3 grid;
  size_t lds = 0;
  MLA_TRY(rows_setup(a, op, p, mb, grid, lds));
  if (mb == 0) return MLA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (mb == 1) linear_rows_kernel<1><<<grid, 256, lds, s>>>(p);
  else if (mb == 2) linear_rows_kernel<2><<<grid, 256, lds, s>>>(p);
  else linear_rows_kernel<4><<<grid, 256, lds, s>>>(p);
  return launch_status(op);
}

extern "C" int mla_linear_rows_rope_append(const mla_linear_rows_args* rows, const mla_rope_append_args* rope,
                                           void* stream) {
  const char* op = "mla_linear_rows_rope_append";
  RowsParams p{};  // left zero when a part has nothing to launch (its blocks are then absent)
  int mb = 0;
  dim3 grid;
  size_t lds = 0;
  MLA_TRY(rows_setup(rows, op, p, mb, grid, lds));
  RopeAppendParams r{};
  int64_t r_blocks = 0;
  MLA_TRY(rope_append_setup(rope, op, r, r_blocks));
  const int64_t n_rows = mb ? (int64_t)grid.x * grid.y : 0;
  MLA_CHECK(n_rows + r_blocks < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: grid too large", op);
  if (n_rows + r_blocks == 0) return MLA_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 g1((unsigned)(n_rows + r_blocks));
  const int nx = (int)grid.x, nr = (int)n_rows;
  if (mb <= 1) linear_rows_rope_append_kernel<1><<<g1, 256, lds, s>>>(p, r, nx, nr);
  else if (mb == 2) linear_rows_rope_append_kernel<2><<<g1, 256, lds, s>>>(p, r, nx, nr);
  else linear_rows_rope_append_kernel<4><<<g1, 256, lds, s>>>(p, r, nx, nr);
  return launch_status(op);
}
