// Fused decoupled RoPE (split-half rotation of a 64-wide slice) over all q and k
// heads of a token in one pass.  Restates transformer.py:55-60 applied at :228-239:
//   y1 = x1 c - x2 s,  y2 = x1 s + x2 c   with (c, s) from the bf16 tables at row
//   pos_offset + t.  Arithmetic is fp32 (rope_pair: one fma over one product per output, the
//   form every kernel that rotates shares) with one rounding to the output dtype.
//
// HBM-bound: 4 threads per 64-wide head vector, each moving 8 pairs as 16-byte
// vectors (bf16) so every wave touches 16 whole vectors = 2 KiB contiguous when
// the heads of a token are adjacent.
#include "mla_common.h"
#include "rope_append.h"

namespace mla {

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, T* y, const bf16* __restrict__ cos_t,
                                                   const bf16* __restrict__ sin_t, uint32_t n_vec, uint32_t T_len,
                                                   uint32_t n_heads, int64_t pos_offset, mla_strides xs,
                                                   mla_strides ys, float sin_sign) {
  // 32-bit index arithmetic: the host keeps n_vec below 2^31
  const uint32_t vec = blockIdx.x * 64u + (threadIdx.x >> 2);
  if (vec >= n_vec) return;
  const int part = threadIdx.x & 3;  // pairs [8 part, 8 part + 8)
  const uint32_t bt = vec / n_heads;
  const int64_t h = vec - bt * n_heads;
  const uint32_t bq = bt / T_len;
  const int64_t t = bt - bq * T_len;
  const int64_t b = bq;
  const int64_t pos = pos_offset + t;

  const T* xp = x + b * xs.b + t * xs.t + h * xs.h + part * 8;
  T* yp = y + b * ys.b + t * ys.t + h * ys.h + part * 8;
  float x1[8], x2[8], c[8], s[8];
  RopeIO<T>::load8(xp, x1);
  RopeIO<T>::load8(xp + 32, x2);
  RopeIO<bf16>::load8(cos_t + pos * 32 + part * 8, c);
  RopeIO<bf16>::load8(sin_t + pos * 32 + part * 8, s);
  float y1[8], y2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float si = s[i] * sin_sign;
    rope_pair(x1[i], x2[i], c[i], si, y1[i], y2[i]);
  }
  RopeIO<T>::store8(yp, y1);
  RopeIO<T>::store8(yp + 32, y2);
}

}  // namespace mla

using namespace mla;

extern "C" int mla_rope(const mla_rope_args* a, void* stream) {
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "mla_rope: null args");
  MLA_CHECK(a->x && a->y && a->cos && a->sin, MLA_ERR_INVALID_ARG, "mla_rope: null pointer");
  MLA_CHECK(a->dtype == MLA_DTYPE_BF16 || a->dtype == MLA_DTYPE_F32, MLA_ERR_UNSUPPORTED,
            "mla_rope: dtype %d not supported (bf16=0, f32=1)", a->dtype);
  MLA_CHECK(a->B >= 0 && a->T >= 0 && a->n_heads >= 0, MLA_ERR_INVALID_ARG, "mla_rope: negative size");
  MLA_CHECK(a->pos_offset >= 0 && a->pos_offset + a->T <= a->table_rows, MLA_ERR_INVALID_ARG,
            "mla_rope: positions [%lld, %lld) exceed the %lld-row RoPE table", (long long)a->pos_offset,
            (long long)(a->pos_offset + a->T), (long long)a->table_rows);
  const int64_t esz = a->dtype == MLA_DTYPE_BF16 ? 2 : 4;
  const int64_t vec_elems = 16 / esz;
  const mla_strides xs = a->x_stride, ys = a->y_stride;
  MLA_CHECK(xs.b % vec_elems == 0 && xs.t % vec_elems == 0 && xs.h % vec_elems == 0 && ys.b % vec_elems == 0 &&
                ys.t % vec_elems == 0 && ys.h % vec_elems == 0,
            MLA_ERR_INVALID_ARG, "mla_rope: strides must be multiples of 16 bytes");
  MLA_CHECK(((uintptr_t)a->x % 16) == 0 && ((uintptr_t)a->y % 16) == 0 && ((uintptr_t)a->cos % 16) == 0 &&
                ((uintptr_t)a->sin % 16) == 0,
            MLA_ERR_INVALID_ARG, "mla_rope: pointers must be 16-byte aligned");
  int64_t n_vec = 0;
  MLA_CHECK(!__builtin_mul_overflow(a->B, a->T, &n_vec) && !__builtin_mul_overflow(n_vec, a->n_heads, &n_vec),
            MLA_ERR_INVALID_ARG, "mla_rope: B * T * heads overflows");
  if (n_vec == 0) return MLA_OK;
  const int64_t blocks = (n_vec + 63) / 64;
  MLA_CHECK(n_vec < (1ll << 31), MLA_ERR_INVALID_ARG, "mla_rope: too many vectors (B * T * heads >= 2^31)");
  hipStream_t s = (hipStream_t)stream;
  const float sign = a->inverse ? -1.0f : 1.0f;
  if (a->dtype == MLA_DTYPE_BF16) {
    rope_kernel<bf16><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const bf16*)a->x, (bf16*)a->y, (const bf16*)a->cos, (const bf16*)a->sin, (uint32_t)n_vec, (uint32_t)a->T,
        (uint32_t)a->n_heads, a->pos_offset, xs, ys, sign);
  } else {
    rope_kernel<float><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const float*)a->x, (float*)a->y, (const bf16*)a->cos, (const bf16*)a->sin, (uint32_t)n_vec, (uint32_t)a->T,
        (uint32_t)a->n_heads, a->pos_offset, xs, ys, sign);
  }
  return launch_status("mla_rope");
}

// ---------------------------------------------------------------- RoPE + cache append
namespace mla {

__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendParams a) { rope_append_block(a, blockIdx.x); }

}  // namespace mla

extern "C" int mla_rope_append(const mla_rope_append_args* a, void* stream) {
  const char* op = "mla_rope_append";
  RopeAppendParams p;
  int64_t blocks = 0;
  MLA_TRY(rope_append_setup(a, op, p, blocks));
  if (blocks == 0) return MLA_OK;
  rope_append_kernel<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(p);
  return launch_status(op);
}
