// RoPE of the new tokens with the cache append (transformer.py:215-218, :228-244), as a block
// body shared by rope_append_kernel (rope.hip) and the decode step's combined launch with the
// q_up product (linear_rows.hip), plus the argument checks both entry points run.
#pragma once
#include <algorithm>

#include "mla_common.h"

namespace mla {

template <typename T>
struct RopeIO;

template <>
struct RopeIO<bf16> {
  // load 8 consecutive elements as floats
  __device__ static void load8(const bf16* p, float v[8]) {
    u32x4 r = ldg16(p);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      v[2 * w] = lo_bf16(r[w]);
      v[2 * w + 1] = hi_bf16(r[w]);
    }
  }
  __device__ static void store8(bf16* p, const float v[8]) {
    u32x4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r[w] = pack_bf16x2(v[2 * w], v[2 * w + 1]);
    stg16(p, r);
  }
};

template <>
struct RopeIO<float> {
  __device__ static void load8(const float* p, float v[8]) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
  __device__ static void store8(float* p, const float v[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
};

struct RopeAppendParams {
  const bf16* qk;
  bf16* q_out;
  const bf16* c_new;
  bf16* latent;
  bf16* k_cache;
  const bf16* cos;
  const bf16* sin;
  const int64_t* pos_dev;
  int32_t* seq_lens;
  int64_t* pos_next;
  int64_t B, T, H, Hr, d_latent, limit, pos_offset;  // limit = min(table_rows, capacity)
  mla_strides qk_s, q_s;
  int64_t c_sb, c_st, l_sb, l_st, k_sb, k_sh, k_st;
  int64_t n_rope_blocks;  // blocks [0, n_rope_blocks) rotate head vectors, the rest copy latent rows
};

// Block blk of the append.  Blocks [0, n_rope_blocks): 4 threads per 64-wide head vector, as rope_kernel; q heads go to
// q_out, k heads into the cache slot at p.  The other blocks copy the new latent rows, one
// 16-byte chunk per thread.  Block 0 also writes seq_lens and the next position.  Every thread reads the position
// itself, so nothing orders the blocks.
__device__ __forceinline__ void rope_append_block(const RopeAppendParams& a, int64_t blk) {
  const int64_t pos0 = a.pos_offset + (a.pos_dev ? *a.pos_dev : 0);
  if (blk == 0 && a.seq_lens)
    for (int64_t b = threadIdx.x; b < a.B; b += 256) a.seq_lens[b] = (int32_t)(pos0 + a.T);
  if (blk == 0 && threadIdx.x == 0 && a.pos_next) *a.pos_next = pos0 + a.T;  // a buffer nobody here reads
  const int64_t nh = a.H + a.Hr;
  if (blk < a.n_rope_blocks) {
    const int64_t vec = blk * 64 + (threadIdx.x >> 2);
    if (vec >= a.B * a.T * nh) return;
    const int part = threadIdx.x & 3;
    const int64_t j = vec % nh;
    const int64_t bt = vec / nh;
    const int64_t t = bt % a.T;
    const int64_t b = bt / a.T;
    const int64_t p = pos0 + t;
    if (p < 0 || p >= a.limit) return;
    const bf16* xp = a.qk + b * a.qk_s.b + t * a.qk_s.t + j * a.qk_s.h + part * 8;
    float x1[8], x2[8], c[8], s[8], y1[8], y2[8];
    RopeIO<bf16>::load8(xp, x1);
    RopeIO<bf16>::load8(xp + 32, x2);
    RopeIO<bf16>::load8(a.cos + p * 32 + part * 8, c);
    RopeIO<bf16>::load8(a.sin + p * 32 + part * 8, s);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      rope_pair(x1[i], x2[i], c[i], s[i], y1[i], y2[i]);
    }
    bf16* yp = j < a.H ? a.q_out + b * a.q_s.b + t * a.q_s.t + j * a.q_s.h + part * 8
                       : a.k_cache + b * a.k_sb + (j - a.H) * a.k_sh + p * a.k_st + part * 8;
    RopeIO<bf16>::store8(yp, y1);
    RopeIO<bf16>::store8(yp + 32, y2);
  } else {
    const int64_t nch = a.d_latent >> 3;
    const int64_t idx = (blk - a.n_rope_blocks) * 256 + threadIdx.x;
    if (idx >= a.B * a.T * nch) return;
    const int64_t ch = idx % nch;
    const int64_t bt = idx / nch;
    const int64_t t = bt % a.T;
    const int64_t b = bt / a.T;
    const int64_t p = pos0 + t;
    if (p < 0 || p >= a.limit) return;
    stg16(a.latent + b * a.l_sb + p * a.l_st + 8 * ch, ldg16(a.c_new + b * a.c_sb + t * a.c_st + 8 * ch));
  }
}

// Checks the arguments of mla_rope_append and fills the kernel parameters; blocks = 0 when there
// is nothing to launch (B == 0 or T == 0).
inline int rope_append_setup(const mla_rope_append_args* a, const char* op, RopeAppendParams& p, int64_t& blocks) {
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->B >= 0 && a->T >= 0 && a->H >= 0 && a->Hr >= 0 && a->d_latent >= 0, MLA_ERR_INVALID_ARG,
            "%s: negative size", op);
  MLA_CHECK(a->d_latent % 8 == 0, MLA_ERR_INVALID_ARG, "%s: d_latent must be a multiple of 8", op);
  MLA_CHECK(a->capacity >= 0 && a->table_rows >= 0, MLA_ERR_INVALID_ARG, "%s: negative capacity", op);
  blocks = 0;
  if (a->B == 0 || a->T == 0) return MLA_OK;
  MLA_CHECK(a->qk && a->q_out && a->cos && a->sin && (a->latent || a->d_latent == 0) && (a->k_cache || a->Hr == 0) &&
                (a->c_new || a->d_latent == 0),
            MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  MLA_CHECK(a->pos_dev || (a->pos_offset >= 0 && a->pos_offset + a->T <= std::min(a->table_rows, a->capacity)),
            MLA_ERR_INVALID_ARG, "%s: positions [%lld, %lld) exceed the table (%lld rows) or the cache (%lld)", op,
            (long long)a->pos_offset, (long long)(a->pos_offset + a->T), (long long)a->table_rows,
            (long long)a->capacity);
  const void* ptrs[] = {a->qk, a->q_out, a->c_new, a->latent, a->k_cache, a->cos, a->sin};
  for (const void* q : ptrs) MLA_CHECK(((uintptr_t)q & 15) == 0, MLA_ERR_INVALID_ARG, "%s: pointers must be 16-byte aligned", op);
  const int64_t st[] = {a->qk_stride.b, a->qk_stride.t, a->qk_stride.h, a->q_stride.b, a->q_stride.t, a->q_stride.h,
                        a->c_new_sb,    a->c_new_st,    a->latent_sb,   a->latent_st, a->k_cache_sb, a->k_cache_sh,
                        a->k_cache_st};
  for (int64_t s : st) MLA_CHECK(s >= 0 && (s & 7) == 0, MLA_ERR_INVALID_ARG, "%s: strides must be non-negative multiples of 8", op);
  p.qk = (const bf16*)a->qk;
  p.q_out = (bf16*)a->q_out;
  p.c_new = (const bf16*)a->c_new;
  p.latent = (bf16*)a->latent;
  p.k_cache = (bf16*)a->k_cache;
  p.cos = (const bf16*)a->cos;
  p.sin = (const bf16*)a->sin;
  MLA_CHECK(!a->pos_next || (const int64_t*)a->pos_next != a->pos_dev, MLA_ERR_INVALID_ARG,
            "%s: pos_next must not be pos_dev (other workgroups still read it)", op);
  p.pos_dev = a->pos_dev;
  p.seq_lens = a->seq_lens;
  p.pos_next = a->pos_next;
  p.B = a->B;
  p.T = a->T;
  p.H = a->H;
  p.Hr = a->Hr;
  p.d_latent = a->d_latent;
  p.limit = std::min(a->table_rows, a->capacity);
  p.pos_offset = a->pos_offset;
  p.qk_s = a->qk_stride;
  p.q_s = a->q_stride;
  p.c_sb = a->c_new_sb;
  p.c_st = a->c_new_st;
  p.l_sb = a->latent_sb;
  p.l_st = a->latent_st;
  p.k_sb = a->k_cache_sb;
  p.k_sh = a->k_cache_sh;
  p.k_st = a->k_cache_st;
  const int64_t n_vec = a->B * a->T * (a->H + a->Hr);
  p.n_rope_blocks = (n_vec + 63) / 64;
  const int64_t n_copy = (a->B * a->T * (a->d_latent / 8) + 255) / 256;
  blocks = std::max<int64_t>(1, p.n_rope_blocks + n_copy);
  MLA_CHECK(blocks < (1ll << 31), MLA_ERR_INVALID_ARG, "%s: too many rows", op);
  return MLA_OK;
}

}  // namespace mla
