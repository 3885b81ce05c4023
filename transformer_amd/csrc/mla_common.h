// Shared device helpers for the gfx950 (CDNA4) MLA kernels.
//
// Conventions used by every kernel in this directory:
//  * wave64; a workgroup of 256 threads is 4 waves;
//  * bf16 data move as 16-byte (8 x bf16) or 8-byte (4 x bf16) vectors;
//  * MFMA tiles are v_mfma_f32_32x32x16_bf16 (prefill, backward) and
//    v_mfma_f32_16x16x32_bf16 (decode).  For an MFMA A[M][K] * B[K][N]:
//      32x32x16: lane l supplies A row (l % 32) and B column (l % 32), with K slots
//                k = 8 * (l / 32) + e, e = 0..7 (one bf16x8 per lane);
//                accumulator register r of lane l holds C[row][col] with
//                col = l % 32, row = 8 * (r / 4) + 4 * (l / 32) + (r % 4).
//      16x16x32: lane l supplies A row (l % 16) and B column (l % 16), K slots
//                k = 8 * (l / 16) + e; accumulator register r holds
//                C[4 * (l / 16) + r][l % 16].
//    Only the M/N placement matters for correctness: the K slot order is the same
//    function for A and B, so any consistent permutation of K is exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mla_mi355x.h"

namespace mla {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float lo_bf16(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

// round-to-nearest-even pack of two floats into (lo, hi) bf16 halves (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(const bf16x8& v) { return __builtin_bit_cast(u32x4, v); }

__device__ __forceinline__ u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void stg16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ldg8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void stg8(void* p, const u32x2& v) { *reinterpret_cast<u32x2*>(p) = v; }

// LDS vector access (addresses are byte offsets into a __shared__ array)
__device__ __forceinline__ u32x4 lds16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void sts16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 lds8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void sts8(void* p, const u32x2& v) { *reinterpret_cast<u32x2*>(p) = v; }

// select 16-bit halves: returns (lo16(a), lo16(b)) or (hi16(a), hi16(b)) packed
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xffff0000u);
}

// Transpose a 4 (rows) x 8 (cols) block of bf16 held as 4 rows of u32x4 into
// 8 (cols) x 4 (rows): out[c] = {r0[c], r1[c], r2[c], r3[c]} as u32x2.
__device__ __forceinline__ void transpose4x8(const u32x4 r[4], u32x2 out[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    out[2 * w + 0] = u32x2{pack_lo16(r[0][w], r[1][w]), pack_lo16(r[2][w], r[3][w])};
    out[2 * w + 1] = u32x2{pack_hi16(r[0][w], r[1][w]), pack_hi16(r[2][w], r[3][w])};
  }
}

// Raw buffer access: a descriptor (base, size in bytes) in SGPRs and 32-bit per-lane byte
// offsets.  Loads at or beyond `nbytes` return zero in hardware, so tiles that run past
// the end of an operand need no clamping.  Word 3 = 0x00020000 (32-bit data format).
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bld16(buf_rsrc r, uint32_t voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0));
}
// bytes covering rows [0, n) of a row-strided operand whose rows are row_bytes wide
__device__ __forceinline__ uint32_t rows_bytes(int n, int64_t stride_elems, int row_bytes) {
  return n <= 0 ? 0u : (uint32_t)((int64_t)(n - 1) * stride_elems * 2 + row_bytes);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b, c) in one v_max3_f32 (the compiler does not form it from fmaxf chains here)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// The decoupled RoPE rotation of one pair of 8-element runs (transformer.py:55-60): x1 holds rope
// dims f .. f + 7, x2 dims f + 32 .. f + 39, c / s the bf16 table entries of frequencies f ..
// f + 7 (sin_sign -1 rotates by the opposite angle).  y1 = x1 c - x2 s, y2 = x1 s + x2 c in fp32,
// each formed as one fma over one product, then rounded to bf16 once: every kernel that rotates
// uses this, so rotated values agree bit for bit wherever they are made.
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float& y1, float& y2) {
  y1 = __builtin_fmaf(x1, c, -(x2 * s));
  y2 = __builtin_fmaf(x1, s, x2 * c);
}
__device__ __forceinline__ void rope_rotate8(bf16x8& x1, bf16x8& x2, const u32x4& cw, const u32x4& sw,
                                             float sin_sign = 1.f) {
  const u32x4 a = as_u32x4(x1), bb = as_u32x4(x2);
  u32x4 ra, rb;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float y1l, y2l, y1h, y2h;
    rope_pair(lo_bf16(a[w]), lo_bf16(bb[w]), lo_bf16(cw[w]), lo_bf16(sw[w]) * sin_sign, y1l, y2l);
    rope_pair(hi_bf16(a[w]), hi_bf16(bb[w]), hi_bf16(cw[w]), hi_bf16(sw[w]) * sin_sign, y1h, y2h);
    ra[w] = pack_bf16x2(y1l, y1h);
    rb[w] = pack_bf16x2(y2l, y2h);
  }
  x1 = as_bf16x8(ra);
  x2 = as_bf16x8(rb);
}

__device__ __forceinline__ float wave_shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }
// v of this lane combined with v of lane l ^ 32 by a commutative op (the result is the same in
// both lanes, bit for bit): v_permlane32_swap of v with itself leaves the lane holding its own
// value and its partner's, with no LDS round trip.
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// the same with lane l ^ 16 (v_permlane16_swap: rows of 16 lanes)
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Wait until at most n (0 <= n <= 15) vector memory operations of this wave are in flight;
// n is wave-uniform.
__device__ __forceinline__ void wait_vmem(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

// One 1 KiB direct-to-LDS load: lane l's 16 bytes land at LDS byte address lds + 16 l.
// Written as inline assembly so that the compiler neither waits for it before unrelated
// LDS reads nor models it as a register result: the kernel orders these loads itself
// (s_waitcnt vmcnt + barrier before a stage is read).  M0 is set here and is not used by
// any other instruction of the kernels that use it.
__device__ __forceinline__ void dma16(buf_rsrc r, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(voff), "s"(r)
               : "memory", "m0");
}
// the same with the non-temporal hint, for data read once (it should not displace lines that
// other workgroups reuse)
__device__ __forceinline__ void dma16_nt(buf_rsrc r, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(lds), "v"(voff), "s"(r)
               : "memory", "m0");
}
// The same with the LDS destination given as a base register plus a constant (M0 =
// lds_base + LDS_OFF is formed here): the compiler then keeps one base per stage in an SGPR
// rather than one M0 value per stage and load.
template <int LDS_OFF>
__device__ __forceinline__ void dma16_at(buf_rsrc r, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_add_u32 m0, %0, %3\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds_base), "v"(voff), "s"(r),
               "i"(LDS_OFF)
               : "memory", "m0", "scc");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace mla

// ------------------------------------------------------------------ host side
namespace mla {
void set_error(const char* fmt, ...);
int launch_status(const char* what);
// validates a [B, T, heads, dim] bf16 operand: non-null, 16-byte aligned, strides
// non-negative multiples of 8 elements
int check_operand(const char* op, const char* name, const void* ptr, const mla_strides& st);
// the softmax scale must be finite and positive: the kernels take a row's reference max
// before scaling (a positive factor commutes with max), and 2^(s * scale * log2 e) must
// stay finite for finite scores
int check_scale(const char* op, float scale);
}  // namespace mla

#define MLA_TRY(expr)              \
  do {                             \
    int _rc = (expr);              \
    if (_rc != MLA_OK) return _rc; \
  } while (0)

#define MLA_CHECK(cond, code, ...)     \
  do {                                 \
    if (!(cond)) {                     \
      ::mla::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)
