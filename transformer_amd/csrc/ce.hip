// One vocabulary chunk of the exact softmax cross-entropy over the tied output weights
// (chunked_linear_cross_entropy, transformer.py:62-115), after hipBLASLt has produced the
// chunk's logits [N, Vc]: bf16 under autocast (the reference's matmul dtype there), fp32 for
// an fp32 caller outside autocast (the reference then computes the logits in fp32).
//
// Forward: per row, the chunk's log-sum-exp in fp32 and its log-add into the running lse,
// plus the target logit when the target falls in the chunk -- what the reference does with
// logits.float(), logsumexp, logaddexp and a masked gather (with a host sync per chunk),
// here one read of the logits.  Backward: dlogits = g (exp(logit - lse) - onehot), written
// in the logits' dtype over the logits (the next GEMMs read it).
//
// HBM-bound: one wave per row; lane l reads 8-column chunks c = l + 64 i as 16-byte
// vectors.  A chunk of up to 4096 columns stays in the lane's registers: the row max
// first (a shuffle butterfly gives it to every lane), then one exp2 per element.  Wider
// chunks keep an online (max, sum) per lane, rescaled once per 8 columns, combined by the
// same butterfly.  exp and log are exp2 / log2 on the hardware units.
#include "mla_common.h"

namespace mla {

constexpr int kCeRegChunks = 8;  // rows up to 64 x 8 x 8 = 4096 columns stay in registers

struct CeParams {
  const void* logits;
  void* dlogits;
  const int64_t* targets;
  float* lse;
  float* tlogit;
  const float* g_vec;
  float g_scale;
  int N, Vc;
  int64_t v0, ld, ld_out;
};

// (m, s) with s = sum exp(x - m), combined with another such pair
__device__ __forceinline__ void lse_combine(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  const float a = m == -INFINITY ? 0.f : fast_exp2((m - mn) * kLog2e);
  const float b = m2 == -INFINITY ? 0.f : fast_exp2((m2 - mn) * kLog2e);
  s = s * a + s2 * b;
  m = mn;
}

// 8 consecutive logits of a row: one 16-byte load of bf16, or two of fp32
template <bool F32>
struct Logit8 {
  u32x4 a, b;
  __device__ __forceinline__ void load(const void* row, int c) {
    if constexpr (F32) {
      a = ldg16(static_cast<const float*>(row) + 8 * c);
      b = ldg16(static_cast<const float*>(row) + 8 * c + 4);
    } else {
      a = ldg16(static_cast<const bf16*>(row) + 8 * c);
    }
  }
  __device__ __forceinline__ void zero() { a = b = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ float get(int e) const {
    if constexpr (F32) return __uint_as_float(e < 4 ? a[e] : b[e - 4]);
    else return (e & 1) ? hi_bf16(a[e >> 1]) : lo_bf16(a[e >> 1]);
  }
};

template <bool F32>
__device__ __forceinline__ float logit_at(const void* row, int64_t j) {
  if constexpr (F32) return static_cast<const float*>(row)[j];
  else return bf16_bits_to_f32(static_cast<const uint16_t*>(row)[j]);
}

template <bool BWD, bool F32>
__global__ __launch_bounds__(256) void ce_chunk_kernel(CeParams p) {
  const int lane = threadIdx.x & 63;
  const int n_waves = gridDim.x * 4;
  const int nch = p.Vc >> 3;
  const int esz = F32 ? 4 : 2;
  for (int row = blockIdx.x * 4 + (threadIdx.x >> 6); row < p.N; row += n_waves) {
    const void* lr = static_cast<const char*>(p.logits) + (int64_t)row * p.ld * esz;
    const int64_t y = p.targets[row] - p.v0;  // the target's column in this chunk, if any
    if constexpr (!BWD) {
      float m = -INFINITY, s = 0.f;
      if (nch <= 64 * kCeRegChunks) {
        // the row fits the lane's registers: exact max first, then one exp2 per element
        Logit8<F32> v[kCeRegChunks];
#pragma unroll
        for (int i = 0; i < kCeRegChunks; ++i) {
          const int c = lane + 64 * i;
          if (c < nch) v[i].load(lr, c);
          else v[i].zero();
        }
#pragma unroll
        for (int i = 0; i < kCeRegChunks; ++i) {
          if (lane + 64 * i < nch) {
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, v[i].get(e));
          }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float mb = m * kLog2e;
#pragma unroll
        for (int i = 0; i < kCeRegChunks; ++i) {
          if (lane + 64 * i < nch) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s += fast_exp2(__builtin_fmaf(v[i].get(e), kLog2e, -mb));
          }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      } else for (int c = lane; c < nch; c += 64) {
        Logit8<F32> v;
        v.load(lr, c);
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = v.get(e);
        float cm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
        float cs = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) cs += fast_exp2((x[e] - cm) * kLog2e);
        lse_combine(m, s, cm, cs);
      }
      if (nch > 64 * kCeRegChunks) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
          lse_combine(m, s, m2, s2);
        }
      }
      if (lane == 0) {
        const float chunk_lse = m + fast_log2(s) * kLn2;
        const float old = p.lse[row];
        const float mx = fmaxf(old, chunk_lse);
        const float a = old == -INFINITY ? 0.f : fast_exp2((old - mx) * kLog2e);
        p.lse[row] = mx + fast_log2(a + fast_exp2((chunk_lse - mx) * kLog2e)) * kLn2;
        if (y >= 0 && y < p.Vc) p.tlogit[row] = logit_at<F32>(lr, y);
      }
    } else {
      const float lse = p.lse[row];
      const float g = p.g_scale * (p.g_vec ? p.g_vec[row] : 1.f);
      char* dr = static_cast<char*>(p.dlogits) + (int64_t)row * p.ld_out * esz;
      for (int c = lane; c < nch; c += 64) {
        Logit8<F32> v;
        v.load(lr, c);
        float d[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pr = fast_exp2((v.get(e) - lse) * kLog2e);
          d[e] = g * (8 * c + e == y ? pr - 1.f : pr);
        }
        if constexpr (F32) {
          float* o = reinterpret_cast<float*>(dr) + 8 * c;
          *reinterpret_cast<f32x4*>(o) = f32x4{d[0], d[1], d[2], d[3]};
          *reinterpret_cast<f32x4*>(o + 4) = f32x4{d[4], d[5], d[6], d[7]};
        } else {
          stg16(reinterpret_cast<bf16*>(dr) + 8 * c, u32x4{pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3]),
                                                           pack_bf16x2(d[4], d[5]), pack_bf16x2(d[6], d[7])});
        }
      }
    }
  }
}

}  // namespace mla

using namespace mla;

extern "C" int mla_ce_chunk(const mla_ce_chunk_args* a, void* stream) {
  const char* op = "mla_ce_chunk";
  MLA_CHECK(a, MLA_ERR_INVALID_ARG, "%s: null args", op);
  MLA_CHECK(a->N >= 0 && a->N < (1ll << 31) && a->Vc >= 0 && a->Vc < (1ll << 30), MLA_ERR_INVALID_ARG,
            "%s: size out of range", op);
  MLA_CHECK(a->Vc % 8 == 0, MLA_ERR_INVALID_ARG, "%s: the chunk width %lld must be a multiple of 8", op,
            (long long)a->Vc);
  MLA_CHECK(a->dtype == MLA_DTYPE_BF16 || a->dtype == MLA_DTYPE_F32, MLA_ERR_UNSUPPORTED, "%s: logits dtype %d", op,
            (int)a->dtype);
  if (a->N == 0 || a->Vc == 0) return MLA_OK;
  MLA_CHECK(a->logits && a->targets && a->lse && (a->backward ? a->dlogits != nullptr : a->tlogit != nullptr),
            MLA_ERR_INVALID_ARG, "%s: null pointer", op);
  MLA_CHECK(((uintptr_t)a->logits & 15) == 0 && (!a->backward || ((uintptr_t)a->dlogits & 15) == 0),
            MLA_ERR_INVALID_ARG, "%s: logits must be 16-byte aligned", op);
  MLA_CHECK(a->ld >= a->Vc && a->ld % 8 == 0 && (!a->backward || (a->ld_out >= a->Vc && a->ld_out % 8 == 0)),
            MLA_ERR_INVALID_ARG, "%s: row strides must cover Vc and be multiples of 8", op);
  CeParams p{a->logits, a->dlogits, a->targets, a->lse, a->tlogit, a->g_vec, a->g_scale,
             (int)a->N, (int)a->Vc, a->v0, a->ld, a->ld_out};
  const int grid = (int)std::min<int64_t>((a->N + 3) / 4, 4096);
  hipStream_t s = (hipStream_t)stream;
  const bool f32 = a->dtype == MLA_DTYPE_F32;
  if (a->backward) {
    if (f32) ce_chunk_kernel<true, true><<<grid, 256, 0, s>>>(p);
    else ce_chunk_kernel<true, false><<<grid, 256, 0, s>>>(p);
  } else {
    if (f32) ce_chunk_kernel<false, true><<<grid, 256, 0, s>>>(p);
    else ce_chunk_kernel<false, false><<<grid, 256, 0, s>>>(p);
  }
  return launch_status(op);
}
