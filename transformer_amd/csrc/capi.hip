// C-ABI bookkeeping shared by all entry points: thread-local error text,
// launch status, ABI introspection.
#include <stdarg.h>
#include <stdio.h>

#include <cmath>

#include "mla_common.h"

namespace mla {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MLA_ERR_LAUNCH;
  }
  return MLA_OK;
}

// shared host-side validation for the [B, T, heads, dim] bf16 operands
int check_operand(const char* op, const char* name, const void* ptr, const mla_strides& st) {
  MLA_CHECK(ptr, MLA_ERR_INVALID_ARG, "%s: %s is null", op, name);
  MLA_CHECK(((uintptr_t)ptr & 15) == 0, MLA_ERR_INVALID_ARG, "%s: %s must be 16-byte aligned", op, name);
  MLA_CHECK((st.b & 7) == 0 && (st.t & 7) == 0 && (st.h & 7) == 0, MLA_ERR_INVALID_ARG,
            "%s: %s strides (%lld, %lld, %lld) must be multiples of 8 elements", op, name, (long long)st.b,
            (long long)st.t, (long long)st.h);
  MLA_CHECK(st.b >= 0 && st.t >= 0 && st.h >= 0, MLA_ERR_INVALID_ARG, "%s: %s has negative strides", op, name);
  return MLA_OK;
}

int check_scale(const char* op, float scale) {
  MLA_CHECK(std::isfinite(scale) && scale > 0.f && std::isfinite(scale * kLog2e), MLA_ERR_INVALID_ARG,
            "%s: scale must be finite and positive (got %g)", op, (double)scale);
  return MLA_OK;
}

}  // namespace mla

extern "C" const char* mla_last_error(void) { return mla::g_err; }

extern "C" int mla_abi_version(void) { return MLA_ABI_VERSION; }

extern "C" size_t mla_args_size(int which) {
  switch (which) {
    case 0: return sizeof(mla_rope_args);
    case 1: return sizeof(mla_prefill_fwd_args);
    case 2: return sizeof(mla_prefill_bwd_args);
    case 3: return sizeof(mla_decode_args);
    case 4: return sizeof(mla_rmsnorm_args);
    case 5: return sizeof(mla_rmsnorm_bwd_args);
    case 6: return sizeof(mla_decode_out_args);
    case 7: return sizeof(mla_rope_append_args);
    case 8: return sizeof(mla_absorb_q_args);
    case 9: return sizeof(mla_ce_chunk_args);
    case 10: return sizeof(mla_linear_rows_args);
    case 11: return sizeof(mla_prefill_cached_args);
    case 12: return sizeof(mla_norm_linear_args);
    default: return 0;
  }
}
