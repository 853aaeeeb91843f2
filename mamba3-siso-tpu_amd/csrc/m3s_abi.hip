// Library identity, error reporting and capability queries of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "m3s_internal.h"

namespace m3s {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace m3s

extern "C" int32_t m3s_abi_version(void) { return M3S_ABI_VERSION; }

extern "C" const char* m3s_last_error(void) { return m3s::g_err; }

extern "C" int32_t m3s_supported(int32_t which, int32_t dtype, int32_t chunk, int32_t state_dim,
                                 int32_t headdim) {
  switch (which) {
    case 0: return m3s::fwd_supported(dtype, chunk, state_dim, headdim);
    case 1: return m3s::bwd_supported(dtype, chunk, state_dim, headdim);
    case 2: return m3s::decode_supported(dtype, state_dim, headdim);
    default: return 0;
  }
}

extern "C" int32_t m3s_fwd_raw_supported(int32_t dtype, int32_t chunk, int32_t state_dim,
                                         int32_t headdim, int32_t n_angles) {
  return m3s::fwd_raw_supported_impl(dtype, chunk, state_dim, headdim, n_angles);
}
