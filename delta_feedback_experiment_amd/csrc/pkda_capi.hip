// Library identity and error reporting for the PKDA C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "pkda_common.h"

namespace pkda {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace pkda

extern "C" int pkda_abi_version(void) { return PKDA_ABI_VERSION; }

extern "C" const char* pkda_last_error(void) { return pkda::g_last_error; }

extern "C" int64_t pkda_args_size(int which) {
  switch (which) {
    case PKDA_ARGS_RECURRENT: return sizeof(pkda_recurrent_args);
    case PKDA_ARGS_GATE: return sizeof(pkda_gate_args);
    case PKDA_ARGS_PRECOND: return sizeof(pkda_precond_args);
    case PKDA_ARGS_CHUNK_FWD: return sizeof(pkda_chunk_fwd_args);
    case PKDA_ARGS_CHUNK_BWD: return sizeof(pkda_chunk_bwd_args);
    case PKDA_ARGS_QKV_CONV: return sizeof(pkda_qkv_conv_args);
    case PKDA_ARGS_NORM_GATE: return sizeof(pkda_norm_gate_args);
    case PKDA_ARGS_CONTROLS: return sizeof(pkda_controls_args);
    default: return -1;
  }
}
