// Error reporting and version of the C ABI (include/xenc_hip.h).
#include "xenc_common.h"

namespace xenc {
static thread_local int g_last_hip_error = 0;
void set_hip_error(hipError_t e) { g_last_hip_error = static_cast<int>(e); }
}  // namespace xenc

extern "C" const char* xenc_strerror(int code) {
  switch (code) {
    case XENC_OK: return "ok";
    case XENC_EINVAL: return "invalid size or argument";
    case XENC_ENULL: return "required pointer is NULL";
    case XENC_EALIGN: return "pointer or stride is not 16-byte aligned";
    case XENC_EWORKSPACE: return "workspace is smaller than the size query returned";
    case XENC_EHIP: return "HIP kernel launch failed";
    case XENC_ESCRATCH: return "the call needs more than the fixed scratch of the allocation-free entry point";
    default: return "unknown error code";
  }
}

extern "C" int xenc_last_hip_error(void) { return xenc::g_last_hip_error; }

extern "C" int xenc_abi_version(void) { return 18; }
