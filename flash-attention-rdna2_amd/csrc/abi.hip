// abi.hip — library-wide entry points of the C-ABI: version, struct sizes, last error.
#include <string.h>

#include "attn_device.hpp"
#include "status.hpp"

static thread_local char g_last_error[512] = "";

namespace fa {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return FA_OK;
}

}  // namespace fa

static_assert(sizeof(fa_strides) == 24, "fa_strides layout");
static_assert(offsetof(FwdParams, sQ) == 40, "FwdParams layout");

extern "C" int fable_attn_abi_version(void) { return FABLE_ATTN_ABI_VERSION; }

extern "C" size_t fable_attn_struct_size(int which) {
  switch (which) {
    case 0: return sizeof(FwdParams);
    case 1: return sizeof(BwdParams);
    case 2: return sizeof(DecParams);
    case 3: return sizeof(CombineParams);
    case 4: return sizeof(fa_strides);
    default: return 0;
  }
}

extern "C" const char* fable_attn_last_error(void) { return g_last_error; }
