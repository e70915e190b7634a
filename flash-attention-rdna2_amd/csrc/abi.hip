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
static_assert(offsetof(FableFwdParams, sQ) == 40, "FableFwdParams layout");
// the reference layouts (fa_iface.h:9-63 compiled for x86-64 / gfx950, both LP64)
static_assert(sizeof(FwdParams) == 256 && offsetof(FwdParams, sc_q) == 220 && offsetof(FwdParams, seqused_k) == 248,
              "FwdParams must match the reference layout");
static_assert(sizeof(BwdParams) == 368 && offsetof(BwdParams, shQ) == 352, "BwdParams must match the reference layout");
static_assert(sizeof(DecParams) == 192 && offsetof(DecParams, page_shift) == 104 && offsetof(DecParams, rotary_pos) == 184,
              "DecParams must match the reference layout");

extern "C" int fable_attn_abi_version(void) { return FABLE_ATTN_ABI_VERSION; }

extern "C" size_t fable_attn_struct_size(int which) {
  switch (which) {
    case 0: return sizeof(FableFwdParams);
    case 1: return sizeof(FableBwdParams);
    case 2: return sizeof(FableDecParams);
    case 3: return sizeof(CombineParams);
    case 4: return sizeof(fa_strides);
    case 5: return sizeof(FwdParams);
    case 6: return sizeof(BwdParams);
    case 7: return sizeof(DecParams);
    default: return 0;
  }
}

extern "C" const char* fable_attn_last_error(void) { return g_last_error; }
