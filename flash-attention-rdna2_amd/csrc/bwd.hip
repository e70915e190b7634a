// bwd.hip — backward entry point (kernels land in a following change).
#include "attn_device.hpp"
#include "status.hpp"

extern "C" int fable_attn_backward_launch(BwdParams p, int dtype, void* stream) {
  (void)p; (void)dtype; (void)stream;
  return fa::fail(FA_ERR_UNSUPPORTED, "fable_attn_backward_launch: not implemented yet");
}
