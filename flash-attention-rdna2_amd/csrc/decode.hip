// decode.hip — paged decode entry points (kernels land in a following change).
#include "attn_device.hpp"
#include "status.hpp"

extern "C" int fa_decode_num_splits(int batch, int nq, int NH, int gqa, int64_t ctx_bound, int hint) {
  (void)batch; (void)nq; (void)NH; (void)gqa; (void)ctx_bound;
  return hint > 0 ? hint : 1;
}

extern "C" int fa_decode_launch(DecParams p, int dtype, void* stream, const void* nk, const void* nv) {
  (void)p; (void)dtype; (void)stream; (void)nk; (void)nv;
  return fa::fail(FA_ERR_UNSUPPORTED, "fa_decode_launch: not implemented yet");
}
