// ref_drop.cpp — exports the reference's host replica of its dropout multiplier (hdrop,
// kernels/backward.hip:530-537, the host twin of dropout_mul in kernels/fa_common.hpp:71-88),
// so the Philox stream and keep rule of oracle.c can be checked against it bit for bit.
// TEST INFRASTRUCTURE ONLY. backward.hip is included from where it lies under the read-only
// reference tree (include path from oracle/Makefile) with its standalone gate enabled, whose
// entry point is renamed so it does not clash; nothing from the reference is copied here.
#define FA_STANDALONE
#define main fa_reference_backward_gate_main
#include "backward.hip"
#undef main

extern "C" float ref_drop_mul(unsigned long long seed, unsigned long long idx, float p, float keep_scale) {
  return hdrop(seed, idx, p, keep_scale);
}
