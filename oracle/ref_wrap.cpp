// ref_wrap.cpp — exports the reference's own fp64 forward oracle (ref_attention,
// kernels/fa_common.hpp:93-134) from a host-only shared library, so the restatement in
// oracle.c can be checked against it on identical inputs. TEST INFRASTRUCTURE ONLY.
// The header is included from where it lies under the read-only reference tree (the include
// path is given by oracle/Makefile); nothing from the reference is copied into this repository.
#include "fa_common.hpp"

extern "C" void ref_fwd(const float* Q, const float* K, const float* V, float* O, float* LSE,
                        int SQ, int SK, int HD, int NH, int gqa, float scale, float softcap,
                        int win_left, int win_right, int causal, const float* alibi_slopes,
                        int attn_chunk) {
  RefCfg c{SQ, SK, HD, NH, gqa, scale, softcap, win_left, win_right, causal != 0,
           alibi_slopes != nullptr, alibi_slopes, attn_chunk};
  ref_attention(Q, K, V, O, LSE, c);
}
