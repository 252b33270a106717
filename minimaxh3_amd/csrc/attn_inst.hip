// Instantiates the FP8 attention kernels for one (head dim, output dtype) pair; the
// build compiles this file once per pair with MXF8_ATTN_D / MXF8_ATTN_ODT defined.
#include "attn_kernel.h"

#ifndef MXF8_ATTN_D
#error "MXF8_ATTN_D must be defined (64 or 128)"
#endif
#ifndef MXF8_ATTN_ODT
#error "MXF8_ATTN_ODT must be defined (0 = bf16, 1 = fp16)"
#endif


// expand the two defines before MXF8_ATTN_DECL pastes them into the function name
#define MXF8_ATTN_DECL_X(d, o) MXF8_ATTN_DECL(d, o)

namespace mxf8 {
MXF8_ATTN_DECL_X(MXF8_ATTN_D, MXF8_ATTN_ODT) {
  attn_dispatch_flags<MXF8_ATTN_D, MXF8_ATTN_ODT>(hm, hb, rep, q8, k8, v8t, sq, sk, sv, km, kb, tau, out, os, B, H, Sq,
                                                   Sk, qa, kv_mode, st);
}
}  // namespace mxf8
