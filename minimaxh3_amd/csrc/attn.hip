// C entry point of the FP8 attention forward (kernels in attn_kernel.h).
#include "attn_kernel.h"

using namespace mxf8;

extern "C" int mxf8_attn_fwd(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t, const float* sq,
                             const float* sk, const float* sv, const uint8_t* key_mask, const float* key_bias,
                             float repair_tau, void* out, int out_dtype, const int64_t out_strides[4], int64_t B,
                             int64_t H, int64_t Sq, int64_t Sk, int64_t D, hipStream_t stream) {
  if (!q8 || !k8 || !v8t || !sq || !sk || !sv || !out || !out_strides)
    return set_error(MXF8_EINVAL, "attn_fwd: null pointer");
  if (D != 64 && D != 128) return set_error(MXF8_EINVAL, "attn_fwd: D must be 64 or 128");
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0) return set_error(MXF8_EINVAL, "attn_fwd: empty shape");
  if (cdiv(Sq, 128) * B * H >= ((int64_t)1 << 31)) return set_error(MXF8_EINVAL, "attn_fwd: too many Q tiles");
  if (out_dtype != MXF8_BF16 && out_dtype != MXF8_F16) return set_error(MXF8_EINVAL, "attn_fwd: out dtype");
  const int64_t Skp = cdiv(Sk, 128) * 128;
  if (Skp * D >= ((int64_t)1 << 31) || cdiv(Sq, 128) * 128 * D >= ((int64_t)1 << 31))
    return set_error(MXF8_EINVAL, "attn_fwd: sequence too long for one head (S*D must be < 2^31)");
  if (((uintptr_t)q8 % 16) || ((uintptr_t)k8 % 16) || ((uintptr_t)v8t % 16))
    return set_error(MXF8_EINVAL, "attn_fwd: FP8 operands must be 16-byte aligned");
  if (out_strides[3] == 1 && (((uintptr_t)out % 8) || (out_strides[0] % 4) || (out_strides[1] % 4) ||
                              (out_strides[2] % 4)))
    return set_error(MXF8_EINVAL, "attn_fwd: contiguous-channel output must be 8-byte aligned");
  const bool hm = key_mask != nullptr, hb = key_bias != nullptr, rep = repair_tau >= 0.0f;
  if (D == 128) {
    if (out_dtype == MXF8_BF16)
      attn_launch_128_0(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                        Sq, Sk, stream);
    else
      attn_launch_128_1(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                        Sq, Sk, stream);
  } else {
    if (out_dtype == MXF8_BF16)
      attn_launch_64_0(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                       Sq, Sk, stream);
    else
      attn_launch_64_1(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                       Sq, Sk, stream);
  }
  return check_launch("attn_fwd");
}
