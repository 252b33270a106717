// C entry points of the FP8 attention forward (kernels in attn_kernel.h).
#include "attn_kernel.h"

using namespace mxf8;

// Checks shared by both entry points, then the launch; qa == nullptr reads q8 / sq.
static int attn_fwd_common(const char* name, const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t,
                           const float* sq, const float* sk, const float* sv, const uint8_t* key_mask,
                           const float* key_bias, float repair_tau, void* out, int out_dtype,
                           const int64_t out_strides[4], int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                           const AttnQ16* qa, int kv_mode, hipStream_t stream) {
  if (!k8 || !v8t || !sk || !sv || !out || !out_strides) return set_error(MXF8_EINVAL, "%s: null pointer", name);
  if (D != 64 && D != 128) return set_error(MXF8_EINVAL, "%s: D must be 64 or 128", name);
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0) return set_error(MXF8_EINVAL, "%s: empty shape", name);
  if (cdiv(Sq, 128) * B * H >= ((int64_t)1 << 31)) return set_error(MXF8_EINVAL, "%s: too many Q tiles", name);
  if (out_dtype != MXF8_BF16 && out_dtype != MXF8_F16) return set_error(MXF8_EINVAL, "%s: out dtype", name);
  if (kv_mode != MXF8_ATTN_KV_AUTO && kv_mode != MXF8_ATTN_KV_STREAM) return set_error(MXF8_EINVAL, "%s: kv_mode", name);
  const int64_t Skp = cdiv(Sk, 128) * 128;
  if (Skp * D >= ((int64_t)1 << 31) || cdiv(Sq, 128) * 128 * D >= ((int64_t)1 << 31))
    return set_error(MXF8_EINVAL, "%s: sequence too long for one head (S*D must be < 2^31)", name);
  if ((q8 && ((uintptr_t)q8 % 16)) || ((uintptr_t)k8 % 16) || ((uintptr_t)v8t % 16))
    return set_error(MXF8_EINVAL, "%s: FP8 operands must be 16-byte aligned", name);
  if (out_strides[3] == 1 && (((uintptr_t)out % 8) || (out_strides[0] % 4) || (out_strides[1] % 4) ||
                              (out_strides[2] % 4)))
    return set_error(MXF8_EINVAL, "%s: contiguous-channel output must be 8-byte aligned", name);
  const bool hm = key_mask != nullptr, hb = key_bias != nullptr, rep = repair_tau >= 0.0f;
  if (D == 128) {
    if (out_dtype == MXF8_BF16)
      attn_launch_128_0(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                        Sq, Sk, qa, kv_mode, stream);
    else
      attn_launch_128_1(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                        Sq, Sk, qa, kv_mode, stream);
  } else {
    if (out_dtype == MXF8_BF16)
      attn_launch_64_0(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                       Sq, Sk, qa, kv_mode, stream);
    else
      attn_launch_64_1(hm, hb, rep, q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_strides, B, H,
                       Sq, Sk, qa, kv_mode, stream);
  }
  return check_launch(name);
}

extern "C" int mxf8_attn_fwd(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t, const float* sq,
                             const float* sk, const float* sv, const uint8_t* key_mask, const float* key_bias,
                             float repair_tau, void* out, int out_dtype, const int64_t out_strides[4], int64_t B,
                             int64_t H, int64_t Sq, int64_t Sk, int64_t D, int kv_mode, hipStream_t stream) {
  if (!q8 || !sq) return set_error(MXF8_EINVAL, "attn_fwd: null pointer");
  return attn_fwd_common("attn_fwd", q8, k8, v8t, sq, sk, sv, key_mask, key_bias, repair_tau, out, out_dtype,
                         out_strides, B, H, Sq, Sk, D, nullptr, kv_mode, stream);
}

extern "C" int mxf8_attn_fwd_q(const void* q, const int64_t q_strides[4], float c, const uint8_t* k8,
                               const uint8_t* v8t, const float* sk, const float* sv, const uint8_t* key_mask,
                               const float* key_bias, float repair_tau, float* sq_out, void* out, int out_dtype,
                               const int64_t out_strides[4], int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                               int64_t D, int kv_mode, hipStream_t stream) {
  if (!q || !q_strides) return set_error(MXF8_EINVAL, "attn_fwd_q: null pointer");
  if (q_strides[3] != 1 || (q_strides[0] % 8) || (q_strides[1] % 8) || (q_strides[2] % 8) || ((uintptr_t)q % 16))
    return set_error(MXF8_EINVAL,
                     "attn_fwd_q: q needs unit channel stride, 16-byte alignment and strides that are multiples of 8 "
                     "elements (quantize with mxf8_attn_quant_q and call mxf8_attn_fwd otherwise)");
  const AttnQ16 qa{static_cast<const uint16_t*>(q), q_strides[0], q_strides[1], q_strides[2], c, sq_out};
  return attn_fwd_common("attn_fwd_q", nullptr, k8, v8t, nullptr, sk, sv, key_mask, key_bias, repair_tau, out,
                         out_dtype, out_strides, B, H, Sq, Sk, D, &qa, kv_mode, stream);
}
