/*
 * mxf8.h - C ABI of the MI355X (gfx950) FP8 hot path: dynamic e4m3 quantizers, the
 * row-wise scaled FP8 GEMM with a fused epilogue, and the FP8 flash-attention forward.
 *
 * Conventions
 *  - Every pointer is a device pointer; every size, leading dimension and stride is in
 *    ELEMENTS (int64).  FP8 data is OCP float8 e4m3fn, one byte per element.
 *  - Every entry point launches asynchronously on `stream` (a hipStream_t; NULL is the
 *    legacy default stream), synchronises nothing, allocates nothing and caches no
 *    pointer between calls.  Scratch memory, where a kernel needs it, is passed in as
 *    `workspace` with the size reported by the matching *_workspace_bytes() function.
 *  - Return value: 0 on success; non-zero on an invalid argument (checked on the host
 *    before any launch) or a launch failure.  mxf8_last_error() then describes the
 *    problem (thread-local; valid until the next call on the same thread).
 */
#ifndef MXF8_H_
#define MXF8_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of floating-point inputs / outputs */
enum { MXF8_BF16 = 0, MXF8_F16 = 1, MXF8_F32 = 2 };
/* GEMM epilogue activation */
enum { MXF8_ACT_NONE = 0, MXF8_ACT_GELU_TANH = 1 };
/* status codes */
enum { MXF8_OK = 0, MXF8_EINVAL = 1, MXF8_ELAUNCH = 2 };
/* kv_mode of the attention forward: AUTO holds each head's K/V in LDS when they fit, STREAM
 * always streams K/V tiles (same bits either way) */
enum { MXF8_ATTN_KV_AUTO = 0, MXF8_ATTN_KV_STREAM = 1 };

/* Version of this ABI (major * 100 + minor). */
int mxf8_abi_version(void);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* mxf8_last_error(void);

/*
 * Per-row dynamic e4m3 quantization.
 * Replaces _quantize_rows_kernel + quantize_rows (kernels/fp8_linear.py:8-42), used for
 * activations in FP8Linear.forward (fp8_linear.py:94) and weights in
 * FP8Linear.from_linear (fp8_linear.py:72).
 *   x      [M, K] of `dtype` with row stride ldx (ldx >= K)
 *   x8     [M, K] e4m3 codes, row stride K (written)
 *   scale  [M] fp32 (written): scale = max(max_k |x|, 1e-12) / 448
 *   x8 = e4m3(clamp(x / scale, -448, 448)), IEEE fp32 division, round to nearest even.
 * M == 0 or K == 0 launches nothing (K == 0 with M > 0 writes scale = 1e-12/448).
 */
int mxf8_quant_rows(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx,
                    uint8_t* x8, float* scale, hipStream_t stream);

/*
 * adaLN modulation fused with the per-row quantizer.  No counterpart in the reference's
 * files: it fuses the DiT block's pre-linear adaLN (diffusers, outside the reference) with
 * the activation quantization of FP8Linear.forward (kernels/fp8_linear.py:94).
 *   x      [M, C] bf16, row stride ldx; rows of batch item b are [b S, (b + 1) S)
 *   shift, scale  [ceil(M / S), C] bf16, row stride ldm (one row per batch item)
 *   n = (x - mean) * rstd   (fp32 row mean, biased variance, rstd = 1 / sqrt(var + eps))
 *   eager == 0: y = bf16(n * (1 + scale[b]) + shift[b])       (fp32, one rounding)
 *   eager != 0: y = bf16(bf16(bf16(n) * bf16(1 + scale[b])) + shift[b])   (torch eager bf16)
 *   x8 [M, C] e4m3 and sa [M] fp32 = quant_rows(y) (written); y [M, C] bf16 (written when
 *   not NULL, row stride C).
 * Requires C % 8 == 0, C <= 8192, ldx and ldm multiples of 8, 16-byte aligned operands.
 */
int mxf8_adaln_quant_rows(const void* x, int64_t M, int64_t C, int64_t ldx, int64_t S,
                          const void* shift, const void* scale, int64_t ldm, float eps, int eager,
                          uint8_t* x8, float* sa, void* y, hipStream_t stream);

/*
 * Row-wise scaled FP8 GEMM with fused epilogue.
 * Replaces torch._scaled_mm(x8, w8.t(), scale_a, scale_b, bias, out_dtype=bf16)
 * (kernels/fp8_linear.py:95-102), the un-padding slice (105-106), the LoRA adds of
 * apply_lora_adapters (45-55) and the tanh-GELU that follows the FFN up-projection.
 *   a8   [M, K] e4m3 row-major (activations), w8 [N, K] e4m3 row-major (weights)
 *   sa   [M] fp32 per-token scales, sw [N] fp32 per-channel scales
 *   bias [N] bf16 or NULL
 *   out  [M, N] bf16, row stride ld_out (>= N)
 *   o = bf16(sum_k a8[m,k] w8[n,k] * sa[m] * sw[n] + bias[n])          (fp32 accumulate)
 *   with lora_t != NULL (one adapter, rank r): lora_t [M, r] bf16 = bf16(x A^T),
 *   lora_b [N, r] bf16 = B:   o = bf16(o + bf16(bf16(sum_j lora_t[m,j] lora_b[n,j]) * lora_scale))
 *   act == MXF8_ACT_GELU_TANH: o = bf16(gelu_tanh(o)) after the LoRA add.
 * Requires K % 16 == 0 (the reference converts only linears with in/out % 16 == 0,
 * fp8_linear.py:146), K <= 2^22, and r % 16 == 0 (r <= 4096) when a LoRA is given.
 */
int mxf8_gemm_rowwise(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                      const void* bias, int act,
                      const void* lora_t, const void* lora_b, int64_t r, float lora_scale,
                      void* out, int64_t M, int64_t N, int64_t K, int64_t ld_out,
                      hipStream_t stream);

/* Bytes of the K/V column statistics that mxf8_gemm_rowwise_kv_stats writes for M rows and
 * C columns per part: 2 statistics x ceil(M/128) blocks x C fp32. */
int64_t mxf8_gemm_kv_stats_bytes(int64_t M, int64_t C);

/*
 * mxf8_gemm_rowwise (no LoRA, no activation) of a fused QKV projection that also emits the
 * column statistics of its key and value parts, so that the attention's K/V quantizers
 * read K and V once.  Replaces k.float().mean(dim=2) (kernels/fp8_attention.py:338) and the
 * first pass of _quantize_v_kernel (122-155, the per-channel |max| over the sequence),
 * taken over the bf16 outputs as they are stored.
 *   out [M, N] bf16 is mxf8_gemm_rowwise's output bit for bit; rows of batch item b are
 *   [b S, (b + 1) S) (M % S == 0, S >= 128).
 *   Key columns [k_col0, k_col0 + C) (k_col0 < 0: none): per-channel sums; value columns
 *   [v_col0, v_col0 + C) (v_col0 < 0: none): per-channel |max| (NaN skipped).
 *   part (written, mxf8_gemm_kv_stats_bytes(M, C) bytes): [2][ceil(M/128)][C] fp32, the
 *   statistic of each 128-row block p that lies inside one batch item; the blocks holding an
 *   item boundary or row M are not written (mxf8_attn_quant_kv_gemm_stats reads their rows).
 *   Fixed order.
 * Requires N % 256 == 0, ld_out % 8 == 0 (ld_out >= N), 16-byte aligned out, a8, w8 and
 * part, C % 256 == 0, column ranges starting at multiples of 256 inside [0, N), K % 16 == 0.
 */
int mxf8_gemm_rowwise_kv_stats(const uint8_t* a8, const uint8_t* w8, const float* sa, const float* sw,
                               const void* bias, void* out, int64_t M, int64_t N, int64_t K, int64_t ld_out,
                               int64_t S, int64_t k_col0, int64_t v_col0, int64_t C, float* part,
                               hipStream_t stream);

/*
 * LoRA down-projection t = bf16(x A^T) used by the LoRA epilogue (the first matmul of
 * apply_lora_adapters, kernels/fp8_linear.py:53).
 *   x [M, K] bf16 (row stride ldx >= K), a [r, K] bf16 row-major, t [M, r] bf16 (written).
 * Requires r % 16 == 0 (r <= 4096), K % 8 == 0 and ldx % 8 == 0.
 */
int mxf8_lora_down(const void* x, int64_t ldx, const void* a, void* t,
                   int64_t M, int64_t K, int64_t r, hipStream_t stream);

/*
 * Attention tensors.  q/k/v are [B, H, S, D] of `dtype` (bf16 or fp16) with arbitrary
 * element strides strides[4] = {b, h, s, d}; D is 64 or 128.
 * Internal FP8 layouts (all written by the quantizers, read by mxf8_attn_fwd):
 *   q8  [B, H, Sqp, D]   Sqp = ceil(Sq/128)*128, rows >= Sq are zero
 *   k8  [B, H, Skp, D]   Skp = ceil(Sk/128)*128, rows >= Sk are zero
 *   v8t [B, H, D, Skp]   V transposed, columns >= Sk are zero
 *   sq  [B, H, ceil(Sq/128)], sk [B, H, ceil(Sk/128)], sv [B, H, D]  fp32
 */

/* Scratch bytes needed by mxf8_attn_kmean / mxf8_attn_quant_v (and mxf8_attn_prepare). */
int64_t mxf8_attn_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D);

/*
 * Q quantizer.  Replaces _quantize_q_kernel (kernels/fp8_attention.py:39-77, launch 321-336).
 *   q~ = fp32(q) * c  (c = softmax scale * log2(e)), per (b, h, 128-row block):
 *   sq = max(max|q~|, 1e-12) / 448, q8 = e4m3(clamp(q~ / sq)).
 */
int mxf8_attn_quant_q(const void* q, int dtype, const int64_t strides[4],
                      int64_t B, int64_t H, int64_t S, int64_t D, float c,
                      uint8_t* q8, float* sq, hipStream_t stream);

/*
 * Key mean over the sequence axis in fp32.  Replaces k.float().mean(dim=2, keepdim=True)
 * (kernels/fp8_attention.py:338).  mean [B, H, D] fp32 (written).  Deterministic
 * (fixed reduction order); needs `workspace`.
 */
int mxf8_attn_kmean(const void* k, int dtype, const int64_t strides[4],
                    int64_t B, int64_t H, int64_t S, int64_t D,
                    float* mean, void* workspace, hipStream_t stream);

/*
 * K quantizer.  Replaces _quantize_k_kernel (kernels/fp8_attention.py:80-119, launch 339-354).
 *   k~ = fp32(k) - mean, per (b, h, 128-key block): sk = max(max|k~|, 1e-12) / 448,
 *   k8 = e4m3(clamp(k~ / sk)).  mean [B, H, D] fp32 (from mxf8_attn_kmean or the caller).
 */
int mxf8_attn_quant_k(const void* k, int dtype, const int64_t strides[4], const float* mean,
                      int64_t B, int64_t H, int64_t S, int64_t D,
                      uint8_t* k8, float* sk, hipStream_t stream);

/*
 * V quantizer.  Replaces _quantize_v_kernel (kernels/fp8_attention.py:122-170, launch 356-369).
 *   sv[b,h,d] = max(max_s |v|, 1e-12) / 448, v8t[b,h,d,s] = e4m3(clamp(v / sv)).  Needs `workspace`.
 */
int mxf8_attn_quant_v(const void* v, int dtype, const int64_t strides[4],
                      int64_t B, int64_t H, int64_t S, int64_t D,
                      uint8_t* v8t, float* sv, void* workspace, hipStream_t stream);

/* Scratch bytes needed by mxf8_attn_quant_kv. */
int64_t mxf8_attn_kv_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D);

/*
 * K and V quantizers together.  Replaces k.float().mean(dim=2) (kernels/fp8_attention.py:338),
 * _quantize_k_kernel (80-119, launch 339-354) and _quantize_v_kernel (122-170, launch
 * 356-369) of one attention call: the same outputs as mxf8_attn_kmean + mxf8_attn_quant_k +
 * mxf8_attn_quant_v, in three launches (one pass over K and V for the key mean and the
 * per-channel V amax, one fold of both, one pass that quantizes K and V).
 *   k, v [B, H, S, D] of `dtype` with element strides k_strides[4], v_strides[4]
 *   k8 [B, H, Skp, D], sk [B, H, ceil(S/128)], v8t [B, H, D, Skp], sv [B, H, D] (written)
 *   mean [B, H, D] fp32 key mean (written when not NULL; kept in `workspace` otherwise)
 *   workspace: mxf8_attn_kv_workspace_bytes(B, H, S, D) bytes.  Deterministic.
 */
int mxf8_attn_quant_kv(const void* k, const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
                       int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                       uint8_t* k8, float* sk, uint8_t* v8t, float* sv, float* mean, void* workspace,
                       hipStream_t stream);

/*
 * K and V quantizers fed by the QKV projection's column statistics: the key mean
 * (kernels/fp8_attention.py:338), _quantize_k_kernel (80-119) and _quantize_v_kernel
 * (122-170) of one attention call whose k and v are views of the output of
 * mxf8_gemm_rowwise_kv_stats (rows b S + s, key / value columns h D + d of its parts).  One
 * fold launch turns `part` (and the rows of the blocks it leaves out, at most two per batch
 * item) into the key mean and the V scales, one pass quantizes K and V: K and V are read
 * once.
 *   part: the statistics written by mxf8_gemm_rowwise_kv_stats (M = B S, C = H D).
 *   key_stats != 0: the key mean comes from part's key sums (mean written); key_stats == 0:
 *   `mean` [B, H, D] fp32 is an input (e.g. mxf8_attn_kmean of keys transformed after the
 *   projection), and only the V statistics are taken from part.
 *   Other arguments and outputs as mxf8_attn_quant_kv; requires S >= 128, (H D) % 256 == 0.
 */
int mxf8_attn_quant_kv_gemm_stats(const void* k, const int64_t k_strides[4], const void* v,
                                  const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S,
                                  int64_t D, const float* part, int key_stats, uint8_t* k8, float* sk,
                                  uint8_t* v8t, float* sv, float* mean, hipStream_t stream);

/*
 * mxf8_attn_quant_kv without a workspace argument and without any device allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its scratch is a 4 MiB device array inside the library (one copy per GPU, held until the
 * process ends), enough for every B*H <= 1638 at D = 128 (<= 5461 at D = 64); larger shapes
 * are rejected with MXF8_EINVAL before any launch.  Every call on one GPU shares that
 * GPU's copy, so calls must not overlap on one GPU.  Outside graph capture the entry point
 * orders them itself: a call on another stream than the previous call waits for that call's
 * event (hipStreamWaitEvent on an event created with the first call on the device), and calls
 * from several threads are serialized.  Calls captured into a HIP graph are not ordered by the
 * library: replays of such a graph must not overlap other calls on the GPU.  Outputs are
 * those of mxf8_attn_quant_kv bit for bit.
 */
int mxf8_attn_quant_kv_noalloc(const void* k, const int64_t k_strides[4], const void* v,
                               const int64_t v_strides[4], int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                               uint8_t* k8, float* sk, uint8_t* v8t, float* sv, float* mean, hipStream_t stream);

/*
 * FP8 flash-attention forward.  Replaces _fp8_attn_kernel (kernels/fp8_attention.py:185-297,
 * launch 380-402) with BLOCK_N = 128: log2-domain scores, staggered KV visit order, lazy
 * row max (moves only when the tile max exceeds it by more than 8), exp2-free e4m3 P codes,
 * optional exact repair of codes >= repair_tau (repair_tau < 0 disables it).
 *   key_mask [B, Sk] uint8 (nonzero = keep) or NULL; key_bias [B, Sk] fp32 natural-log
 *   additive bias or NULL (entries <= -1e8 mask the key).
 *   out [B, H, Sq, D] of out_dtype (bf16/fp16) with element strides out_strides[4].
 *   Fully masked rows give 0.  kv_mode MXF8_ATTN_KV_AUTO: short key sequences (Sk <= 512
 *   at D = 128, <= 1024 at D = 64) without repair run a kernel that holds each head's K/V
 *   in LDS; MXF8_ATTN_KV_STREAM always streams K/V tiles.  Both give the same bits.
 */
int mxf8_attn_fwd(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8t,
                  const float* sq, const float* sk, const float* sv,
                  const uint8_t* key_mask, const float* key_bias, float repair_tau,
                  void* out, int out_dtype, const int64_t out_strides[4],
                  int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                  int kv_mode, hipStream_t stream);

/*
 * Q quantizer fused into the attention forward: _quantize_q_kernel + _fp8_attn_kernel
 * (kernels/fp8_attention.py:39-77 and 185-297, launches 321-336 and 380-402) in one launch.
 * Each workgroup quantizes its own (b, h, 128-row) Q block with the arithmetic of
 * mxf8_attn_quant_q, so the result equals mxf8_attn_quant_q followed by mxf8_attn_fwd bit
 * for bit, without the q8 round trip through memory.
 *   q [B, H, Sq, D] 16-bit, of out_dtype, element strides q_strides[4]: q_strides[3] == 1,
 *   the other three multiples of 8, q 16-byte aligned (other layouts: the two-call path).
 *   c = softmax scale * log2(e); sq_out [B, H, ceil(Sq/128)] fp32 receives the Q scales
 *   (NULL: not written).  Other arguments as mxf8_attn_fwd.
 */
int mxf8_attn_fwd_q(const void* q, const int64_t q_strides[4], float c,
                    const uint8_t* k8, const uint8_t* v8t, const float* sk, const float* sv,
                    const uint8_t* key_mask, const float* key_bias, float repair_tau,
                    float* sq_out, void* out, int out_dtype, const int64_t out_strides[4],
                    int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                    int kv_mode, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MXF8_H_ */
