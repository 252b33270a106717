// Generator of tests/golden/mfma_f8_dot.npz: what v_mfma_f32_32x32x64_f8f6f4 and
// v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3, fp32 accumulator) return for given operands, called
// as the attention and GEMM kernels call them.  A [64][128] and B [64][128] e4m3 codes; wave (bi, bj) computes the 32x32 block
// C[32 bi + r][32 bj + c] = sum_k A[.][k] B[.][k], once over k < 64 (one instruction from a
// zero accumulator) and once over all 128 (a second instruction chained on the first).
// Operand bytes: lane l holds row l % 32 of its block, byte j <-> k = 64 h + 32 (l / 32) + j.
// Accumulator: value i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(64) mfma_f8_dot_probe(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
                                                        float* __restrict__ c1, float* __restrict__ c2) {
  const int bi = blockIdx.x >> 1, bj = blockIdx.x & 1, l = threadIdx.x;
  const int ra = 32 * bi + (l & 31), rb = 32 * bj + (l & 31);
  v8i fa[2], fb[2];
  for (int h = 0; h < 2; ++h)
    for (int d = 0; d < 8; ++d) {
      const int k = 64 * h + 32 * (l >> 5) + 4 * d;
      fa[h][d] = *reinterpret_cast<const int*>(a + ra * 128 + k);
      fb[h][d] = *reinterpret_cast<const int*>(b + rb * 128 + k);
    }
  v16f z;
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  const v16f s1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[0], fb[0], z, 0, 0, 0, 0, 0, 0);
  const v16f s2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[1], fb[1], s1, 0, 0, 0, 0, 0, 0);
  for (int i = 0; i < 16; ++i) {
    const int row = 32 * bi + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3), col = 32 * bj + (l & 31);
    c1[row * 64 + col] = s1[i];
    c2[row * 64 + col] = s2[i];
  }
}

// The 16x16x128 form: wave (bi, bj) of a 4 x 4 grid computes C16[16 bi + r][16 bj + c] over all
// 128 k in one instruction.  Operand bytes: lane l holds row l % 16 of its block, byte j <->
// k = 32 (l / 16) + j.  Accumulator: value i of lane l is row 4 (l / 16) + i, column l % 16.
__global__ void __launch_bounds__(64) mfma_f8_dot16_probe(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
                                                          float* __restrict__ c16) {
  const int bi = blockIdx.x >> 2, bj = blockIdx.x & 3, l = threadIdx.x;
  const int ra = 16 * bi + (l & 15), rb = 16 * bj + (l & 15);
  v8i fa, fb;
  for (int d = 0; d < 8; ++d) {
    const int k = 32 * (l >> 4) + 4 * d;
    fa[d] = *reinterpret_cast<const int*>(a + ra * 128 + k);
    fb[d] = *reinterpret_cast<const int*>(b + rb * 128 + k);
  }
  v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
  const v4f s = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fa, fb, z, 0, 0, 0, 0, 0, 0);
  for (int i = 0; i < 4; ++i) c16[(16 * bi + 4 * (l >> 4) + i) * 64 + 16 * bj + (l & 15)] = s[i];
}

// a, b: 64 x 128 codes; c1, c2: 64 x 64 fp32; c16: 64 x 64 fp32 (device pointers).  Returns the
// launch status.
extern "C" int mfma_f8_dot_probe_run(const void* a, const void* b, void* c1, void* c2, void* c16) {
  hipLaunchKernelGGL(mfma_f8_dot_probe, dim3(4), dim3(64), 0, 0, (const uint8_t*)a, (const uint8_t*)b, (float*)c1,
                     (float*)c2);
  hipLaunchKernelGGL(mfma_f8_dot16_probe, dim3(16), dim3(64), 0, 0, (const uint8_t*)a, (const uint8_t*)b,
                     (float*)c16);
  return (int)hipGetLastError();
}
