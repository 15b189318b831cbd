// RMSNorm's canonical inverse RMS of one row, for kernels that normalise
// their input while staging it (the router chunks and the gate/up product of
// moe_block) instead of reading a normalised copy from memory.
//
// Reference: src/core/kernels/reduce/rmsNorm.ts:84-140 (f32 sums, then
// v = x·inv·w stored in the input dtype). The order is norm.hip's canonical
// one, so a fused kernel sees the same bits the standalone norm writes:
// lane l sums the quads q ≡ l (mod 64) of the row in ascending q, each
// quad's elements in ascending order (s = s + x·x, no fused multiply-add:
// including files are compiled with -ffp-contract=off); the 64 lane sums
// meet in an xor butterfly, strides 32 … 1; inv = 1 / sqrt(s / n + eps).
#pragma once
#include "moe_internal.h"

namespace moe_dev {

template <typename T>
__device__ __forceinline__ float wave_row_inv(const T *x, int n, float eps, int lane) {
  float s = 0.f;
  for (int q = lane; 4 * q < n; q += 64) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = 4 * q + j;
      if (i < n) {
        const float v = (float)x[i];
        s = s + v * v;
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s = s + __shfl_xor(s, m);
  return 1.0f / sqrtf(s / (float)n + eps);
}

// One element of x's dtype through a raw buffer load, as f32 (0 for an
// offset past the buffer).
template <typename T>
__device__ __forceinline__ float buf_elem(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <>
__device__ __forceinline__ float buf_elem<float>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
template <>
__device__ __forceinline__ float buf_elem<_Float16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}

// wave_row_inv of NB rows (row b at x + b·stride, 1 ≤ count ≤ NB rows
// valid) with every load issued before the first sum: one memory latency
// for the NB rows instead of NB. The lane's quads q = lane + 64m (m < QM,
// rows of at most 256·QM elements) are raw buffer loads whose offset is out
// of range (the load returns 0) past n or count: no branch, so the loads
// stay together (a load under a branch makes the compiler wait for it at
// the join). A zero term adds +0 to a sum that is ≥ +0, so the sums, the
// butterfly and inv are wave_row_inv's bit for bit.
template <typename T, int NB, int QM>
__device__ __forceinline__ void wave_rows_inv(const T *x, int64_t stride, int count, int n, float eps,
                                              int lane, float (&inv)[NB]) {
  const uint32_t bytes = (uint32_t)(((int64_t)(count - 1) * stride + n) * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (int)bytes, 0x00020000 /* raw, 32-bit */);
  float v[NB][QM][4];
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int m = 0; m < QM; m++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = 4 * (lane + 64 * m) + j;
        const uint32_t off = (b < count && i < n)
                                 ? (uint32_t)(((int64_t)b * stride + i) * (int64_t)sizeof(T))
                                 : 0x80000000u;
        v[b][m][j] = buf_elem<T>(r, off);
      }
#pragma unroll
  for (int b = 0; b < NB; b++) {
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < QM; m++)
#pragma unroll
      for (int j = 0; j < 4; j++) s = s + v[b][m][j] * v[b][m][j];
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) s = s + __shfl_xor(s, msk);
    inv[b] = 1.0f / sqrtf(s / (float)n + eps);
  }
}

// The normalised value as the standalone norm stores it: x·inv·w in f32,
// left to right, rounded to the input dtype. The f32 product is rounded
// before the conversion: the empty asm keeps the compiler from merging the
// last multiply and the conversion to f16 into one mixed-precision fma
// (v_fma_mixlo_f16), which rounds once and so differs in the last f16 bit.
template <typename T>
__device__ __forceinline__ float norm_value(float x, float inv, float w) {
  float v = x * inv * w;
  __asm__ volatile("" : "+v"(v));
  return (float)(T)v;
}

}  // namespace moe_dev
