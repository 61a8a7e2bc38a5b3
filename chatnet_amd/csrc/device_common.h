// device_common.h — helpers shared by the gfx950 kernels of libchatnet_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t cn_u32x4 __attribute__((ext_vector_type(4)));

#define CN_WAVE 64
#define CN_BLOCK 256

// Exact IEEE binary16 -> binary32 (v_cvt_f32_f16 keeps f16 subnormals; the
// reference's System.Half conversion, DequantQ4_0.cs:190-194, is exact too).
__device__ __forceinline__ float cn_h2f(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
  return (float)h;
}

// Byte `b` (compile-time) of a dword as float: v_cvt_f32_ubyte{0..3}.
template <int B>
__device__ __forceinline__ float cn_ubyte(uint32_t v) {
  return (float)((v >> (8 * B)) & 0xFFu);
}

__device__ __forceinline__ float cn_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, CN_WAVE);
  return v;
}

__device__ __forceinline__ float cn_wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, CN_WAVE));
  return v;
}

// Sum over a 256-thread block; every thread gets the result.  `red` needs 4 floats.
__device__ __forceinline__ float cn_block_sum(float v, float* red) {
  v = cn_wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0] + red[1] + red[2] + red[3];
  return t;
}

__device__ __forceinline__ float cn_block_max(float v, float* red) {
  v = cn_wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
