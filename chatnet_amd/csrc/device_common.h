// device_common.h — helpers shared by the gfx950 kernels of libchatnet_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t cn_u32x4 __attribute__((ext_vector_type(4)));

// Global-memory address space.  A pointer rebuilt from integers (a segment
// chosen with masks, a realigned address) is generic to the compiler, and
// generic ("flat") loads count against both the vector-memory and the
// LDS/scalar wait counters, so every LDS or scalar wait would also wait for
// the weight stream in flight.  Weight rows are read through pointers cast
// back to this address space, which compiles to global loads.
#define CN_GLOBAL __attribute__((address_space(1)))
typedef CN_GLOBAL const uint8_t cn_gbyte;

#define CN_WAVE 64
#define CN_BLOCK 256

// A zero the compiler cannot see through.  Indexing a uniform address with it
// makes the load a vector load, which is issued with the loads around it and
// waited for only where its value is used; a scalar load of the same word is
// waited for at the first scalar wait of the kernel, before any later load is
// issued.  (A register move only; no memory is touched.)
__device__ __forceinline__ int cn_opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// *p read as a vector load that the kernel consumes late (see cn_opaque_zero);
// the value is uniform, so __builtin_amdgcn_readfirstlane recovers it.
__device__ __forceinline__ int cn_load_late(const int* p) { return p[cn_opaque_zero()]; }

// RoPE (cos, sin) of the pair at even element i of a head at position pos:
// theta = pos * exp(i * (1/hd) * (-ln base)), TensorMath.ApplyRoPE's angle
// (TensorMath.cs:418-432), evaluated exactly as the span kernels' table.
__device__ __forceinline__ float2 cn_rope_cs(int pos, int i, float dim_inv, float neg_log_base) {
  const float theta = (float)pos * expf((float)i * dim_inv * neg_log_base);
  float s, c;
  sincosf(theta, &s, &c);
  return make_float2(c, s);
}

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

// Inputs of the exact-weight span GEMM (x of every projection in a span) are
// two fp16 planes, hi = fp16(x) and lo = fp16(x - hi) (about 22 significant
// bits while |x| stays in fp16's normal range), with each 32-element block
// stored in the order its Q4_0 weight dwords deliver the elements: groups of
// four, G0 G4 G1 G5 G2 G6 G3 G7 (group g = elements 4g..4g+3).  Position of
// element k in a row (every row length is a multiple of 32):
__host__ __device__ __forceinline__ int cn_span_pos(int k) {
  const int g = (k >> 2) & 7;
  return (k & ~31) + 4 * (g < 4 ? 2 * g : 2 * g - 7) + (k & 3);
}

typedef _Float16 cn_half2 __attribute__((ext_vector_type(2)));
typedef float cn_float2 __attribute__((ext_vector_type(2)));

// (a, b) as packed fp16 high parts and packed fp16 low parts.
__device__ __forceinline__ void cn_split_f16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const cn_half2 h = __builtin_convertvector((cn_float2){a, b}, cn_half2);
  const cn_half2 l = __builtin_convertvector((cn_float2){a - (float)h[0], b - (float)h[1]}, cn_half2);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
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
