// gemv_float.hip — GEMV for F32 and F16 weight matrices, and for packed units
// (the block types without a digit-path kernel), on gfx950.
//
// Replaces the two float branches of LlamaModel.MatVecMulByType
// (src/ChatNet.Core/Models/Llama/LlamaModel.cs:470-567):
//   F32  TensorMath.MatVecMul (TensorMath.cs:527-540): y[r] = dot(W[r], x)
//   F16  LlamaModel.MatVecMulF16 (LlamaModel.cs:570-598): every half of the
//        row converted exactly (DequantQ4_0.HalfToFloat), then the dot.
// Rows are independent (TensorMath.cs:47-51); the GPU sums in its own order
// with fp32 FMAs, within the GEMV tolerance of the reference's order.
//
// x (times the RMSNorm weight when one is fused) is staged once per
// workgroup in LDS as fp32; 1/rms is applied to the finished dots, as in the
// quantized GEMV.  A wave owns RPW consecutive rows at a time: lane l reads
// the 16-byte pieces l, l+64, ... of each row (1 KB per wave and row per
// step, fully coalesced), U steps of all RPW rows issued before any FMA, and
// the row sums are reduced across the wave.  The epilogues are the quantized
// GEMV's (gemv_common.h): store, residual add, QKV + RoPE + KV-cache write,
// SiLU(gate)*up on interleaved rows, LM head, and the attention merge folded
// into the O projection's x staging.
#include "device_common.h"
#include "gemv_common.h"
#include "kernels.h"

namespace {

constexpr int WT_F32 = 0, WT_F16 = 1;

// 16-byte pieces of a row: 4 F32 or 8 F16 weights.
template <int WT>
constexpr int piece_elems() { return WT == WT_F32 ? 4 : 8; }

template <int WT>
__device__ __forceinline__ float piece_dot(const cn_u32x4& w, const float* xs) {
  if constexpr (WT == WT_F32) {
    const float4 xv = *reinterpret_cast<const float4*>(xs);
    float t = __uint_as_float(w.x) * xv.x;
    t = fmaf(__uint_as_float(w.y), xv.y, t);
    t = fmaf(__uint_as_float(w.z), xv.z, t);
    return fmaf(__uint_as_float(w.w), xv.w, t);
  } else {
    const float4 x0 = *reinterpret_cast<const float4*>(xs);
    const float4 x1 = *reinterpret_cast<const float4*>(xs + 4);
    float t = cn_h2f(w.x) * x0.x;
    t = fmaf(cn_h2f(w.x >> 16), x0.y, t);
    t = fmaf(cn_h2f(w.y), x0.z, t);
    t = fmaf(cn_h2f(w.y >> 16), x0.w, t);
    t = fmaf(cn_h2f(w.z), x1.x, t);
    t = fmaf(cn_h2f(w.z >> 16), x1.y, t);
    t = fmaf(cn_h2f(w.w), x1.z, t);
    return fmaf(cn_h2f(w.w >> 16), x1.w, t);
  }
}

template <int WT, int RPW, int EPI, int U>
__global__ __launch_bounds__(CN_BLOCK) void gemv_f_kernel(GemvArgs a) {
  constexpr int NWV = CN_BLOCK / CN_WAVE;
  constexpr int PE = piece_elems<WT>();
  constexpr int NR = res_count<EPI, RPW>();
  constexpr bool NORM = EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_SWIGLU || EPI == GEMV_EPI_LOGITS;
  constexpr bool MERGE = EPI == GEMV_EPI_ADD_MERGE;
  extern __shared__ float smem[];  // [K] staged x, then NWV partial sums of squares
  const int K = a.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos_v = (EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_ADD_MERGE) ? cn_load_late(a.pos) : 0;
  const int stop_v = cn_load_late(stop_flag(a));
  float* red = smem + K;

  // ---- stage x * g as fp32 (sum of squares of x for the RMS factor) ----
  MergeSrc ms{};
  if constexpr (MERGE) {
    ms.o = a.part_o;
    ms.ml = a.part_ml;
    ms.hd = a.head_dim;
    ms.splits = a.msplits;
    ms.s_eff = min(a.msplits, (__builtin_amdgcn_readfirstlane(pos_v) + a.mchunk) / a.mchunk);
  }
  float ss = 0.f;
  for (int c = threadIdx.x; c < (K >> 2); c += CN_BLOCK) {
    float4 v;
    if constexpr (MERGE) v = merged_x4<kFoldMaxSplits>(ms, 4 * c);
    else v = reinterpret_cast<const float4*>(a.x)[c];
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    if constexpr (NORM) {
      const float4 g = reinterpret_cast<const float4*>(a.norm_w)[c];
      v.x *= g.x;
      v.y *= g.y;
      v.z *= g.z;
      v.w *= g.w;
    }
    reinterpret_cast<float4*>(smem)[c] = v;
  }
  ss = cn_wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float sst = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; w++) sst += red[w];
  const float rms = NORM ? 1.0f / sqrtf(sst / (float)K + a.eps) : 1.0f;
  if (__builtin_amdgcn_readfirstlane(stop_v)) return;
  const int pos = __builtin_amdgcn_readfirstlane(pos_v);

  const size_t row_bytes = (size_t)K * (WT == WT_F32 ? 4 : 2);
  const int npieces = K / PE;  // 16-byte pieces per row
  const int n_iters = (a.n_vrows + RPW - 1) / RPW;
  for (int it = blockIdx.x * NWV + wave; it < n_iters; it += gridDim.x * NWV) {
    const int vr0 = it * RPW;
    const cn_gbyte* rp[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int vr = vr0 + i < a.n_vrows ? vr0 + i : a.n_vrows - 1;  // rows past the end re-read the last
      int seg, r;
      map_row<EPI>(a, vr, seg, r);
      rp[i] = seg_w(a, seg) + (size_t)r * row_bytes;
    }
    float res[NR];
    load_residual<EPI, RPW, NR>(a, vr0, lane, pos, res);
    load_rope<EPI, RPW, NR>(a, vr0, pos, res);
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[i] = 0.f;
    for (int p0 = 0; p0 < npieces; p0 += CN_WAVE * U) {
      cn_u32x4 w[U][RPW];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int p = p0 + CN_WAVE * u + lane;
#pragma unroll
        for (int i = 0; i < RPW; i++)
          w[u][i] = p < npieces ? *(const CN_GLOBAL cn_u32x4*)(rp[i] + (size_t)p * 16) : cn_u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int p = p0 + CN_WAVE * u + lane;
        if (p < npieces) {
#pragma unroll
          for (int i = 0; i < RPW; i++) acc[i] += piece_dot<WT>(w[u][i], smem + (size_t)p * PE);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[i] = cn_wave_sum(acc[i]) * rms;
    if (lane == 0) epilogue<EPI, RPW>(a, vr0, acc, res, pos);
  }
}

size_t gemv_f_smem(int K) { return sizeof(float) * ((size_t)K + 16); }

// Packed-unit weights (gemm_pack_kernel: 64 u8 codes, then 4 fp32 scales and
// 4 fp32 offsets, one pair per 16 weights; weight = fmaf(code, scale,
// offset), the block type's dequantized value): the generic branches of
// MatVecMulByType (LlamaModel.cs:488-511, 517-528: Q4_1, Q5_0, Q5_1, Q2_K,
// Q3_K, Q8_K through TensorMath.MatVecMulGeneric, TensorMath.cs:624-656).
// x * g is staged as above, plus the sum of every 16-element group, so a
// group contributes scale * sum(code * x) + offset * sum(x).  Lane l of a wave
// takes units l, l+64, ... of each of the wave's RPW rows (six 16-byte loads
// per unit and row).
template <int RPW, int EPI>
__global__ __launch_bounds__(CN_BLOCK) void gemv_pk_kernel(GemvArgs a) {
  constexpr int NWV = CN_BLOCK / CN_WAVE;
  constexpr int NR = res_count<EPI, RPW>();
  constexpr bool NORM = EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_SWIGLU || EPI == GEMV_EPI_LOGITS;
  constexpr bool MERGE = EPI == GEMV_EPI_ADD_MERGE;
  extern __shared__ float smem[];  // [K] staged x, [K/16] group sums, then NWV partial sums of squares
  const int K = a.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos_v = (EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_ADD_MERGE) ? cn_load_late(a.pos) : 0;
  const int stop_v = cn_load_late(stop_flag(a));
  float* gsum = smem + K;
  float* red = gsum + K / 16;

  MergeSrc ms{};
  if constexpr (MERGE) {
    ms.o = a.part_o;
    ms.ml = a.part_ml;
    ms.hd = a.head_dim;
    ms.splits = a.msplits;
    ms.s_eff = min(a.msplits, (__builtin_amdgcn_readfirstlane(pos_v) + a.mchunk) / a.mchunk);
  }
  float ss = 0.f;
  for (int c = threadIdx.x; c < (K >> 2); c += CN_BLOCK) {
    float4 v;
    if constexpr (MERGE) v = merged_x4<kFoldMaxSplits>(ms, 4 * c);
    else v = reinterpret_cast<const float4*>(a.x)[c];
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    if constexpr (NORM) {
      const float4 g = reinterpret_cast<const float4*>(a.norm_w)[c];
      v.x *= g.x;
      v.y *= g.y;
      v.z *= g.z;
      v.w *= g.w;
    }
    reinterpret_cast<float4*>(smem)[c] = v;
  }
  ss = cn_wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  for (int gi = threadIdx.x; gi < (K >> 4); gi += CN_BLOCK) {
    const float4* p = reinterpret_cast<const float4*>(smem + 16 * gi);
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) t += (p[q].x + p[q].y) + (p[q].z + p[q].w);
    gsum[gi] = t;
  }
  float sst = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; w++) sst += red[w];
  __syncthreads();
  const float rms = NORM ? 1.0f / sqrtf(sst / (float)K + a.eps) : 1.0f;
  if (__builtin_amdgcn_readfirstlane(stop_v)) return;
  const int pos = __builtin_amdgcn_readfirstlane(pos_v);

  const int nunits = K / 64;
  const size_t row_bytes = (size_t)nunits * kGemmPackUnit;
  const int n_iters = (a.n_vrows + RPW - 1) / RPW;
  for (int it = blockIdx.x * NWV + wave; it < n_iters; it += gridDim.x * NWV) {
    const int vr0 = it * RPW;
    const cn_gbyte* rp[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int vr = vr0 + i < a.n_vrows ? vr0 + i : a.n_vrows - 1;  // rows past the end re-read the last
      int seg, r;
      map_row<EPI>(a, vr, seg, r);
      rp[i] = seg_w(a, seg) + (size_t)r * row_bytes;
    }
    float res[NR];
    load_residual<EPI, RPW, NR>(a, vr0, lane, pos, res);
    load_rope<EPI, RPW, NR>(a, vr0, pos, res);
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[i] = 0.f;
    for (int u = lane; u < nunits; u += CN_WAVE) {
      cn_u32x4 w[RPW][6];
#pragma unroll
      for (int i = 0; i < RPW; i++)
#pragma unroll
        for (int q = 0; q < 6; q++)
          w[i][q] = *(const CN_GLOBAL cn_u32x4*)(rp[i] + (size_t)u * kGemmPackUnit + 16 * q);
      const float* xs = smem + 64 * u;
      const float* gs = gsum + 4 * u;
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        float t = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const cn_u32x4 c = w[i][g];
          const float4 x0 = *reinterpret_cast<const float4*>(xs + 16 * g);
          const float4 x1 = *reinterpret_cast<const float4*>(xs + 16 * g + 4);
          const float4 x2 = *reinterpret_cast<const float4*>(xs + 16 * g + 8);
          const float4 x3 = *reinterpret_cast<const float4*>(xs + 16 * g + 12);
          float d = cn_ubyte<0>(c.x) * x0.x;
          d = fmaf(cn_ubyte<1>(c.x), x0.y, d);
          d = fmaf(cn_ubyte<2>(c.x), x0.z, d);
          d = fmaf(cn_ubyte<3>(c.x), x0.w, d);
          d = fmaf(cn_ubyte<0>(c.y), x1.x, d);
          d = fmaf(cn_ubyte<1>(c.y), x1.y, d);
          d = fmaf(cn_ubyte<2>(c.y), x1.z, d);
          d = fmaf(cn_ubyte<3>(c.y), x1.w, d);
          d = fmaf(cn_ubyte<0>(c.z), x2.x, d);
          d = fmaf(cn_ubyte<1>(c.z), x2.y, d);
          d = fmaf(cn_ubyte<2>(c.z), x2.z, d);
          d = fmaf(cn_ubyte<3>(c.z), x2.w, d);
          d = fmaf(cn_ubyte<0>(c.w), x3.x, d);
          d = fmaf(cn_ubyte<1>(c.w), x3.y, d);
          d = fmaf(cn_ubyte<2>(c.w), x3.z, d);
          d = fmaf(cn_ubyte<3>(c.w), x3.w, d);
          const float scale = __uint_as_float(w[i][4][g]), offset = __uint_as_float(w[i][5][g]);
          t = fmaf(scale, d, fmaf(offset, gs[g], t));
        }
        acc[i] += t;
      }
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[i] = cn_wave_sum(acc[i]) * rms;
    if (lane == 0) epilogue<EPI, RPW>(a, vr0, acc, res, pos);
  }
}

size_t gemv_pk_smem(int K) { return sizeof(float) * ((size_t)K + (size_t)K / 16 + 16); }

template <int EPI>
hipError_t launch_pk(const GemvArgs& a, int num_cus, hipStream_t st) {
  constexpr int RPW = 2;
  const size_t smem = gemv_pk_smem(a.K);
  const auto kern = &gemv_pk_kernel<RPW, EPI>;
  if (smem > 65536) {  // more than 64 KB of dynamic LDS must be allowed (once per device)
    static std::atomic<uint64_t> lds_done{0};
    const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(kern), lds_done);
    if (e != hipSuccess) return e;
  }
  const int n_iters = (a.n_vrows + RPW - 1) / RPW;
  int grid = (n_iters + 3) / 4;
  if (grid > 4 * num_cus) grid = 4 * num_cus;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(CN_BLOCK), smem, st, a);
  return hipGetLastError();
}

template <int WT, int EPI>
hipError_t launch_wt(const GemvArgs& a, int num_cus, hipStream_t st) {
  constexpr int RPW = 2, U = 4;
  const size_t smem = gemv_f_smem(a.K);
  const auto kern = &gemv_f_kernel<WT, RPW, EPI, U>;
  if (smem > 65536) {  // more than 64 KB of dynamic LDS must be allowed (once per device)
    static std::atomic<uint64_t> lds_done{0};
    const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(kern), lds_done);
    if (e != hipSuccess) return e;
  }
  const int n_iters = (a.n_vrows + RPW - 1) / RPW;
  int grid = (n_iters + 3) / 4;
  if (grid > 4 * num_cus) grid = 4 * num_cus;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(CN_BLOCK), smem, st, a);
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_f_epi(int qtype, const GemvArgs& a, int num_cus, hipStream_t st) {
  if (qtype == 0) return launch_wt<WT_F32, EPI>(a, num_cus, st);
  if (qtype == 1) return launch_wt<WT_F16, EPI>(a, num_cus, st);
  return launch_pk<EPI>(a, num_cus, st);
}

}  // namespace

hipError_t gemv_float_launch(int qtype, int epi, const GemvArgs& a, int num_cus, hipStream_t st) {
  if ((qtype != 0 && qtype != 1 && qtype != kGemvPacked) || a.K <= 0 || a.K % 64 != 0 || a.K > 16384)
    return hipErrorInvalidValue;
  switch (epi) {
    case GEMV_EPI_STORE: return launch_f_epi<GEMV_EPI_STORE>(qtype, a, num_cus, st);
    case GEMV_EPI_ADD: return launch_f_epi<GEMV_EPI_ADD>(qtype, a, num_cus, st);
    case GEMV_EPI_QKV: return launch_f_epi<GEMV_EPI_QKV>(qtype, a, num_cus, st);
    case GEMV_EPI_SWIGLU: return launch_f_epi<GEMV_EPI_SWIGLU>(qtype, a, num_cus, st);
    case GEMV_EPI_LOGITS: return launch_f_epi<GEMV_EPI_LOGITS>(qtype, a, num_cus, st);
    case GEMV_EPI_ADD_MERGE:
      if (a.msplits < 2 || a.msplits > kFoldMaxSplits || a.mchunk < 1 || a.head_dim % 32 != 0)
        return hipErrorInvalidValue;
      return launch_f_epi<GEMV_EPI_ADD_MERGE>(qtype, a, num_cus, st);
    default: return hipErrorInvalidValue;
  }
}
