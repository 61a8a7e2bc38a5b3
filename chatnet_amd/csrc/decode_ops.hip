// decode_ops.hip — per-token kernels around the GEMVs: embedding gather,
// GQA decode attention over the device KV cache, greedy argmax, state update.
#include "device_common.h"
#include "kernels.h"

namespace {

// LlamaModel.LoadEmbedding (LlamaModel.cs:365-394): F32 row copy, F16
// per-element conversion, Q4_0 row dequantization (DequantQ4_0.cs:28-58).
__global__ __launch_bounds__(CN_BLOCK) void embed_kernel(const void* emb, int type, int dim,
                                                         const int* tok, float* x) {
  const int t = tok[blockIdx.y];
  x += (size_t)blockIdx.y * dim;
  const int i = blockIdx.x * CN_BLOCK + threadIdx.x;
  if (i >= dim) return;
  if (type == 0) {
    x[i] = reinterpret_cast<const float*>(emb)[(size_t)t * dim + i];
  } else if (type == 1) {
    const uint16_t* e = reinterpret_cast<const uint16_t*>(emb);
    x[i] = cn_h2f(e[(size_t)t * dim + i]);
  } else {  // Q4_0
    const uint8_t* row = reinterpret_cast<const uint8_t*>(emb) + (size_t)t * (dim / 32) * 18;
    const uint8_t* blk = row + (size_t)(i / 32) * 18;
    const int j = i & 31;
    const float d = cn_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const int q = j < 16 ? (blk[2 + j] & 0x0F) : (blk[2 + j - 16] >> 4);
    x[i] = (float)(q - 8) * d;
  }
}

// Fewest positions a decode-attention split takes: one per wave.  Decode
// attention is latency-bound, so short contexts still spread over many
// workgroups; the cap on splits bounds the merge.
constexpr int kAttnMinChunk = 4;

// Splits that carry positions at sequence length seq: min(splits, ceil(seq / kAttnMinChunk)).
// The decode kernel and the merge both derive it from the device-side position,
// so one captured decode step serves every position.
__device__ __forceinline__ int attn_active_splits(int splits, int seq) {
  return min(splits, (seq + kAttnMinChunk - 1) / kAttnMinChunk);
}

template <bool F16>
__device__ __forceinline__ float kv_load(const void* base, size_t idx) {
  if constexpr (F16) return (float)reinterpret_cast<const _Float16*>(base)[idx];
  else return reinterpret_cast<const float*>(base)[idx];
}

// Split-position GQA decode attention (LlamaModel.ComputeAttention,
// LlamaModel.cs:241-346): for query head h with kvh = h / kv_mul (:265),
//   s[p] = (q_h . K[p][kvh]) * scale  for p <= pos,  w = softmax(s) (TensorMath.cs:177-241),
//   out_h = sum_p w[p] V[p][kvh].
// Grid = n_kv_heads x splits; workgroup (kvh, c) takes positions
// [c*chunk, (c+1)*chunk) of seq = pos+1, and wave w of it the positions
// p = c*chunk + w + 4i.  A wave issues the K and V row loads of PW positions
// at once (lane l owns head elements l*EPL..), keeps q of up to KVM query
// heads of the group in registers, reduces each score across the wave and
// folds it into a running (max, sum, o) per head (online softmax).  The four
// wave partials of a head are folded through LDS into one partial per split
// for attn_merge_kernel.
template <int HD, bool F16, int KVM>
__global__ __launch_bounds__(CN_BLOCK) void attn_decode_kernel(AttnArgs a) {
  constexpr int EPL = HD >= 64 ? HD / 64 : 1;  // head elements per lane
  constexpr int PW = 8;                        // positions whose loads are in flight together
  constexpr int NW = CN_BLOCK / CN_WAVE;
  const int kvh = blockIdx.x / a.splits;
  const int split = blockIdx.x % a.splits;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int seq = *a.pos + 1;
  // Active splits for this position: at least kAttnMinChunk positions each, so
  // short contexts use few workgroups and long ones spread over many.
  const int s_eff = attn_active_splits(a.splits, seq);
  if (split >= s_eff) return;  // uniform over the workgroup, before any barrier
  const int chunk = (seq + s_eff - 1) / s_eff;
  const int p0 = split * chunk;
  const int p1 = min(seq, p0 + chunk);
  const size_t koff = (size_t)kvh * HD;
  const int h0 = kvh * a.kv_mul;
  __shared__ float so[KVM * NW * HD];
  __shared__ float sml[KVM * NW * 2];

  for (int jg = 0; jg < a.kv_mul; jg += KVM) {
    const int nj = min(KVM, a.kv_mul - jg);
    float q[KVM][EPL], m[KVM], l[KVM], o[KVM][EPL];
#pragma unroll
    for (int j = 0; j < KVM; j++) {
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const int d = lane * EPL + e;
        q[j][e] = (j < nj && d < HD) ? a.q[(size_t)(h0 + jg + j) * HD + d] : 0.f;
        o[j][e] = 0.f;
      }
    }
    for (int pb = p0 + wave; pb < p1; pb += NW * PW) {
      float kr[PW][EPL], vr[PW][EPL];
#pragma unroll
      for (int i = 0; i < PW; i++) {
        const int p = pb + NW * i;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
          const int d = lane * EPL + e;
          const bool ok = p < p1 && d < HD;
          const size_t idx = (size_t)p * a.kv_dim + koff + d;
          kr[i][e] = ok ? kv_load<F16>(a.kc, idx) : 0.f;
          vr[i][e] = ok ? kv_load<F16>(a.vc, idx) : 0.f;
        }
      }
#pragma unroll
      for (int i = 0; i < PW; i++) {
        if (pb + NW * i >= p1) break;  // uniform across the wave
#pragma unroll
        for (int j = 0; j < KVM; j++) {
          if (j >= nj) break;
          float sdot = 0.f;
#pragma unroll
          for (int e = 0; e < EPL; e++) sdot += q[j][e] * kr[i][e];
          const float sc = cn_wave_sum(sdot) * a.scale;
          const float mn = fmaxf(m[j], sc);
          const float c = expf(m[j] - mn);
          const float pe = expf(sc - mn);
          l[j] = l[j] * c + pe;
#pragma unroll
          for (int e = 0; e < EPL; e++) o[j][e] = o[j][e] * c + pe * vr[i][e];
          m[j] = mn;
        }
      }
    }
    // fold the NW wave partials of each head through LDS, one partial per split
#pragma unroll
    for (int j = 0; j < KVM; j++) {
      if (j >= nj) break;
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const int d = lane * EPL + e;
        if (d < HD) so[(j * NW + wave) * HD + d] = o[j][e];
      }
      if (lane == 0) {
        sml[2 * (j * NW + wave)] = m[j];
        sml[2 * (j * NW + wave) + 1] = l[j];
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nj * HD; i += CN_BLOCK) {
      const int j = i / HD, d = i % HD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; w++)
        if (sml[2 * (j * NW + w) + 1] > 0.f) M = fmaxf(M, sml[2 * (j * NW + w)]);
      float L = 0.f, acc = 0.f;
#pragma unroll
      for (int w = 0; w < NW; w++) {
        const float lw = sml[2 * (j * NW + w) + 1];
        if (lw > 0.f) {
          const float f = expf(sml[2 * (j * NW + w)] - M);
          L += lw * f;
          acc += so[(j * NW + w) * HD + d] * f;
        }
      }
      const size_t slot = (size_t)(h0 + jg + j) * a.splits + split;
      a.part_o[slot * HD + d] = acc;
      if (d == 0) {
        a.part_ml[2 * slot] = M;
        a.part_ml[2 * slot + 1] = L;
      }
    }
    __syncthreads();
  }
}

// Merges the active split partials of one query head (grid = n_heads, block = HD):
//   M = max_c m_c,  L = sum_c l_c e^(m_c - M),  out = sum_c o_c e^(m_c - M) / L,
// empty splits (l_c = 0) contributing nothing.  Partials are read in rounds of
// R, all loads of a round in flight together, with the running (M, L, acc)
// rescaled when a round raises the maximum.
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(AttnArgs a) {
  constexpr int R = 16;
  const int h = blockIdx.x, d = threadIdx.x;
  const int s_eff = attn_active_splits(a.splits, *a.pos + 1);
  const size_t base = (size_t)h * a.splits;
  float M = -INFINITY, L = 0.f, acc = 0.f;
  for (int c0 = 0; c0 < s_eff; c0 += R) {
    float mc[R], lc[R], oc[R];
#pragma unroll
    for (int c = 0; c < R; c++) {
      const bool on = c0 + c < s_eff;
      mc[c] = on ? a.part_ml[2 * (base + c0 + c)] : 0.f;
      lc[c] = on ? a.part_ml[2 * (base + c0 + c) + 1] : 0.f;
      oc[c] = on ? a.part_o[(base + c0 + c) * HD + d] : 0.f;
    }
    float Mn = M;
#pragma unroll
    for (int c = 0; c < R; c++)
      if (lc[c] > 0.f) Mn = fmaxf(Mn, mc[c]);
    if (Mn == -INFINITY) continue;  // nothing in this round or before it
    const float r = (M == -INFINITY) ? 0.f : expf(M - Mn);
    L *= r;
    acc *= r;
#pragma unroll
    for (int c = 0; c < R; c++) {
      if (lc[c] > 0.f) {
        const float f = expf(mc[c] - Mn);
        L += lc[c] * f;
        acc += oc[c] * f;
      }
    }
    M = Mn;
  }
  a.out[(size_t)h * HD + d] = acc / L;
}

// GreedySampler.Sample: strict '>' scan => the lowest index of the maximum;
// NaN never wins unless it sits at index 0, in which case the answer is 0.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, int n, int* state,
                                                      int* out_tokens, int out_cap) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  float best = -INFINITY;
  int idx = 0x7FFFFFFF;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = logits[i];
    if (v > best) {
      best = v;
      idx = i;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (ov > best || (ov == best && oi < idx)) {
      best = ov;
      idx = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    best = bv[0];
    idx = bi[0];
    for (int w = 1; w < 16; w++)
      if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
        best = bv[w];
        idx = bi[w];
      }
    if (idx == 0x7FFFFFFF || logits[0] != logits[0]) idx = 0;
    state[1] = idx;
    const int step = state[2];
    if (out_tokens && step < out_cap) out_tokens[step] = idx;
    state[2] = step + 1;
    state[0] = state[0] + 1;
  }
}

__global__ void set_state_kernel(int* state, int pos, int tok, int step) {
  state[0] = pos;
  state[1] = tok;
  if (step >= 0) state[2] = step;
}

template <int HD, bool F16>
hipError_t attn_launch_t(const AttnArgs& a, hipStream_t st) {
  const int n_kv = a.n_heads / a.kv_mul;
  if (a.kv_mul == 1)
    hipLaunchKernelGGL((attn_decode_kernel<HD, F16, 1>), dim3(n_kv * a.splits), dim3(CN_BLOCK), 0, st, a);
  else
    hipLaunchKernelGGL((attn_decode_kernel<HD, F16, 8>), dim3(n_kv * a.splits), dim3(CN_BLOCK), 0, st, a);
  hipLaunchKernelGGL((attn_merge_kernel<HD>), dim3(a.n_heads), dim3(HD), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t embed_launch(const void* emb, int type, int dim, const int* tok, float* x, hipStream_t st, int n) {
  if (n < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_kernel, dim3((dim + CN_BLOCK - 1) / CN_BLOCK, n), dim3(CN_BLOCK), 0, st, emb,
                     type, dim, tok, x);
  return hipGetLastError();
}

hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t st) {
  if (a.splits < 1 || a.splits > 64) return hipErrorInvalidValue;
  if (a.head_dim == 64) return a.kv_f16 ? attn_launch_t<64, true>(a, st) : attn_launch_t<64, false>(a, st);
  if (a.head_dim == 128) return a.kv_f16 ? attn_launch_t<128, true>(a, st) : attn_launch_t<128, false>(a, st);
  if (a.head_dim == 32) return a.kv_f16 ? attn_launch_t<32, true>(a, st) : attn_launch_t<32, false>(a, st);
  if (a.head_dim == 256) return a.kv_f16 ? attn_launch_t<256, true>(a, st) : attn_launch_t<256, false>(a, st);
  return hipErrorInvalidValue;
}

hipError_t argmax_launch(const float* logits, int n, int* state, int* out_tokens, int out_cap,
                         hipStream_t st) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, st, logits, n, state, out_tokens, out_cap);
  return hipGetLastError();
}

hipError_t set_state_launch(int* state, int pos, int tok, int step, hipStream_t st) {
  hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(1), 0, st, state, pos, tok, step);
  return hipGetLastError();
}
