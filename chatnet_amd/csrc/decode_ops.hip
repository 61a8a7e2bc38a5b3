// decode_ops.hip — per-token kernels around the GEMVs: embedding gather,
// GQA decode attention over the device KV cache, greedy argmax, state update.
#include "device_common.h"
#include "kernels.h"

namespace {

// LlamaModel.LoadEmbedding (LlamaModel.cs:365-394): F32 row copy, F16
// per-element conversion, Q4_0 row dequantization (DequantQ4_0.cs:28-58).
__global__ __launch_bounds__(CN_BLOCK) void embed_kernel(const void* emb, int type, int dim,
                                                         const int* tok, float* x) {
  const int t = *tok;
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

template <bool F16>
__device__ __forceinline__ float kv_load(const void* base, size_t idx) {
  if constexpr (F16) return (float)reinterpret_cast<const _Float16*>(base)[idx];
  else return reinterpret_cast<const float*>(base)[idx];
}

// Split-position GQA decode attention (LlamaModel.ComputeAttention,
// LlamaModel.cs:241-346):  for query head h with kvh = h / kv_mul (:265),
//   s[p] = (q_h . K[p][kvh]) * scale  for p <= pos,  w = softmax(s),
//   out_h = sum_p w[p] V[p][kvh].
// Grid = n_kv_heads x splits.  Workgroup (kvh, c) takes positions
// [c*chunk, (c+1)*chunk) of seq = pos+1 and every query head of the group, so
// each K/V row is read once for all kv_mul heads; waves take positions, lanes
// take head_dim elements (coalesced rows).  Each split leaves (max, sum, o)
// for attn_merge_kernel.
template <int HD, bool F16, int GMAX>
__global__ __launch_bounds__(CN_BLOCK) void attn_decode_kernel(AttnArgs a) {
  constexpr int EPL = HD >= 64 ? HD / 64 : 1;  // head elements per lane
  constexpr int G = CN_BLOCK / HD;             // position groups in the V pass
  extern __shared__ float sm[];
  const int kvh = blockIdx.x / a.splits;
  const int split = blockIdx.x % a.splits;
  const int kv_mul = a.kv_mul;
  const int seq = *a.pos + 1;
  const int chunk = (seq + a.splits - 1) / a.splits;
  const int p0 = split * chunk;
  const int p1 = min(seq, p0 + chunk);
  const int cap = a.chunk_cap;
  float* qs = sm;                       // kv_mul * HD
  float* sc = qs + kv_mul * HD;         // kv_mul * cap
  float* ml = sc + kv_mul * cap;        // kv_mul * 2
  float* op = ml + 2 * kv_mul;          // G * GMAX * HD
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t koff = (size_t)kvh * HD;
  const int h0 = kvh * kv_mul;

  for (int i = threadIdx.x; i < kv_mul * HD; i += CN_BLOCK) qs[i] = a.q[(size_t)h0 * HD + i];
  __syncthreads();

  // scores
  for (int p = p0 + wave; p < p1; p += CN_BLOCK / CN_WAVE) {
    float kv[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const int d = lane * EPL + e;
      kv[e] = d < HD ? kv_load<F16>(a.kc, (size_t)p * a.kv_dim + koff + d) : 0.f;
    }
    for (int j = 0; j < kv_mul; j++) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const int d = lane * EPL + e;
        if (d < HD) s += qs[j * HD + d] * kv[e];
      }
      s = cn_wave_sum(s);
      if (lane == 0) sc[j * cap + (p - p0)] = s * a.scale;
    }
  }
  __syncthreads();

  // per-head max and exp-sum of this split (one wave per head)
  for (int j = wave; j < kv_mul; j += CN_BLOCK / CN_WAVE) {
    float m = -INFINITY;
    for (int i = lane; i < p1 - p0; i += CN_WAVE) m = fmaxf(m, sc[j * cap + i]);
    m = cn_wave_max(m);
    float l = 0.f;
    for (int i = lane; i < p1 - p0; i += CN_WAVE) {
      const float e = expf(sc[j * cap + i] - m);
      sc[j * cap + i] = e;
      l += e;
    }
    l = cn_wave_sum(l);
    if (lane == 0) {
      ml[2 * j] = m;
      ml[2 * j + 1] = l;
    }
  }
  __syncthreads();

  // o_j[d] = sum_p e_j[p] V[p][d], GMAX heads at a time
  const int d = threadIdx.x % HD, g = threadIdx.x / HD;
  for (int jb = 0; jb < kv_mul; jb += GMAX) {
    float o[GMAX];
#pragma unroll
    for (int j = 0; j < GMAX; j++) o[j] = 0.f;
    for (int p = p0 + g; p < p1; p += G) {
      const float v = kv_load<F16>(a.vc, (size_t)p * a.kv_dim + koff + d);
#pragma unroll
      for (int j = 0; j < GMAX; j++)
        if (jb + j < kv_mul) o[j] += sc[(jb + j) * cap + (p - p0)] * v;
    }
#pragma unroll
    for (int j = 0; j < GMAX; j++) op[(g * GMAX + j) * HD + d] = o[j];
    __syncthreads();
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < GMAX; j++) {
        if (jb + j >= kv_mul) break;
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < G; k++) t += op[(k * GMAX + j) * HD + d];
        if (a.splits == 1) {  // single split: normalise in place
          a.out[(size_t)(h0 + jb + j) * HD + d] = t / ml[2 * (jb + j) + 1];
          continue;
        }
        const size_t slot = (size_t)(h0 + jb + j) * a.splits + split;
        a.part_o[slot * HD + d] = t;
        if (d == 0) {
          a.part_ml[2 * slot] = ml[2 * (jb + j)];
          a.part_ml[2 * slot + 1] = ml[2 * (jb + j) + 1];
        }
      }
    }
    __syncthreads();
  }

}

// Merges the split partials of one query head (grid = n_heads, block = HD):
//   M = max_c m_c,  L = sum_c l_c e^(m_c - M),  out = sum_c o_c e^(m_c - M) / L.
// Empty splits (l_c = 0) contribute nothing.
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(AttnArgs a) {
  const int h = blockIdx.x, d = threadIdx.x;
  const size_t base = (size_t)h * a.splits;
  float M = -INFINITY;
  for (int c = 0; c < a.splits; c++)
    if (a.part_ml[2 * (base + c) + 1] > 0.f) M = fmaxf(M, a.part_ml[2 * (base + c)]);
  float L = 0.f, acc = 0.f;
  for (int c = 0; c < a.splits; c++) {
    const float lc = a.part_ml[2 * (base + c) + 1];
    if (lc == 0.f) continue;
    const float f = expf(a.part_ml[2 * (base + c)] - M);
    L += lc * f;
    acc += a.part_o[(base + c) * HD + d] * f;
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
  constexpr int GMAX = 8;
  const int G = CN_BLOCK / HD;
  const size_t smem = sizeof(float) * ((size_t)a.kv_mul * HD + (size_t)a.kv_mul * a.chunk_cap + 2 * a.kv_mul +
                                       (size_t)G * GMAX * HD);
  const int n_kv = a.n_heads / a.kv_mul;
  hipLaunchKernelGGL((attn_decode_kernel<HD, F16, GMAX>), dim3(n_kv * a.splits), dim3(CN_BLOCK), smem, st, a);
  if (a.splits > 1) hipLaunchKernelGGL((attn_merge_kernel<HD>), dim3(a.n_heads), dim3(HD), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t embed_launch(const void* emb, int type, int dim, const int* tok, float* x, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3((dim + CN_BLOCK - 1) / CN_BLOCK), dim3(CN_BLOCK), 0, st, emb,
                     type, dim, tok, x);
  return hipGetLastError();
}

hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t st) {
  if (a.splits < 1 || a.chunk_cap * a.splits < a.ctx) return hipErrorInvalidValue;
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
