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

// One workgroup per query head (LlamaModel.cs:262-344):
//   s[p] = (q_h . K[p][kvh]) * scale, p <= pos;  softmax;  out_h = sum_p s[p] V[p][kvh]
// kvh = h / kv_mul (LlamaModel.cs:265).  Scores live in LDS (ctx floats).
template <int HD, bool F16>
__global__ __launch_bounds__(CN_BLOCK) void attn_decode_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  float* qs = sm;             // HD
  float* sc = qs + HD;        // ctx
  float* red = sc + a.ctx;    // 4
  float* opart = red + 4;     // CN_BLOCK
  const int h = blockIdx.x;
  const int kvh = h / a.kv_mul;
  const int seq = *a.pos + 1;
  const size_t koff = (size_t)kvh * HD;
  for (int d = threadIdx.x; d < HD; d += CN_BLOCK) qs[d] = a.q[(size_t)h * HD + d];
  __syncthreads();

  // scores: one position per thread
  float mx = -INFINITY;
  for (int p = threadIdx.x; p < seq; p += CN_BLOCK) {
    const size_t base = (size_t)p * a.kv_dim + koff;
    float s = 0.f;
    if constexpr (F16) {
      const uint4* kp = reinterpret_cast<const uint4*>(reinterpret_cast<const _Float16*>(a.kc) + base);
#pragma unroll
      for (int c = 0; c < HD / 8; c++) {
        uint4 t = kp[c];
        const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          s += cn_h2f(u[e]) * qs[8 * c + 2 * e];
          s += cn_h2f(u[e] >> 16) * qs[8 * c + 2 * e + 1];
        }
      }
    } else {
      const float4* kp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.kc) + base);
#pragma unroll
      for (int c = 0; c < HD / 4; c++) {
        const float4 t = kp[c];
        s += t.x * qs[4 * c] + t.y * qs[4 * c + 1] + t.z * qs[4 * c + 2] + t.w * qs[4 * c + 3];
      }
    }
    s *= a.scale;
    sc[p] = s;
    mx = fmaxf(mx, s);
  }
  mx = cn_block_max(mx, red);
  // TensorMath.Softmax (TensorMath.cs:177-241): exp(x - max), sum, * (1/sum)
  float sum = 0.f;
  for (int p = threadIdx.x; p < seq; p += CN_BLOCK) {
    const float e = expf(sc[p] - mx);
    sc[p] = e;
    sum += e;
  }
  sum = cn_block_sum(sum, red);
  const float inv = 1.0f / sum;
  __syncthreads();

  // out[d] = sum_p w_p V[p][d]: G groups of HD threads split the positions.
  constexpr int G = CN_BLOCK / HD;
  const int d = threadIdx.x % HD, g = threadIdx.x / HD;
  float acc = 0.f;
  for (int p = g; p < seq; p += G) {
    const float wgt = sc[p] * inv;
    acc += wgt * kv_load<F16>(a.vc, (size_t)p * a.kv_dim + koff + d);
  }
  opart[threadIdx.x] = acc;
  __syncthreads();
  if (g == 0) {
    float o = acc;
#pragma unroll
    for (int k = 1; k < G; k++) o += opart[k * HD + d];
    a.out[(size_t)h * HD + d] = o;
  }
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
  const size_t smem = sizeof(float) * ((size_t)HD + a.ctx + 4 + CN_BLOCK);
  hipLaunchKernelGGL((attn_decode_kernel<HD, F16>), dim3(a.n_heads), dim3(CN_BLOCK), smem, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t embed_launch(const void* emb, int type, int dim, const int* tok, float* x, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3((dim + CN_BLOCK - 1) / CN_BLOCK), dim3(CN_BLOCK), 0, st, emb,
                     type, dim, tok, x);
  return hipGetLastError();
}

hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t st) {
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
