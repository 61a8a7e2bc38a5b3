// prefill.hip — the per-span kernels of a multi-token LlamaModel.Forward
// (src/ChatNet.Core/Models/Llama/LlamaModel.cs:93-238) run as one batch: the
// RoPE + K/V cache write of all span tokens, and causal GQA attention of every
// span token over the cache.  The matrix products of the span run on the MFMA
// GEMM (gemm.hip).
#include "device_common.h"
#include "kernels.h"

namespace {

// The RoPE table (TensorMath.ApplyRoPE, TensorMath.cs:418-432): one thread per
// (position, pair), theta = pos * exp(i * (1/hd) * (-ln base)) for the pair's
// even index i = 2j.  Built once per model, so the per-token kernels read the
// angles instead of evaluating expf and sincosf (whose large-argument
// reduction would give them a scratch allocation).
__global__ __launch_bounds__(CN_BLOCK) void rope_table_kernel(float2* tab, int ctx, int half, float dim_inv,
                                                              float neg_log_base) {
  const int idx = blockIdx.x * CN_BLOCK + threadIdx.x;
  if (idx >= ctx * half) return;
  const int pos = idx / half, i = 2 * (idx % half);
  const float theta = (float)pos * expf((float)i * dim_inv * neg_log_base);
  float s, c;
  sincosf(theta, &s, &c);
  tab[idx] = make_float2(c, s);
}

// RoPE of the pair (x0, x1) with the table entry cs = (cos, sin).
__device__ __forceinline__ void rope_pair(float& x0, float& x1, float2 cs) {
  const float c = cs.x, s = cs.y;
  const float y0 = x0 * c - x1 * s;
  const float y1 = x0 * s + x1 * c;
  x0 = y0;
  x1 = y1;
}

// One thread per (token, pair): q pairs rotated in place, k pairs rotated and
// stored at cache row p0+t, v pairs copied there (LlamaModel.cs:137-153).
__global__ __launch_bounds__(CN_BLOCK) void rope_kv_kernel(RopeKvArgs a) {
  const int t = blockIdx.y;
  const int pairs_q = a.dim / 2, pairs_kv = a.kv_dim / 2;
  const int i = blockIdx.x * CN_BLOCK + threadIdx.x;
  if (i >= pairs_q + 2 * pairs_kv) return;
  float* row = a.qkv + (size_t)t * a.ld;
  const int pos = a.p0 + t;
  if (i < pairs_q) {
    float2* p = reinterpret_cast<float2*>(row) + i;
    float2 v = *p;
    rope_pair(v.x, v.y, a.rope[(size_t)pos * (a.head_dim / 2) + i % (a.head_dim / 2)]);
    *p = v;
    return;
  }
  const bool is_k = i < pairs_q + pairs_kv;
  const int j = is_k ? i - pairs_q : i - pairs_q - pairs_kv;  // pair index within k or v
  float2 v = reinterpret_cast<const float2*>(row + a.dim + (is_k ? 0 : a.kv_dim))[j];
  if (is_k) rope_pair(v.x, v.y, a.rope[(size_t)pos * (a.head_dim / 2) + j % (a.head_dim / 2)]);
  const size_t off = (size_t)pos * a.kv_dim + 2 * j;
  void* base = is_k ? a.kcache : a.vcache;
  if (a.kv_f16) {
    _Float16* d = reinterpret_cast<_Float16*>(base) + off;
    d[0] = (_Float16)v.x;
    d[1] = (_Float16)v.y;
  } else {
    *reinterpret_cast<float2*>(reinterpret_cast<float*>(base) + off) = v;
  }
}

template <bool F16>
__device__ __forceinline__ float4 kv_load4(const void* base, size_t idx) {
  if constexpr (F16) {
    const _Float16* p = reinterpret_cast<const _Float16*>(base) + idx;
    return make_float4((float)p[0], (float)p[1], (float)p[2], (float)p[3]);
  } else {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + idx);
  }
}

__device__ __forceinline__ float group16_max(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, CN_WAVE));
  return v;
}
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, CN_WAVE);
  return v;
}

// Causal GQA attention of a span (LlamaModel.ComputeAttention,
// LlamaModel.cs:241-346, for every token of the span): token t at position
// p0+t, query head h, kv head h / kv_mul,
//   out[t][h] = softmax_p<=p0+t( q . K[p] * scale ) . V[p].
// A workgroup owns 64 rows = QB consecutive tokens x the kv_mul query heads of
// one kv head (QB = 64 / kv_mul), so each K/V chunk of 64 positions staged in
// LDS serves all of them.  Thread (tr, tc) = (tid / 16, tid % 16) scores rows
// 4tr..4tr+3 against keys tc + 16j, keeps the online-softmax state of its rows
// (the 16 threads of a row group reduce with shuffles), and accumulates
// out[rows][4tc + 64e .. +3].  fp32 throughout; output written as bf16 (and
// its low part, when out_lo is given) for the O-projection GEMM.
template <int HD, bool F16>
__global__ __launch_bounds__(CN_BLOCK) void attn_prefill_kernel(PrefillAttnArgs a) {
  constexpr int R = 64, KB = 64;
  constexpr int S = HD + 4;   // padded LDS row (floats)
  constexpr int OE = HD / 64; // float4 output groups per thread (HD 64 -> 1, 128 -> 2)
  extern __shared__ float lds[];
  float* Qs = lds;            // [R][S]
  float* Ks = Qs + R * S;     // [KB][S]
  float* Vs = Ks + KB * S;    // [KB][S]
  float* Ps = Vs + KB * S;    // [R][KB + 4]
  constexpr int PS = KB + 4;

  const int kvh = blockIdx.x;
  const int qb = blockIdx.y;
  const int QB = R / a.kv_mul;
  const int t0 = qb * QB;
  const int tid = threadIdx.x;
  const int tr = tid >> 4, tc = tid & 15;

  // Q rows: r -> token t0 + r / kv_mul, head kvh*kv_mul + r % kv_mul
  for (int i = tid; i < R * (HD / 4); i += CN_BLOCK) {
    const int r = i / (HD / 4), d4 = i % (HD / 4);
    const int t = t0 + r / a.kv_mul, hh = kvh * a.kv_mul + r % a.kv_mul;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < a.n) v = *reinterpret_cast<const float4*>(a.qkv + (size_t)t * a.ld + hh * HD + 4 * d4);
    *reinterpret_cast<float4*>(&Qs[r * S + 4 * d4]) = v;
  }

  int qpos[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int r = 4 * tr + k;
    const int t = t0 + r / a.kv_mul;
    qpos[k] = t < a.n ? a.p0 + t : -1;  // -1: padding row, every key masked
  }
  const int t_last = min(a.n, t0 + QB) - 1;
  const int kend = a.p0 + t_last + 1;  // keys [0, kend)

  float m_run[4], l_run[4];
  float4 o[4][OE];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    m_run[k] = -INFINITY;
    l_run[k] = 0.f;
#pragma unroll
    for (int e = 0; e < OE; e++) o[k][e] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  for (int c0 = 0; c0 < kend; c0 += KB) {
    __syncthreads();  // previous chunk's readers are done (and Q is staged)
    for (int i = tid; i < KB * (HD / 4); i += CN_BLOCK) {
      const int kk = i / (HD / 4), d4 = i % (HD / 4);
      const int p = c0 + kk;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (p < kend) {
        const size_t idx = (size_t)p * a.kv_dim + kvh * HD + 4 * d4;
        kv = kv_load4<F16>(a.kc, idx);
        vv = kv_load4<F16>(a.vc, idx);
      }
      *reinterpret_cast<float4*>(&Ks[kk * S + 4 * d4]) = kv;
      *reinterpret_cast<float4*>(&Vs[kk * S + 4 * d4]) = vv;
    }
    __syncthreads();

    // scores of rows 4tr..+3 x keys tc + 16j
    float s[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 4; j++) s[k][j] = 0.f;
#pragma unroll 4
    for (int d = 0; d < HD; d += 4) {
      float4 q[4], kk[4];
#pragma unroll
      for (int k = 0; k < 4; k++) q[k] = *reinterpret_cast<const float4*>(&Qs[(4 * tr + k) * S + d]);
#pragma unroll
      for (int j = 0; j < 4; j++) kk[j] = *reinterpret_cast<const float4*>(&Ks[(tc + 16 * j) * S + d]);
#pragma unroll
      for (int k = 0; k < 4; k++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          s[k][j] += q[k].x * kk[j].x + q[k].y * kk[j].y + q[k].z * kk[j].z + q[k].w * kk[j].w;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int p = c0 + tc + 16 * j;
        s[k][j] = (p <= qpos[k]) ? s[k][j] * a.scale : -INFINITY;
        mx = fmaxf(mx, s[k][j]);
      }
      mx = group16_max(mx);
      const float m_new = fmaxf(m_run[k], mx);
      // rows with every key so far masked keep m = -inf and contribute nothing
      const float alpha = (m_new == -INFINITY) ? 1.f : expf(m_run[k] - m_new);
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float p = (m_new == -INFINITY) ? 0.f : expf(s[k][j] - m_new);
        s[k][j] = p;
        sum += p;
      }
      sum = group16_sum(sum);
      l_run[k] = l_run[k] * alpha + sum;
      m_run[k] = m_new;
#pragma unroll
      for (int e = 0; e < OE; e++) {
        o[k][e].x *= alpha; o[k][e].y *= alpha; o[k][e].z *= alpha; o[k][e].w *= alpha;
      }
#pragma unroll
      for (int j = 0; j < 4; j++) Ps[(4 * tr + k) * PS + tc + 16 * j] = s[k][j];
    }
    __syncthreads();
    const int nk = min(KB, kend - c0);
    for (int kk = 0; kk < nk; kk++) {
      float p[4];
#pragma unroll
      for (int k = 0; k < 4; k++) p[k] = Ps[(4 * tr + k) * PS + kk];
#pragma unroll
      for (int e = 0; e < OE; e++) {
        const float4 v = *reinterpret_cast<const float4*>(&Vs[kk * S + 64 * e + 4 * tc]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
          o[k][e].x += p[k] * v.x; o[k][e].y += p[k] * v.y;
          o[k][e].z += p[k] * v.z; o[k][e].w += p[k] * v.w;
        }
      }
    }
  }

#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int r = 4 * tr + k;
    const int t = t0 + r / a.kv_mul, hh = kvh * a.kv_mul + r % a.kv_mul;
    if (t >= a.n) continue;
    const float inv = 1.0f / l_run[k];
    const size_t base = (size_t)t * a.ldo + hh * HD;
#pragma unroll
    for (int e = 0; e < OE; e++) {
      const int d = 64 * e + 4 * tc;
      const float v[4] = {o[k][e].x * inv, o[k][e].y * inv, o[k][e].z * inv, o[k][e].w * inv};
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const __bf16 b = (__bf16)v[j];
        hi[j] = __builtin_bit_cast(uint16_t, b);
        lo[j] = __builtin_bit_cast(uint16_t, (__bf16)(v[j] - (float)b));
      }
      *reinterpret_cast<uint2*>(a.out + base + d) = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
      if (a.out_lo)
        *reinterpret_cast<uint2*>(a.out_lo + base + d) = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
    }
  }
}

template <int HD>
size_t prefill_lds_bytes() {
  return sizeof(float) * (size_t)(3 * 64 * (HD + 4) + 64 * 68);
}

template <int HD, bool F16>
hipError_t attn_prefill_t(const PrefillAttnArgs& a, hipStream_t st) {
  const int QB = 64 / a.kv_mul;
  const dim3 grid(a.n_heads / a.kv_mul, (a.n + QB - 1) / QB);
  static bool lds_set = false;  // > 64 KB of dynamic LDS must be allowed explicitly
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_prefill_kernel<HD, F16>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)prefill_lds_bytes<HD>());
    if (e != hipSuccess) return e;
    lds_set = true;
  }
  hipLaunchKernelGGL((attn_prefill_kernel<HD, F16>), grid, dim3(CN_BLOCK), prefill_lds_bytes<HD>(), st, a);
  return hipGetLastError();
}

}  // namespace

bool attn_prefill_supports(int head_dim, int kv_mul) {
  return (head_dim == 64 || head_dim == 128) && kv_mul >= 1 && kv_mul <= 64 && (64 % kv_mul) == 0;
}

hipError_t attn_prefill_launch(const PrefillAttnArgs& a, hipStream_t st) {
  if (!attn_prefill_supports(a.head_dim, a.kv_mul) || a.n <= 0) return hipErrorInvalidValue;
  if (a.head_dim == 64) return a.kv_f16 ? attn_prefill_t<64, true>(a, st) : attn_prefill_t<64, false>(a, st);
  return a.kv_f16 ? attn_prefill_t<128, true>(a, st) : attn_prefill_t<128, false>(a, st);
}

hipError_t rope_table_launch(float2* tab, int ctx, int head_dim, float dim_inv, float neg_log_base, hipStream_t st) {
  if (ctx <= 0 || head_dim <= 0 || (head_dim & 1)) return hipErrorInvalidValue;
  const int n = ctx * (head_dim / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((n + CN_BLOCK - 1) / CN_BLOCK), dim3(CN_BLOCK), 0, st, tab, ctx,
                     head_dim / 2, dim_inv, neg_log_base);
  return hipGetLastError();
}

hipError_t rope_kv_launch(const RopeKvArgs& a, int n, hipStream_t st) {
  if (n <= 0 || (a.dim & 1) || (a.kv_dim & 1)) return hipErrorInvalidValue;
  const int pairs = a.dim / 2 + a.kv_dim;
  hipLaunchKernelGGL(rope_kv_kernel, dim3((pairs + CN_BLOCK - 1) / CN_BLOCK, n), dim3(CN_BLOCK), 0, st, a);
  return hipGetLastError();
}
