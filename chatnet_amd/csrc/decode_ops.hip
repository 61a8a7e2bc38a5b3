// decode_ops.hip — per-token kernels around the GEMVs: embedding gather,
// GQA decode attention over the device KV cache, greedy argmax, state update.
#include "device_common.h"
#include "kernels.h"

namespace {

// The stop flag of launches outside a decode loop (never set).
static __device__ int g_never_stop = 0;

// LlamaModel.LoadEmbedding (LlamaModel.cs:365-394): F32 row copy, F16
// per-element conversion, Q4_0 / Q8_0 row dequantization (DequantQ4_0.cs:28-58,
// DequantQ8_0.cs:19-41), and every other block type through its packed units
// (type kGemvPacked: fmaf(code, scale, offset), the type's dequantized value,
// the generic branch at LlamaModel.cs:384-393).
__global__ __launch_bounds__(CN_BLOCK) void embed_kernel(const void* emb, int type, int dim,
                                                         const int* tok, float* x) {
  const int t = tok[blockIdx.y];
  x += (size_t)blockIdx.y * dim;
  const int i = blockIdx.x * CN_BLOCK + threadIdx.x;
  if (i >= dim) return;
  if (type == kGemvPacked) {
    const uint8_t* u = reinterpret_cast<const uint8_t*>(emb) + ((size_t)t * (dim / 64) + i / 64) * kGemmPackUnit;
    const float* sc = reinterpret_cast<const float*>(u + 64);
    const int g = (i & 63) >> 4;
    x[i] = fmaf((float)u[i & 63], sc[g], sc[4 + g]);
  } else if (type == 0) {
    x[i] = reinterpret_cast<const float*>(emb)[(size_t)t * dim + i];
  } else if (type == 1) {
    const uint16_t* e = reinterpret_cast<const uint16_t*>(emb);
    x[i] = cn_h2f(e[(size_t)t * dim + i]);
  } else if (type == 8) {  // Q8_0: DequantQ8_0.Dequantize (DequantQ8_0.cs:19-41), qs[j] * d
    const uint8_t* blk = reinterpret_cast<const uint8_t*>(emb) + ((size_t)t * (dim / 32) + i / 32) * 34;
    const float d = cn_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    x[i] = (float)(int8_t)blk[2 + (i & 31)] * d;
  } else {  // Q4_0
    const uint8_t* row = reinterpret_cast<const uint8_t*>(emb) + (size_t)t * (dim / 32) * 18;
    const uint8_t* blk = row + (size_t)(i / 32) * 18;
    const int j = i & 31;
    const float d = cn_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const int q = j < 16 ? (blk[2 + j] & 0x0F) : (blk[2 + j - 16] >> 4);
    x[i] = (float)(q - 8) * d;
  }
}

// n consecutive floats of a K/V cache row (fp32 or fp16) starting at idx.
template <bool F16, int N>
__device__ __forceinline__ void kv_load_n(const void* base, size_t idx, float* out) {
  if constexpr (F16) {
    const _Float16* p = reinterpret_cast<const _Float16*>(base) + idx;
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 4) {
        const uint2 u = *reinterpret_cast<const uint2*>(p + i);
        out[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.x & 0xFFFFu));
        out[i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.x >> 16));
        out[i + 2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y & 0xFFFFu));
        out[i + 3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y >> 16));
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; i++) out[i] = (float)p[i];
    }
  } else {
    const float* p = reinterpret_cast<const float*>(base) + idx;
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + i);
        out[i] = v.x; out[i + 1] = v.y; out[i + 2] = v.z; out[i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; i++) out[i] = p[i];
    }
  }
}

// Sum over the 16 lanes of a row (DPP: quad xor 1, quad xor 2, half-row
// mirror, row mirror); every lane of the row gets the sum.
__device__ __forceinline__ float row_sum16(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
  return v;
}

// One (head, element) result of a split: the final output when the launch
// has a single chunk (nothing to merge), else the split's partial.
template <int HD>
__device__ __forceinline__ void attn_put(const AttnArgs& a, int h, int split, int d, float M, float L, float acc) {
  if (a.splits == 1) {
    a.out[(size_t)h * HD + d] = acc / L;
    return;
  }
  const size_t slot = (size_t)h * a.splits + split;
  a.part_o[slot * HD + d] = acc;
  if (d == 0) {
    a.part_ml[2 * slot] = M;
    a.part_ml[2 * slot + 1] = L;
  }
}

// Split-position GQA decode attention (LlamaModel.ComputeAttention,
// LlamaModel.cs:241-346): for query head h with kvh = h / kv_mul (:265),
//   s[p] = (q_h . K[p][kvh]) * scale  for p <= pos,  w = softmax(s) (TensorMath.cs:177-241),
//   out_h = sum_p w[p] V[p][kvh].
// Grid = n_kv_heads x a.splits; workgroup (kvh, c) takes the positions
// [c*chunk, (c+1)*chunk) below seq = pos+1.  Its four waves split the kv_mul
// query heads WH ways (WH = 4, 2 or 1 as kv_mul allows, HPW heads per wave
// and pass) and the positions WP = 4/WH ways.  A wave is 4 rows of 16 lanes:
// row r holds one position, lane i of the row the head elements
// [i*EPL, (i+1)*EPL) (EPL = HD/16).  A wave step covers SP = 4*PG consecutive
// positions for the wave's heads: 16-lane dot products reduced with DPP inside
// the row, one max over the step's positions per head, one rescale of the
// running (max, sum, o) per head (online softmax; sums and o stay per row
// until the end, then add across rows).  The first step's K/V loads depend
// only on the chunk, so they are in flight before the position arrives.  With
// WP = 1 each wave holds its heads' complete result for the chunk; otherwise
// the WP waves of a head fold through LDS.  A launch of one chunk writes the
// output itself; more chunks (at most kFoldMaxSplits) leave partials that the
// O projection combines as it stages its x (GEMV_EPI_ADD_MERGE).
template <int HD, bool F16, int HPW, int PG>
__global__ __launch_bounds__(CN_BLOCK) void attn_decode_kernel(AttnArgs a) {
  constexpr int EPL = HD / 16;   // head elements per lane
  constexpr int NW = CN_BLOCK / CN_WAVE;
  constexpr int SP = 4 * PG;     // positions per wave step
  // workgroup (kv head, head group, split): a.hsplit workgroups share a kv
  // head, each taking kvm = kv_mul / hsplit of its query heads
  const int split = blockIdx.x % a.splits;
  const int hs = (blockIdx.x / a.splits) % a.hsplit;
  const int kvh = blockIdx.x / (a.splits * a.hsplit);
  const int kvm = a.kv_mul / a.hsplit;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = lane >> 4, col = lane & 15;
  const int WH = kvm >= 4 ? 4 : (kvm >= 2 ? 2 : 1);
  const int WP = NW / WH;
  const int hw = wave % WH, pw = wave / WH;
  const int h0 = kvh * a.kv_mul + hs * kvm;
  const int p0 = split * a.chunk;
  const int pcap = min(p0 + a.chunk, a.ctx);  // this split's positions, all inside the cache (p0 < ctx)
  const size_t koff = (size_t)kvh * HD + col * EPL;
  __shared__ float so[NW * HPW * HD];
  __shared__ float sml[NW * HPW * 2];
  // position and stop flag: vector loads consumed after the first K/V loads
  // are issued (a scalar read would be waited for before them)
  const int pos_v = cn_load_late(a.pos);
  const int stop_v = cn_load_late(a.stop ? a.stop : &g_never_stop);
  bool first_pass = true;

  for (int jg = 0; jg < kvm; jg += WH * HPW) {
    const int jb = jg + hw * HPW;                      // the wave's first head of this pass
    const int nj = max(0, min(HPW, kvm - jb));         // its heads in this pass
    float q[HPW][EPL], m[HPW], l[HPW], o[HPW][EPL];
#pragma unroll
    for (int j = 0; j < HPW; j++) {
      // straight-line loads: heads past the wave's last re-read a valid head, unused
      const int hq = h0 + min(jb + j, kvm - 1);
      kv_load_n<false, EPL>(a.q, (size_t)hq * HD + col * EPL, q[j]);
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e++) o[j][e] = 0.f;
    }
    // K/V rows of a wave step starting at position pb: rows past the chunk
    // re-read its last position (masked below), so every load is issued
    auto load_step = [&](int pb, float (&kr)[PG][EPL], float (&vr)[PG][EPL]) {
#pragma unroll
      for (int g = 0; g < PG; g++) {
        const int p = min(pb + 4 * g + row, pcap - 1);
        kv_load_n<F16, EPL>(a.kc, (size_t)p * a.kv_dim + koff, kr[g]);
        kv_load_n<F16, EPL>(a.vc, (size_t)p * a.kv_dim + koff, vr[g]);
      }
    };
    // first step: positions below pcap regardless of seq
    int pb = p0 + pw * SP;
    float kr[PG][EPL], vr[PG][EPL];
    load_step(pb, kr, vr);
    if (first_pass) {
      if (__builtin_amdgcn_readfirstlane(stop_v)) return;  // uniform: before any barrier
      first_pass = false;
    }
    const int seq = __builtin_amdgcn_readfirstlane(pos_v) + 1;
    const int p1 = nj > 0 ? min(seq, pcap) : 0;
    while (pb < p1) {  // uniform across the wave
      // the next step's loads go out before this step is computed
      float kn[PG][EPL], vn[PG][EPL];
      load_step(pb + WP * SP, kn, vn);
      float sc[PG][HPW];
#pragma unroll
      for (int g = 0; g < PG; g++) {
        const bool on = pb + 4 * g + row < p1;
        // rows past the sequence hold re-read or stale rows: their scores
        // become -inf and their V rows 0 by selection
#pragma unroll
        for (int e = 0; e < EPL; e++) vr[g][e] = on ? vr[g][e] : 0.f;
#pragma unroll
        for (int j = 0; j < HPW; j++) {
          float t = 0.f;
#pragma unroll
          for (int e = 0; e < EPL; e++) t += q[j][e] * kr[g][e];
          t = row_sum16(t) * a.scale;
          sc[g][j] = on ? t : -INFINITY;
        }
      }
#pragma unroll
      for (int j = 0; j < HPW; j++) {
        if (j >= nj) break;
        float mx = sc[0][j];
#pragma unroll
        for (int g = 1; g < PG; g++) mx = fmaxf(mx, sc[g][j]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, CN_WAVE));
        mx = fmaxf(mx, __shfl_xor(mx, 32, CN_WAVE));
        const float mn = fmaxf(m[j], mx);  // finite: position pb (row 0, g 0) is below p1
        const float c = expf(m[j] - mn);
        float pe[PG], ps = 0.f;
#pragma unroll
        for (int g = 0; g < PG; g++) {
          pe[g] = expf(sc[g][j] - mn);
          ps += pe[g];
        }
        l[j] = l[j] * c + ps;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
          float t = o[j][e] * c;
#pragma unroll
          for (int g = 0; g < PG; g++) t += pe[g] * vr[g][e];
          o[j][e] = t;
        }
        m[j] = mn;
      }
      pb += WP * SP;
#pragma unroll
      for (int g = 0; g < PG; g++)
#pragma unroll
        for (int e = 0; e < EPL; e++) {
          kr[g][e] = kn[g][e];
          vr[g][e] = vn[g][e];
        }
    }
    // rows -> wave: sums and o add across the 4 rows (common running max)
#pragma unroll
    for (int j = 0; j < HPW; j++) {
      if (j >= nj) break;
      l[j] += __shfl_xor(l[j], 16, CN_WAVE);
      l[j] += __shfl_xor(l[j], 32, CN_WAVE);
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        o[j][e] += __shfl_xor(o[j][e], 16, CN_WAVE);
        o[j][e] += __shfl_xor(o[j][e], 32, CN_WAVE);
      }
    }
    if (WP == 1) {
      // the wave's heads are complete over the chunk (a split with positions
      // has them all in wave step 0, so l > 0)
      if (row == 0) {
#pragma unroll
        for (int j = 0; j < HPW; j++) {
          if (j >= nj) break;
#pragma unroll
          for (int e = 0; e < EPL; e++) attn_put<HD>(a, h0 + jb + j, split, col * EPL + e, m[j], l[j], o[j][e]);
        }
      }
      continue;
    }
    // fold the WP position waves of each head through LDS (uniform branch)
#pragma unroll
    for (int j = 0; j < HPW; j++) {
      if (row == 0) {
#pragma unroll
        for (int e = 0; e < EPL; e++) so[(wave * HPW + j) * HD + col * EPL + e] = o[j][e];
      }
      if (lane == 0) {
        sml[2 * (wave * HPW + j)] = j < nj ? m[j] : -INFINITY;
        sml[2 * (wave * HPW + j) + 1] = j < nj ? l[j] : 0.f;
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < WH * HPW * HD; i += CN_BLOCK) {
      const int d = i % HD, jj = (i / HD) % HPW, hh = i / (HD * HPW);  // head jg + hh*HPW + jj
      if (jg + hh * HPW + jj >= kvm) continue;
      float M = -INFINITY;
      for (int w = 0; w < WP; w++) {
        const int sl = (w * WH + hh) * HPW + jj;
        if (sml[2 * sl + 1] > 0.f) M = fmaxf(M, sml[2 * sl]);
      }
      float L = 0.f, acc = 0.f;
      for (int w = 0; w < WP; w++) {
        const int sl = (w * WH + hh) * HPW + jj;
        const float lw = sml[2 * sl + 1];
        if (lw > 0.f) {
          const float f = expf(sml[2 * sl] - M);
          L += lw * f;
          acc += so[sl * HD + d] * f;
        }
      }
      attn_put<HD>(a, h0 + jg + hh * HPW + jj, split, d, M, L, acc);
    }
    __syncthreads();
  }
}

// GreedySampler.Sample: strict '>' scan => the lowest index of the maximum;
// NaN never wins unless it sits at index 0, in which case the answer is 0.
// A decode-loop pick (out_tokens given) does nothing once the loop has
// stopped, and stops it when the winner is the EOS token.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, int n, int* state,
                                                      int* out_tokens, int out_cap) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  // Every logit load of a round is issued before the first comparison (one
  // memory latency per round instead of one per element); the decode
  // loop's stop flag is read as a vector load behind them.
  constexpr int U = 8;  // float4 per thread per round
  const int tid = threadIdx.x;
  const int n4 = n >> 2;
  const float4* l4 = reinterpret_cast<const float4*>(logits);
  float best = -INFINITY;
  int idx = 0x7FFFFFFF;
  for (int base = 0; base < n4; base += 1024 * U) {
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int j = base + u * 1024 + tid;
      v[u] = l4[j < n4 ? j : n4 - 1];
    }
    // a thread's elements come in increasing index order, so the strict '>'
    // keeps the lowest index of its maximum
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int j = base + u * 1024 + tid;
      if (j < n4) {
        const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int k = 0; k < 4; k++)
          if (e[k] > best) {
            best = e[k];
            idx = 4 * j + k;
          }
      }
    }
  }
  if (tid < (n & 3)) {
    const int i = 4 * n4 + tid;
    const float e = logits[i];
    if (e > best) {  // above every element this thread has seen: all have lower indices
      best = e;
      idx = i;
    }
  }
  const int stop = out_tokens ? cn_load_late(state + kDecStop) : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (ov > best || (ov == best && oi < idx)) {
      best = ov;
      idx = oi;
    }
  }
  const int lane = tid & 63, wave = tid >> 6;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (tid == 0 && !stop) {
    best = bv[0];
    idx = bi[0];
    for (int w = 1; w < 16; w++)
      if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
        best = bv[w];
        idx = bi[w];
      }
    if (idx == 0x7FFFFFFF || logits[0] != logits[0]) idx = 0;
    state[kDecTok] = idx;
    if (out_tokens) {
      const int step = state[kDecStep];
      if (step < out_cap) out_tokens[step] = idx;
      state[kDecStep] = step + 1;
      if (idx == state[kDecEos]) state[kDecStop] = 1;
    }
    state[kDecPos] = state[kDecPos] + 1;
  }
}

__global__ __launch_bounds__(CN_BLOCK) void silu_mul_kernel(const float* g, const float* u, float* h, int n) {
  const int i = blockIdx.x * CN_BLOCK + threadIdx.x;
  if (i < n) {
    const float gv = g[i];
    h[i] = (gv / (1.0f + expf(-gv))) * u[i];
  }
}

__global__ void set_state_kernel(int* state, int pos, int tok, int step, int eos) {
  state[kDecPos] = pos;
  state[kDecTok] = tok;
  if (step >= 0) {
    state[kDecStep] = step;
    state[kDecStop] = 0;
    state[kDecEos] = eos;
  }
}

// Heads per wave and pass for a group of kv_mul query heads (four waves split
// the group when kv_mul >= 4), and positions per row per step (register
// budget: K and V rows of the step, q and o of the wave's heads).
int attn_hpw(int kv_mul) {
  const int wh = kv_mul >= 4 ? 4 : (kv_mul >= 2 ? 2 : 1);
  const int need = (kv_mul + wh - 1) / wh;
  return need <= 1 ? 1 : (need <= 2 ? 2 : 4);
}
// (One head per wave at head_dim 128 keeps 8-position steps: four waves then
// cover 32 positions a round, and more chunks spread the work.)
constexpr int attn_pg(int hd, int hpw) {
  return hd <= 64 ? (hpw <= 2 ? 8 : 4) : (hd == 128 ? (hpw == 1 ? 2 : 4) : 2);
}

template <int HD, bool F16, int HPW>
void attn_launch_k(const AttnArgs& a, hipStream_t st) {
  const int n_kv = a.n_heads / a.kv_mul;
  hipLaunchKernelGGL((attn_decode_kernel<HD, F16, HPW, attn_pg(HD, HPW)>), dim3(n_kv * a.hsplit * a.splits),
                     dim3(CN_BLOCK), 0, st, a);
}

template <int HD, bool F16>
hipError_t attn_launch_t(const AttnArgs& a, hipStream_t st) {
  const int hpw = attn_hpw(a.kv_mul / a.hsplit);
  if (hpw == 1) attn_launch_k<HD, F16, 1>(a, st);
  else if (hpw == 2 || HD > 128) attn_launch_k<HD, F16, 2>(a, st);
  else attn_launch_k<HD, F16, 4>(a, st);
  return hipGetLastError();
}

}  // namespace

hipError_t embed_launch(const void* emb, int type, int dim, const int* tok, float* x, hipStream_t st, int n) {
  if (n < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_kernel, dim3((dim + CN_BLOCK - 1) / CN_BLOCK, n), dim3(CN_BLOCK), 0, st, emb,
                     type, dim, tok, x);
  return hipGetLastError();
}

int attn_decode_hsplit(int n_kv_heads, int kv_mul, int splits, int num_cus) {
  // split a kv head's query heads over workgroups while the launch stays within
  // one workgroup per CU and every workgroup keeps at least two heads
  int hs = 1;
  while (kv_mul % (2 * hs) == 0 && kv_mul / (2 * hs) >= 2 && n_kv_heads * 2 * hs * splits <= num_cus) hs *= 2;
  return hs;
}

int attn_decode_round(int head_dim, int kv_mul) {
  const int wh = kv_mul >= 4 ? 4 : (kv_mul >= 2 ? 2 : 1);
  int hpw = attn_hpw(kv_mul);
  if (head_dim > 128 && hpw > 2) hpw = 2;
  return (4 / wh) * 4 * attn_pg(head_dim, hpw);
}

hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t st) {
  if (a.splits < 1 || a.splits > kFoldMaxSplits || a.chunk < 1 || a.head_dim % 16 != 0 || a.hsplit < 1 ||
      a.kv_mul % a.hsplit != 0)
    return hipErrorInvalidValue;
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

hipError_t set_state_launch(int* state, int pos, int tok, int step, hipStream_t st, int eos) {
  hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(1), 0, st, state, pos, tok, step, eos);
  return hipGetLastError();
}

hipError_t silu_mul_launch(const float* g, const float* u, float* h, int n, hipStream_t st) {
  if (n <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + CN_BLOCK - 1) / CN_BLOCK), dim3(CN_BLOCK), 0, st, g, u, h, n);
  return hipGetLastError();
}
