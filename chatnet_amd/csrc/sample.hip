// sample.hip — TemperatureSampler.Sample
// (src/ChatNet.Core/Samplers/TemperatureSampler.cs:33-112) on the device, and
// the seeded System.Random whose draws it consumes.
//
// One workgroup of 1024 threads over the last logits:
//   p[i] = logits[i] * (1/T)                                   (:50-55)
//   softmax (TensorMath.Softmax, TensorMath.cs:177-241)         (:58)
//   the k = min(top_k, n) largest p, descending                 (:62-67)
//   cutoff = first i with sum(p[0..i]) >= top_p, else k         (:70-80)
//   renormalise the cutoff tokens, first i with r < acc         (:83-106)
// The reference finds the top k by quickselect and insertion sort; here a
// 4-pass radix select on the float bit patterns (p >= 0, so they order like
// the values) finds the k-th largest key, the k winners are gathered in index
// order, and a bitonic sort in LDS orders them by (p descending, index
// ascending).  Equal probabilities may therefore come out in another order
// than the reference's quickselect leaves them.  The softmax sum is a tree
// here and a left-to-right sum in the reference (a few ulps apart); the
// top-p, renormalisation and draw loops run on one thread in the reference's
// order, with products kept apart from the sums as the reference rounds them.
#include "device_common.h"
#include "kernels.h"

namespace {

constexpr int kST = 1024;  // threads of the sampler workgroup
constexpr int kSW = kST / CN_WAVE;

__device__ __forceinline__ float st_max(float v, float* red) {
  v = cn_wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kSW; w++) m = fmaxf(m, red[w]);
  __syncthreads();  // red is reused by the next reduction
  return m;
}

__device__ __forceinline__ float st_sum(float v, float* red) {
  v = cn_wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kSW; w++) s += red[w];
  __syncthreads();
  return s;
}

// p is a scratch array of n floats; each thread only ever touches its own
// elements i = tid + 1024j, so no barrier is needed between the passes over it.
__global__ __launch_bounds__(kST) void sample_kernel(const float* __restrict__ logits, int n,
                                                     const SampleParams* __restrict__ prm,
                                                     const float* __restrict__ draws, int* state,
                                                     int* out_tokens, int out_cap, float* __restrict__ p) {
  __shared__ float red[kSW];
  __shared__ int hist[256];
  __shared__ int sel[2];
  __shared__ int wcnt[2][kSW];
  __shared__ float cp[kSampleMaxK];
  __shared__ int ci[kSampleMaxK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float inv_temp = prm->inv_temp;
  const float top_p = prm->top_p;
  const int k = prm->top_k < n ? prm->top_k : n;

  // temperature and softmax
  float mx = -INFINITY;
  for (int i = tid; i < n; i += kST) {
    const float v = __fmul_rn(logits[i], inv_temp);
    p[i] = v;
    mx = fmaxf(mx, v);
  }
  mx = st_max(mx, red);
  float s = 0.f;
  for (int i = tid; i < n; i += kST) {
    const float e = expf(p[i] - mx);
    p[i] = e;
    s += e;
  }
  s = st_sum(s, red);
  if (s > 0.f) {
    const float inv = 1.0f / s;
    for (int i = tid; i < n; i += kST) p[i] = __fmul_rn(p[i], inv);
  }

  // radix select of the k-th largest key, most significant byte first
  uint32_t prefix = 0, pmask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256; b += kST) hist[b] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kST) {
      const uint32_t key = __float_as_uint(p[i]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int cum = 0, d = 255;
      for (; d > 0; d--) {
        if (cum + hist[d] >= remaining) break;
        cum += hist[d];
      }
      sel[0] = d;
      sel[1] = remaining - cum;
    }
    __syncthreads();
    prefix |= (uint32_t)sel[0] << shift;
    pmask |= 255u << shift;
    remaining = sel[1];
    __syncthreads();
  }
  // keys above `prefix` are all taken; of those equal to it, the first
  // `remaining` in index order

  // gather the k winners in index order
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  int eq_seen = 0, taken = 0;
  for (int base = 0; base < n; base += kST) {
    const int i = base + tid;
    const uint32_t key = i < n ? __float_as_uint(p[i]) : 0u;
    const bool gt = i < n && key > prefix;
    const bool eq = i < n && key == prefix;
    const uint64_t beq = __ballot(eq);
    if (lane == 0) wcnt[0][wave] = __popcll(beq);
    __syncthreads();
    int eq_before = eq_seen + __popcll(beq & below), eq_tot = 0;
    for (int w = 0; w < kSW; w++) {
      if (w < wave) eq_before += wcnt[0][w];
      eq_tot += wcnt[0][w];
    }
    const bool take = gt || (eq && eq_before < remaining);
    const uint64_t bt = __ballot(take);
    if (lane == 0) wcnt[1][wave] = __popcll(bt);
    __syncthreads();
    int pos = taken + __popcll(bt & below), t_tot = 0;
    for (int w = 0; w < kSW; w++) {
      if (w < wave) pos += wcnt[1][w];
      t_tot += wcnt[1][w];
    }
    if (take && pos < kSampleMaxK) {
      cp[pos] = p[i];
      ci[pos] = i;
    }
    eq_seen += eq_tot;
    taken += t_tot;
    __syncthreads();
  }

  // bitonic sort of the winners: p descending, then index ascending
  int k2 = 1;
  while (k2 < k) k2 <<= 1;
  for (int j = k + tid; j < k2; j += kST) {
    cp[j] = -1.0f;
    ci[j] = 0x7FFFFFFF;
  }
  __syncthreads();
  for (int size = 2; size <= k2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const int o = tid ^ stride;
      if (tid < k2 && o > tid) {
        const bool first = (tid & size) == 0;
        const float pa = cp[tid], pb = cp[o];
        const int ia = ci[tid], ib = ci[o];
        const bool b_first = pb > pa || (pb == pa && ib < ia);
        if (b_first == first) {
          cp[tid] = pb;
          cp[o] = pa;
          ci[tid] = ib;
          ci[o] = ia;
        }
      }
      __syncthreads();
    }
  }

  if (tid == 0) {
    float cumulative = 0.f;
    int cutoff = k;
    for (int i = 0; i < k; i++) {
      cumulative += cp[i];
      if (cumulative >= top_p) {
        cutoff = i + 1;
        break;
      }
    }
    float sum = 0.f;
    for (int i = 0; i < cutoff; i++) sum += cp[i];
    const float inv = 1.0f / sum;
    const int step = state[2];
    const float r = draws ? draws[step] : prm->draw;
    float acc = 0.f;
    int tok = ci[cutoff - 1];
    for (int i = 0; i < cutoff; i++) {
      acc += __fmul_rn(cp[i], inv);
      if (r < acc) {
        tok = ci[i];
        break;
      }
    }
    state[1] = tok;
    if (out_tokens && step < out_cap) out_tokens[step] = tok;
    state[2] = step + 1;
    state[0] = state[0] + 1;
  }
}

}  // namespace

hipError_t sample_launch(const float* logits, int n, const SampleParams* params, const float* draws, int* state,
                         int* out_tokens, int out_cap, float* scratch, hipStream_t st) {
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kST), 0, st, logits, n, params, draws, state, out_tokens, out_cap,
                     scratch);
  return hipGetLastError();
}

// System.Random(int seed): the .NET BCL's seeded compat generator, Knuth's
// subtractive method after Numerical Recipes in C (2nd ed.) "ran3":
// MBIG = int.MaxValue, MSEED = 161803398, a 55-entry table with lags 21/55,
// NextDouble = InternalSample * (1.0 / MBIG).  TemperatureSampler constructs
// one per sampler (TemperatureSampler.cs:29) and draws once per Sample (:97).
NetRandom::NetRandom(int32_t seed) {
  const int32_t mbig = 2147483647, mseed = 161803398;
  const int32_t subtraction = seed == INT32_MIN ? INT32_MAX : (seed < 0 ? -seed : seed);
  int32_t mj = mseed - subtraction;
  a_[0] = 0;
  a_[55] = mj;
  int32_t mk = 1;
  for (int i = 1; i < 55; i++) {
    const int ii = (21 * i) % 55;
    a_[ii] = mk;
    mk = mj - mk;
    if (mk < 0) mk += mbig;
    mj = a_[ii];
  }
  for (int k = 1; k < 5; k++)
    for (int i = 1; i < 56; i++) {
      a_[i] -= a_[1 + (i + 30) % 55];
      if (a_[i] < 0) a_[i] += mbig;
    }
  inext_ = 0;
  inextp_ = 21;
}

int32_t NetRandom::internal_sample() {
  const int32_t mbig = 2147483647;
  if (++inext_ >= 56) inext_ = 1;
  if (++inextp_ >= 56) inextp_ = 1;
  int32_t v = a_[inext_] - a_[inextp_];
  if (v == mbig) v--;
  if (v < 0) v += mbig;
  a_[inext_] = v;
  return v;
}

double NetRandom::next_double() { return internal_sample() * (1.0 / 2147483647); }
