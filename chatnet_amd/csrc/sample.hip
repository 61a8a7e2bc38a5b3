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
// radix select on the float bit patterns (p >= 0, so they order like the
// values), a byte per pass, narrows the keys down to the k-th largest, or
// stops early once at most 64 keys lie at or above the selected bin.  The
// keys at or above that bound are gathered (an index-ordered scan instead
// when more than 1024 tie with the k-th), and a bitonic sort orders them by
// (p descending, index ascending), the first k being the winners: across
// the lanes of one wave for at most 64 keys, in LDS for more.  Equal
// probabilities may therefore come out in another order than the
// reference's quickselect leaves them.  The softmax sum is a tree here and
// a left-to-right sum in the reference (a few ulps apart); the top-p,
// renormalisation and draw loops run in the reference's order on one list
// (wave 0's lanes or LDS), with products kept apart from the sums as the
// reference rounds them.
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

// Element i = tid + 1024j of the vocabulary belongs to thread tid.  REG keeps
// a thread's (at most kRegPerThread) probabilities in registers; otherwise
// they live in the scratch array p (n floats), where each thread only ever
// touches its own elements, so no barrier is needed between the passes.
constexpr int kRegPerThread = 32;

// The unroll pragmas below keep rv[] in registers for REG (32 iterations known
// at compile time); in the scratch-array form the trip count is a run-time
// value and clang reports that it could not unroll, which is expected there.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <bool REG>
__global__ __launch_bounds__(kST) void sample_kernel(const float* __restrict__ logits, int n,
                                                     const SampleParams* __restrict__ prm,
                                                     const float* __restrict__ draws, int* state,
                                                     int* out_tokens, int out_cap, float* __restrict__ p) {
  __shared__ float red[kSW];
  __shared__ int hist[256 * 8];
  __shared__ int sel[3];
  __shared__ int wcnt[2][kSW];
  __shared__ float cp[kSampleMaxK];
  __shared__ int ci[kSampleMaxK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the decode loop's stop flag (set at EOS) and step: vector loads consumed
  // at the end, so the logits loads go out without waiting for them; a
  // stopped loop's launch computes and writes nothing
  const int stop_v = out_tokens ? cn_load_late(state + kDecStop) : 0;
  const int step_v = cn_load_late(state + kDecStep);
  const float inv_temp = prm->inv_temp;
  const float top_p = prm->top_p;
  const int k = prm->top_k < n ? prm->top_k : n;
  const int nj = REG ? kRegPerThread : (n + kST - 1) / kST;
  float rv[REG ? kRegPerThread : 1];
  auto get = [&](int j) -> float {
    if constexpr (REG) return rv[j];
    else return p[tid + kST * j];
  };
  auto put = [&](int j, float x) {
    if constexpr (REG) rv[j] = x;
    else p[tid + kST * j] = x;
  };

  // temperature and softmax (REG: every logits load issued before the first
  // use of the parameters)
  float mx = -INFINITY;
  if constexpr (REG) {
#pragma unroll
    for (int j = 0; j < nj; j++) rv[j] = tid + kST * j < n ? logits[tid + kST * j] : 0.f;
  }
  // this step's draw, loaded while the logits arrive (it waits for the step
  // only, which was loaded first)
  const float r_draw = draws ? draws[step_v] : prm->draw;
#pragma unroll
  for (int j = 0; j < nj; j++) {
    const int i = tid + kST * j;
    const float v = i < n ? __fmul_rn(REG ? rv[j] : logits[i], inv_temp) : -INFINITY;
    if (REG || i < n) put(j, v);
    mx = fmaxf(mx, v);
  }
  mx = st_max(mx, red);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < nj; j++) {
    if (tid + kST * j < n) {
      const float e = expf(get(j) - mx);
      put(j, e);
      s += e;
    }
  }
  s = st_sum(s, red);
  if (s > 0.f) {
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < nj; j++)
      if (tid + kST * j < n) put(j, __fmul_rn(get(j), inv));
  }

  // radix select of the k-th largest key, most significant byte first.  Each
  // bin is counted in 8 lane-striped copies: probabilities share a handful of
  // exponents, and single counters would serialise the LDS atomics.
  uint32_t prefix = 0, pmask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256 * 8; b += kST) hist[b] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < nj; j++) {
      const uint32_t key = __float_as_uint(get(j));
      if (tid + kST * j < n && (key & pmask) == prefix)
        atomicAdd(&hist[(((key >> shift) & 255) << 3) | (lane & 7)], 1);
    }
    __syncthreads();
    if (wave == 0) {
      // lane l holds bins 255-4l .. 252-4l; running sums from the top bin down
      int c[4], s4 = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int b = 255 - 4 * lane - j;
        int v = 0;
#pragma unroll
        for (int r = 0; r < 8; r++) v += hist[(b << 3) | r];
        c[j] = v;
        s4 += v;
      }
      int incl = s4;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, CN_WAVE);
        if (lane >= o) incl += t;
      }
      const int excl = incl - s4;
      if (excl < remaining && remaining <= incl) {  // exactly one lane
        int cum = excl, j = 0;
        for (; j < 3; j++) {
          if (cum + c[j] >= remaining) break;
          cum += c[j];
        }
        sel[0] = 255 - 4 * lane - j;
        sel[1] = remaining - cum;
        sel[2] = c[j];
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sel[0] << shift;
    pmask |= 255u << shift;
    remaining = sel[1];
    // keys at or above the selected bin's lower bound: the k - remaining
    // taken before it and the whole bin.  At most a wave's worth: gather them
    // all now, the sort below still leaves the same k first.
    const int at_or_above = k - sel[1] + sel[2];
    __syncthreads();
    if (at_or_above <= CN_WAVE) break;
  }
  // after all four passes `prefix` is the k-th largest key: keys above it are
  // all taken, of those equal to it the first `remaining` in index order;
  // after an early exit it is the lower bound of a bin, with at most a wave's
  // worth of keys at or above it

  // Gather every key >= prefix in any order: the sort below orders them by
  // (p descending, index ascending), so its first k entries are the winners.
  if (tid == 0) sel[0] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < nj; j++) {
    const int i = tid + kST * j;
    const float v = get(j);
    if (i < n && __float_as_uint(v) >= prefix) {
      const int pos = atomicAdd(&sel[0], 1);
      if (pos < kSampleMaxK) {
        cp[pos] = v;
        ci[pos] = i;
      }
    }
  }
  __syncthreads();
  int m = sel[0];
  if (m > kSampleMaxK) {
    // more keys tie at the k-th value than fit: an ordered scan keeps exactly
    // the k winners, the tied ones with the lowest indices
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    int eq_seen = 0, taken = 0;
#pragma unroll
    for (int j = 0; j < nj; j++) {
      const int i = tid + kST * j;
      const float v = get(j);
      const uint32_t key = i < n ? __float_as_uint(v) : 0u;
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
        cp[pos] = v;
        ci[pos] = i;
      }
      eq_seen += eq_tot;
      taken += t_tot;
      __syncthreads();
    }
    m = k;
  }

  // TemperatureSampler.cs:70-106 in the reference's order on the sorted list
  // in LDS (entry i through P(i) and I(i)): the top-p cutoff, the
  // renormalising sum and the draw, products kept apart from the sums as the
  // reference rounds them
  auto decide = [&](auto P, auto I) -> int {
    float cumulative = 0.f;
    int cutoff = k;
    for (int i = 0; i < k; i++) {
      cumulative += P(i);
      if (cumulative >= top_p) {
        cutoff = i + 1;
        break;
      }
    }
    float sum = 0.f;
    for (int i = 0; i < cutoff; i++) sum += P(i);
    const float inv = 1.0f / sum;
    const float r = r_draw;
    float acc = 0.f;
    int t = I(cutoff - 1);
    for (int i = 0; i < cutoff; i++) {
      acc += __fmul_rn(P(i), inv);
      if (r < acc) {
        t = I(i);
        break;
      }
    }
    return t;
  };
  int tok = 0;
  if (m <= CN_WAVE) {
    // at most a wave's worth of keys: wave 0 sorts them across its lanes with
    // the block sort's network and test below (p descending, then index
    // ascending; lanes past m hold keys that sort last), then makes decide's
    // choice on them, entry i in lane i
    if (wave == 0) {
      float pv = lane < m ? cp[lane] : -1.0f;
      int iv = lane < m ? ci[lane] : 0x7FFFFFFF;
      for (int size = 2; size <= CN_WAVE; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          const float po = __shfl_xor(pv, stride, CN_WAVE);
          const int io = __shfl_xor(iv, stride, CN_WAVE);
          const bool lo = (lane & stride) == 0;  // the pair's lower lane holds a, the upper b
          const float pa = lo ? pv : po, pb = lo ? po : pv;
          const int ia = lo ? iv : io, ib = lo ? io : iv;
          const bool b_first = pb > pa || (pb == pa && ib < ia);
          if (b_first == ((lane & size) == 0)) {
            pv = po;
            iv = io;
          }
        }
      // decide's three loops without a branch per entry: running sums in list
      // order, one add per entry as the reference rounds them, each lane
      // keeping the value after its own entry.  The cutoff is the first lane
      // (below k) whose running sum reaches top_p; the renormalising sum over
      // entries [0, cutoff) is the same sequence of adds, so it is the running
      // sum at cutoff - 1; the draw takes the first lane (below cutoff) whose
      // running sum of products exceeds it, else entry cutoff - 1.
      auto running = [&](float v) {
        float a = 0.f, mine = 0.f;
#pragma unroll
        for (int i = 0; i < CN_WAVE; i++) {
          a += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
          mine = lane == i ? a : mine;
        }
        return mine;
      };
      const float cum = running(pv);
      const uint64_t over = __ballot(lane < k && cum >= top_p);
      const int cutoff = over ? __ffsll((unsigned long long)over) : k;
      const float inv = 1.0f / __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cum), cutoff - 1));
      const float acc = running(__fmul_rn(pv, inv));
      const uint64_t hit = __ballot(lane < cutoff && r_draw < acc);
      tok = __builtin_amdgcn_readlane(iv, hit ? __ffsll((unsigned long long)hit) - 1 : cutoff - 1);
    }
  } else {
    // bitonic sort of the gathered keys: p descending, then index ascending
    int k2 = 1;
    while (k2 < m) k2 <<= 1;
    for (int j = m + tid; j < k2; j += kST) {
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
    if (tid == 0) tok = decide([&](int i) { return cp[i]; }, [&](int i) { return ci[i]; });
  }

  if (tid == 0 && !stop_v) {
    state[kDecTok] = tok;
    if (out_tokens) {
      if (step_v < out_cap) out_tokens[step_v] = tok;
      state[kDecStep] = step_v + 1;
      if (tok == state[kDecEos]) state[kDecStop] = 1;
    }
    state[kDecPos] = state[kDecPos] + 1;
  }
}
#pragma clang diagnostic pop

}  // namespace

hipError_t sample_launch(const float* logits, int n, const SampleParams* params, const float* draws, int* state,
                         int* out_tokens, int out_cap, float* scratch, hipStream_t st) {
  if (n <= kST * kRegPerThread)
    hipLaunchKernelGGL(sample_kernel<true>, dim3(1), dim3(kST), 0, st, logits, n, params, draws, state, out_tokens,
                       out_cap, scratch);
  else
    hipLaunchKernelGGL(sample_kernel<false>, dim3(1), dim3(kST), 0, st, logits, n, params, draws, state, out_tokens,
                       out_cap, scratch);
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
