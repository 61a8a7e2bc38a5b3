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
  tab[idx] = cn_rope_cs(pos, i, dim_inv, neg_log_base);
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
// stored at cache row p0+t, v pairs copied there (LlamaModel.cs:137-153); with
// a bias, q/k/v get it added first (QwenModel.cs:104-125).
// Pair i of row t: from the row itself, or (SPL > 0) as the sum in split
// order of the QKV GEMM's K-split partials [splits][n][ld], exactly as the
// GEMM's reduce would have stored it (((0 + p0) + p1) + ...).
template <int SPL>
__device__ __forceinline__ float2 qkv_pair(const RopeKvArgs& a, int t, int col) {
  if constexpr (SPL == 0) {
    return *reinterpret_cast<const float2*>(a.qkv + (size_t)t * a.ld + col);
  } else {
    float2 pv[SPL];
#pragma unroll
    for (int k = 0; k < SPL; k++)
      pv[k] = *reinterpret_cast<const float2*>(a.part + ((size_t)(k < a.splits ? k : 0) * a.n + t) * a.ld + col);
    float2 s = make_float2(0.f, 0.f);
#pragma unroll
    for (int k = 0; k < SPL; k++)
      if (k < a.splits) {
        s.x += pv[k].x;
        s.y += pv[k].y;
      }
    return s;
  }
}

template <int SPL>
__global__ __launch_bounds__(CN_BLOCK) void rope_kv_kernel(RopeKvArgs a) {
  const int t = blockIdx.y;
  const int pairs_q = a.dim / 2, pairs_kv = a.kv_dim / 2;
  const int i = blockIdx.x * CN_BLOCK + threadIdx.x;
  if (i >= pairs_q + 2 * pairs_kv) return;
  float* row = a.qkv + (size_t)t * a.ld;
  const int pos = a.p0 + t;
  float2 b = make_float2(0.f, 0.f);
  if (a.bias) b = reinterpret_cast<const float2*>(a.bias)[i];
  if (i < pairs_q) {
    float2* p = reinterpret_cast<float2*>(row) + i;
    float2 v = qkv_pair<SPL>(a, t, 2 * i);
    if (a.bias) { v.x += b.x; v.y += b.y; }
    rope_pair(v.x, v.y, a.rope[(size_t)pos * (a.head_dim / 2) + i % (a.head_dim / 2)]);
    *p = v;
    return;
  }
  const bool is_k = i < pairs_q + pairs_kv;
  const int j = is_k ? i - pairs_q : i - pairs_q - pairs_kv;  // pair index within k or v
  float2 v = qkv_pair<SPL>(a, t, a.dim + (is_k ? 0 : a.kv_dim) + 2 * j);
  if (a.bias) { v.x += b.x; v.y += b.y; }
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

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool F16>
__device__ __forceinline__ float4 kv_load4(const void* base, size_t idx) {
  if constexpr (F16) {
    const _Float16* p = reinterpret_cast<const _Float16*>(base) + idx;
    return make_float4((float)p[0], (float)p[1], (float)p[2], (float)p[3]);
  } else {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + idx);
  }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// (a, b) as packed bf16 high parts and packed bf16 low parts (hi + lo carries
// ~16 significant bits; an f16 value is represented exactly).  Pair
// conversions (v_cvt_pk_bf16_f32) and the high parts read back with a shift
// and a mask: three instructions per value.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  const float ha = __builtin_bit_cast(float, hi << 16), hb = __builtin_bit_cast(float, hi & 0xFFFF0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a - ha, b - hb}, bf16x2));
}

__device__ __forceinline__ void split4(float a, float b, float c, float d, uint2& hi, uint2& lo) {
  split2(a, b, hi.x, lo.x);
  split2(c, d, hi.y, lo.y);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Causal GQA attention of a span (LlamaModel.ComputeAttention,
// LlamaModel.cs:241-346, for every token of the span): token t at position
// p0+t, query head h, kv head h / kv_mul,
//   out[t][h] = softmax_p<=p0+t( q . K[p] * scale ) . V[p].
// A workgroup owns 64 rows = QB consecutive tokens x the kv_mul query heads of
// one kv head (QB = floor(64 / kv_mul); when kv_mul does not divide 64 the
// last 64 - QB*kv_mul rows are padding that is never written); wave w owns
// rows 16w..16w+15, lane l the
// row 16w + l%16.  K/V are walked in chunks of 64 positions, staged in LDS as
// bf16 high and low parts (K row-major, V transposed), and both products run
// on v_mfma_f32_16x16x32_bf16 with three passes (hi*hi + hi*lo + lo*hi):
//  - S^T = K Q^T: 16 keys x 16 rows per tile, q held in registers as the B
//    operand; lane l gets the scores of its row against keys 4*(l/16)+0..3 of
//    each tile, so the online softmax (exp2 of scores prescaled by
//    scale*log2 e) is per lane, with two shuffles for the chunk maximum;
//  - O^T = V^T P^T: the probabilities stay in registers as the B operand (the
//    8 k-values of lane l are the 8 keys it scored in two adjacent tiles, and
//    V^T is stored in LDS with its keys in that same order), and lane l
//    accumulates dims 16i + 4*(l/16)+0..3 of its row.
// The workgroup's 8 waves form two groups of 4 that walk alternate chunks
// (group 0 the even ones) with LDS buffers of their own, so two waves share
// each SIMD and the chain of chunks per group is half as long; group 1 hands
// its softmax state and unnormalised output to group 0 through LDS at the end.
// Each group's next chunk is loaded into registers while it computes the
// current one.  The output is written for the O-projection span GEMM: fp16
// hi + lo planes (out, out_lo) in the cn_span_pos order.
constexpr int kSpanThreads = 512;

template <int HD>
constexpr int span_group_lds() {  // bf16 elements of one group's K/V buffers
  return 2 * 64 * (HD + 8) + 2 * HD * (64 + 8);
}

template <int HD, bool F16>
__global__ __launch_bounds__(kSpanThreads) void attn_prefill_kernel(PrefillAttnArgs a) {
  constexpr int KB = 64;                               // positions per chunk
  constexpr int KP = HD + 8;                           // K row pitch (bf16)
  constexpr int VP = KB + 8;                           // V^T row pitch (bf16)
  constexpr int NS = HD / 32;                          // k-steps of q . k
  constexpr int NT = HD / 16;                          // 16-dim output tiles
  constexpr int GT = kSpanThreads / 2;                 // threads per group
  constexpr int KU = KB * (HD / 4) / GT;               // K float4 loads per thread
  constexpr int VU = (KB / 4) * (HD / 4) / GT;         // V 4x4 blocks per thread
  extern __shared__ __align__(16) uint16_t lds_b[];
  const int grp = threadIdx.x / GT;
  uint16_t* Kh = lds_b + grp * span_group_lds<HD>();
  uint16_t* Kl = Kh + KB * KP;
  uint16_t* Vh = Kl + KB * KP;
  uint16_t* Vl = Vh + HD * VP;

  const int tid = threadIdx.x % GT, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int kvh = blockIdx.x;
  const int QB = 64 / a.kv_mul;
  const int t0 = (gridDim.y - 1 - blockIdx.y) * QB;  // longest key ranges dispatched first
  const int r = 16 * w + c;
  const int t = t0 + r / a.kv_mul, hh = kvh * a.kv_mul + r % a.kv_mul;
  const bool real = r < QB * a.kv_mul && t < a.n;
  const int qpos = real ? a.p0 + t : -1;  // -1: padding row, every key masked
  const int t_last = min(a.n, t0 + QB) - 1;
  const int kend = a.p0 + t_last + 1;        // keys [0, kend)

  // q of row r: k-step s, lane group g holds dims 32s + 8g .. +7
  float4 qr[NS][2];
#pragma unroll
  for (int s = 0; s < NS; s++) {
    qr[s][0] = qr[s][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (real) {
      const float* qp = a.qkv + (size_t)t * a.ld + hh * HD + 32 * s + 8 * g;
      qr[s][0] = *reinterpret_cast<const float4*>(qp);
      qr[s][1] = *reinterpret_cast<const float4*>(qp + 4);
    }
  }

  // K/V of one chunk in registers: K as float4 (key, 4 dims), V as 4x4 blocks
  // (4 keys x 4 dims) so the transposed LDS store writes 4 keys at once.
  float4 kr[KU], vr[VU][4];
  const size_t head_off = (size_t)kvh * HD;
  // V block u of this thread: dims 4dq.., keys 4kq...  Each quarter-wave takes
  // 2 dim quads of opposite parity x 8 key quads and each half-wave 4 dim quads,
  // so the transposed 8-byte stores (V^T rows 4dq + e, pitch 36 dwords, 8
  // distinct columns) fall on distinct banks per 16 and per 32 lanes.
  auto vblock = [&](int u, int& dq, int& kq) {
    const int i = tid + GT * u, l = i & 63;
    dq = 4 * (i >> 6) + (l & 1) + 2 * ((l >> 4) & 1);
    kq = 8 * (l >> 5) + ((l >> 1) & 7);
  };
  auto load_chunk = [&](int c0) {
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const int i = tid + GT * u, key = i / (HD / 4), d4 = i % (HD / 4);
      const int p = c0 + key;
      kr[u] = p < kend ? kv_load4<F16>(a.kc, (size_t)p * a.kv_dim + head_off + 4 * d4)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < VU; u++) {
      int dq, kq;
      vblock(u, dq, kq);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int p = c0 + 4 * kq + k;
        vr[u][k] = p < kend ? kv_load4<F16>(a.vc, (size_t)p * a.kv_dim + head_off + 4 * dq)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  // Key kk = 32s + 16h + 4g + v of the chunk sits at V^T column 32s + 8g + 4h + v.
  auto store_chunk = [&]() {
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const int i = tid + GT * u, key = i / (HD / 4), d4 = i % (HD / 4);
      uint2 hi, lo;
      split4(kr[u].x, kr[u].y, kr[u].z, kr[u].w, hi, lo);
      *reinterpret_cast<uint2*>(&Kh[key * KP + 4 * d4]) = hi;
      *reinterpret_cast<uint2*>(&Kl[key * KP + 4 * d4]) = lo;
    }
#pragma unroll
    for (int u = 0; u < VU; u++) {
      int dq, kq;
      vblock(u, dq, kq);
      const int col = 32 * (kq >> 3) + 8 * (kq & 3) + 4 * ((kq >> 2) & 1);
      uint2 hi, lo;
      split4(vr[u][0].x, vr[u][1].x, vr[u][2].x, vr[u][3].x, hi, lo);
      *reinterpret_cast<uint2*>(&Vh[(4 * dq + 0) * VP + col]) = hi;
      *reinterpret_cast<uint2*>(&Vl[(4 * dq + 0) * VP + col]) = lo;
      split4(vr[u][0].y, vr[u][1].y, vr[u][2].y, vr[u][3].y, hi, lo);
      *reinterpret_cast<uint2*>(&Vh[(4 * dq + 1) * VP + col]) = hi;
      *reinterpret_cast<uint2*>(&Vl[(4 * dq + 1) * VP + col]) = lo;
      split4(vr[u][0].z, vr[u][1].z, vr[u][2].z, vr[u][3].z, hi, lo);
      *reinterpret_cast<uint2*>(&Vh[(4 * dq + 2) * VP + col]) = hi;
      *reinterpret_cast<uint2*>(&Vl[(4 * dq + 2) * VP + col]) = lo;
      split4(vr[u][0].w, vr[u][1].w, vr[u][2].w, vr[u][3].w, hi, lo);
      *reinterpret_cast<uint2*>(&Vh[(4 * dq + 3) * VP + col]) = hi;
      *reinterpret_cast<uint2*>(&Vl[(4 * dq + 3) * VP + col]) = lo;
    }
  };

  f32x4 o[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;  // l_part: this lane's keys only

  // group grp walks chunks grp, grp + 2, ...; both groups run the same number
  // of rounds, a group past the last chunk only keeps the barriers
  const int rounds = (kend + 2 * KB - 1) / (2 * KB);
  int c0 = grp * KB;
  if (c0 < kend) load_chunk(c0);

  // q * scale * log2(e) as bf16 hi/lo B operands
  const float qscale = a.scale * 1.4426950408889634f;
  bf16x8 qh[NS], ql[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) {
    uint2 h0, l0, h1, l1;
    split4(qr[s][0].x * qscale, qr[s][0].y * qscale, qr[s][0].z * qscale, qr[s][0].w * qscale, h0, l0);
    split4(qr[s][1].x * qscale, qr[s][1].y * qscale, qr[s][1].z * qscale, qr[s][1].w * qscale, h1, l1);
    qh[s] = as_bf16x8(make_uint4(h0.x, h0.y, h1.x, h1.y));
    ql[s] = as_bf16x8(make_uint4(l0.x, l0.y, l1.x, l1.y));
  }

  for (int it = 0; it < rounds; it++, c0 += 2 * KB) {
    __syncthreads();  // the previous chunk's LDS readers are done
    if (c0 < kend) store_chunk();
    __syncthreads();
    if (c0 >= kend) continue;
    if (c0 + 2 * KB < kend) load_chunk(c0 + 2 * KB);

    f32x4 sc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint16_t* kp = Kh + (16 * j + c) * KP + 32 * s + 8 * g;
        const bf16x8 kh = as_bf16x8(*reinterpret_cast<const uint4*>(kp));
        const bf16x8 kl = as_bf16x8(*reinterpret_cast<const uint4*>(kp + KB * KP));
        sc[j] = mfma16(kh, qh[s], sc[j]);
        sc[j] = mfma16(kh, ql[s], sc[j]);
        sc[j] = mfma16(kl, qh[s], sc[j]);
      }
    }

    // sc[j][v]: key c0 + 16j + 4g + v of row r (log2 domain).  Chunks below
    // the diagonal of the workgroup's first token need no mask (padding rows
    // past n are never written, so they may score anything).
    if (c0 + KB - 1 > a.p0 + t0) {
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int v = 0; v < 4; v++)
          if (c0 + 16 * j + 4 * g + v > qpos) sc[j][v] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int v = 0; v < 4; v++) mx = fmaxf(mx, sc[j][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, CN_WAVE));
    mx = fmaxf(mx, __shfl_xor(mx, 32, CN_WAVE));
    const float m_new = fmaxf(m_run, mx);
    // a row with every key so far masked keeps m = -inf; its sums stay 0
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        sc[j][v] = __builtin_amdgcn_exp2f(sc[j][v] - m_use);
        sum += sc[j][v];
      }
    l_part = l_part * alpha + sum;
#pragma unroll
    for (int i = 0; i < NT; i++) o[i] *= alpha;

#pragma unroll
    for (int s = 0; s < 2; s++) {
      uint2 h0, l0, h1, l1;
      split4(sc[2 * s][0], sc[2 * s][1], sc[2 * s][2], sc[2 * s][3], h0, l0);
      split4(sc[2 * s + 1][0], sc[2 * s + 1][1], sc[2 * s + 1][2], sc[2 * s + 1][3], h1, l1);
      const bf16x8 ph = as_bf16x8(make_uint4(h0.x, h0.y, h1.x, h1.y));
      const bf16x8 pl = as_bf16x8(make_uint4(l0.x, l0.y, l1.x, l1.y));
#pragma unroll
      for (int i = 0; i < NT; i++) {
        const uint16_t* vp = Vh + (16 * i + c) * VP + 32 * s + 8 * g;
        const bf16x8 vh = as_bf16x8(*reinterpret_cast<const uint4*>(vp));
        const bf16x8 vl = as_bf16x8(*reinterpret_cast<const uint4*>(vp + HD * VP));
        o[i] = mfma16(vh, ph, o[i]);
        o[i] = mfma16(vh, pl, o[i]);
        o[i] = mfma16(vl, ph, o[i]);
      }
    }
  }

  float l = l_part + __shfl_xor(l_part, 16, CN_WAVE);
  l += __shfl_xor(l, 32, CN_WAVE);

  // group 1's state to group 0 through LDS (the K/V buffers are free now):
  // the unnormalised output as float4 slots [tile i][lane group g][row], so
  // 16 lanes touch 256 consecutive bytes, then m[64] and l[64]
  float* xs = reinterpret_cast<float*>(lds_b);
  float* xm = xs + 64 * HD;
  __syncthreads();
  if (grp == 1) {
#pragma unroll
    for (int i = 0; i < NT; i++)
      *reinterpret_cast<float4*>(&xs[4 * ((4 * i + g) * 64 + r)]) = make_float4(o[i][0], o[i][1], o[i][2], o[i][3]);
    if (g == 0) {
      xm[r] = m_run;
      xm[64 + r] = l;
    }
  }
  __syncthreads();
  if (grp == 1 || !real) return;
  // group 0 scored key 0 of every real row, so m is finite; a row group 1 never
  // scored has m1 = -inf and weight 0
  const float m1 = xm[r], l1 = xm[64 + r];
  const float m = fmaxf(m_run, m1);
  const float a0 = __builtin_amdgcn_exp2f(m_run - m), a1 = __builtin_amdgcn_exp2f(m1 - m);
  const float inv = 1.0f / (l * a0 + l1 * a1);
  const float s0 = a0 * inv, s1 = a1 * inv;
  const size_t row = (size_t)t * a.ldo;
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const float4 o1 = *reinterpret_cast<const float4*>(&xs[4 * ((4 * i + g) * 64 + r)]);
    const float v0 = o[i][0] * s0 + o1.x * s1, v1 = o[i][1] * s0 + o1.y * s1, v2 = o[i][2] * s0 + o1.z * s1,
                v3 = o[i][3] * s0 + o1.w * s1;
    const int e = hh * HD + 4 * g + 16 * i;  // four adjacent elements, also in the span order
    uint2 hi, lo;
    cn_split_f16x2(v0, v1, hi.x, lo.x);
    cn_split_f16x2(v2, v3, hi.y, lo.y);
    *reinterpret_cast<uint2*>(a.out + row + cn_span_pos(e)) = hi;
    *reinterpret_cast<uint2*>(a.out_lo + row + cn_span_pos(e)) = lo;
  }
}

template <int HD>
size_t prefill_lds_bytes() {
  // the end-of-kernel exchange (64 rows of HD floats, then m and l) fits in
  // group 0's buffers
  static_assert(sizeof(float) * (64 * HD + 128) <= sizeof(uint16_t) * span_group_lds<HD>(), "exchange area");
  return sizeof(uint16_t) * (size_t)(2 * span_group_lds<HD>());
}

template <int HD, bool F16>
hipError_t attn_prefill_t(const PrefillAttnArgs& a, hipStream_t st) {
  const int QB = 64 / a.kv_mul;
  const dim3 grid(a.n_heads / a.kv_mul, (a.n + QB - 1) / QB);
  static std::atomic<uint64_t> lds_done{0};  // > 64 KB of dynamic LDS must be allowed (once per device)
  const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(&attn_prefill_kernel<HD, F16>), lds_done);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_prefill_kernel<HD, F16>), grid, dim3(kSpanThreads), prefill_lds_bytes<HD>(), st, a);
  return hipGetLastError();
}

}  // namespace

bool attn_prefill_supports(int head_dim, int kv_mul) {
  return (head_dim == 64 || head_dim == 128) && kv_mul >= 1 && kv_mul <= 64;
}

hipError_t attn_prefill_launch(const PrefillAttnArgs& a, hipStream_t st) {
  if (!attn_prefill_supports(a.head_dim, a.kv_mul) || a.n <= 0 || !a.out || !a.out_lo) return hipErrorInvalidValue;
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
  const dim3 grid((pairs + CN_BLOCK - 1) / CN_BLOCK, n);
  if (a.splits > 16 || (a.splits > 0 && !a.part)) return hipErrorInvalidValue;
  if (a.splits > 0) {
    RopeKvArgs b = a;
    b.n = n;
    if (a.splits <= 2) hipLaunchKernelGGL(rope_kv_kernel<2>, grid, dim3(CN_BLOCK), 0, st, b);
    else if (a.splits <= 4) hipLaunchKernelGGL(rope_kv_kernel<4>, grid, dim3(CN_BLOCK), 0, st, b);
    else if (a.splits <= 8) hipLaunchKernelGGL(rope_kv_kernel<8>, grid, dim3(CN_BLOCK), 0, st, b);
    else hipLaunchKernelGGL(rope_kv_kernel<16>, grid, dim3(CN_BLOCK), 0, st, b);
  } else {
    hipLaunchKernelGGL(rope_kv_kernel<0>, grid, dim3(CN_BLOCK), 0, st, a);
  }
  return hipGetLastError();
}
