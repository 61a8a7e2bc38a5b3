// gemv_common.h — device pieces shared by the GEMV kernels of gemv.hip
// (quantized weights) and gemv_float.hip (F32 / F16 weights): the virtual-row
// map of a fused launch, the epilogues, and the attention-partial merge that
// the O projection folds into its x staging.
#pragma once

#include "device_common.h"
#include "kernels.h"

namespace {

// The stop flag of launches outside a decode loop (never set).
static __device__ int cn_never_stop = 0;

__device__ __forceinline__ const int* stop_flag(const GemvArgs& a) { return a.stop ? a.stop : &cn_never_stop; }

// x read from the decode attention's per-chunk partials (ADD_MERGE): element
// i belongs to head i / hd; each active chunk c (c < s_eff) holds the running
// max M_c, sum L_c and unnormalised output O_c of its positions, and
//   x = sum_c O_c e^(M_c - M) / sum_c L_c e^(M_c - M),  M = max_c M_c
// (attn_merge_kernel's combination).  Every chunk's loads are issued (their
// addresses do not depend on the position); inactive ones are masked.  The
// weights e^(M_c - M) and the sum depend on the head only: the base-256
// staging (16-element groups of one head) computes them once per group.
struct MergeSrc {
  const float* o;
  const float* ml;
  int hd, splits, s_eff;
};

// ADD_MERGE instances by chunk slots: the epilogue value a launch passes
// (GEMV_EPI_ADD_MERGE, up to kFoldMaxSplits chunks) is dispatched to the
// instance with the fewest slots that hold its chunks, so a launch of 2 or 4
// chunks issues 2 or 4 chunks' loads per element, not kFoldMaxSplits.
constexpr int kEpiMerge4 = 6, kEpiMerge2 = 7;
constexpr bool is_merge(int epi) { return epi == GEMV_EPI_ADD_MERGE || epi == kEpiMerge4 || epi == kEpiMerge2; }
constexpr int merge_slots(int epi) { return epi == kEpiMerge2 ? 2 : (epi == kEpiMerge4 ? 4 : kFoldMaxSplits); }
constexpr int merge_epi(int splits) { return splits <= 2 ? kEpiMerge2 : (splits <= 4 ? kEpiMerge4 : GEMV_EPI_ADD_MERGE); }

// Elements i .. i+3 combined in one round trip: every chunk's (max, sum) and
// outputs are loaded together, then folded.  Used by the base-16 staging,
// whose items (two float4 of one head) gain nothing from sharing the weights.
template <int NS>
__device__ __forceinline__ float4 merged_x4(const MergeSrc& m, int i) {
  const int h = i / m.hd, d = i - h * m.hd;
  const size_t base = (size_t)h * m.splits;
  float2 ml[NS];
  float4 oc[NS];
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < NS; c++) {  // straight-line loads: chunks past splits re-read the last
    const int cc = c < m.splits ? c : m.splits - 1;
    ml[c] = *reinterpret_cast<const float2*>(m.ml + 2 * (base + cc));
    oc[c] = *reinterpret_cast<const float4*>(m.o + (base + cc) * m.hd + d);
    if (c >= m.s_eff) ml[c].y = 0.f;
    if (ml[c].y > 0.f) M = fmaxf(M, ml[c].x);
  }
  float L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int c = 0; c < NS; c++) {
    if (ml[c].y > 0.f) {
      const float f = expf(ml[c].x - M);
      L += ml[c].y * f;
      acc.x += oc[c].x * f;
      acc.y += oc[c].y * f;
      acc.z += oc[c].z * f;
      acc.w += oc[c].w * f;
    }
  }
  return make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L);
}

// Chunk weights of head h: f[c] = e^(M_c - M) for active chunks that hold
// positions (0 otherwise) and their sum L = sum_c L_c f[c].
template <int NS>
struct MergeW {
  float f[NS];
  float L;
};

template <int NS>
__device__ __forceinline__ MergeW<NS> merge_weights(const MergeSrc& m, int h) {
  const size_t base = (size_t)h * m.splits;
  float2 ml[NS];
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < NS; c++) {  // straight-line loads: chunks past splits re-read the last
    ml[c] = *reinterpret_cast<const float2*>(m.ml + 2 * (base + (c < m.splits ? c : m.splits - 1)));
    if (c >= m.s_eff) ml[c].y = 0.f;
    if (ml[c].y > 0.f) M = fmaxf(M, ml[c].x);
  }
  MergeW<NS> w;
  w.L = 0.f;
#pragma unroll
  for (int c = 0; c < NS; c++) {
    w.f[c] = ml[c].y > 0.f ? expf(ml[c].x - M) : 0.f;
    w.L += ml[c].y * w.f[c];
  }
  return w;
}

// Elements d .. d+3 of head h combined with the chunk weights.
template <int NS>
__device__ __forceinline__ float4 merge_apply(const MergeSrc& m, const MergeW<NS>& w, int h, int d) {
  const size_t base = (size_t)h * m.splits;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int c = 0; c < NS; c++) {
    // chunks past splits re-read the last one (finite: every chunk of the
    // launch is written each step) with weight 0
    const float4 o = *reinterpret_cast<const float4*>(m.o + (base + (c < m.splits ? c : m.splits - 1)) * m.hd + d);
    acc.x += o.x * w.f[c];
    acc.y += o.y * w.f[c];
    acc.z += o.z * w.f[c];
    acc.w += o.w * w.f[c];
  }
  return make_float4(acc.x / w.L, acc.y / w.L, acc.z / w.L, acc.w / w.L);
}

// Segment base pointer and row count by run-time segment index, chosen with
// masks: indexing the kernel-argument arrays (or a select chain, which the
// compiler turns into a table) would copy them to scratch, and a scratch load
// waits on every vector-memory operation in flight.
__device__ __forceinline__ const cn_gbyte* seg_w(const GemvArgs& a, int seg) {
  const uintptr_t w0 = reinterpret_cast<uintptr_t>(a.w[0]);
  const uintptr_t w1 = reinterpret_cast<uintptr_t>(a.w[1]);
  const uintptr_t w2 = reinterpret_cast<uintptr_t>(a.w[2]);
  const uintptr_t m1 = 0 - (uintptr_t)(seg == 1), m2 = 0 - (uintptr_t)(seg == 2);
  return (const cn_gbyte*)(w0 ^ ((w0 ^ w1) & m1) ^ ((w0 ^ w2) & m2));
}
__device__ __forceinline__ int seg_n(const GemvArgs& a, int seg) {
  return seg == 0 ? a.seg_rows[0] : (seg == 1 ? a.seg_rows[1] : a.seg_rows[2]);
}

// Virtual row -> (segment, row-in-segment).
template <int EPI>
__device__ __forceinline__ void map_row(const GemvArgs& a, int vr, int& seg, int& r) {
  if constexpr (EPI == GEMV_EPI_SWIGLU) {
    seg = vr & 1;
    r = vr >> 1;
  } else if constexpr (EPI == GEMV_EPI_QKV) {
    if (vr < a.seg_rows[0]) { seg = 0; r = vr; }
    else if (vr < a.seg_rows[0] + a.seg_rows[1]) { seg = 1; r = vr - a.seg_rows[0]; }
    else { seg = 2; r = vr - a.seg_rows[0] - a.seg_rows[1]; }
  } else {
    seg = 0;
    r = vr;
  }
}

// What an epilogue reads besides the dot products, loaded by the lane that
// finishes the rows together with the weights of the same iteration, so the
// epilogue does not wait on a load issued behind the next iteration's weights:
//   ADD: the residual rows;
//   QKV: with a bias (QwenModel.cs:104-120) the rows' biases in
//        res[RPW..2*RPW); the (cos, sin) of the row pairs go to res[0..RPW)
//        once the position is known (load_rope).
template <int EPI, int RPW>
constexpr int res_count() { return EPI == GEMV_EPI_QKV ? 2 * RPW : RPW; }

// Loaded by every lane (the lanes of a row group read the same addresses),
// rows past n_vrows clamped to the last one: straight-line loads, so the
// compiler's count of loads in flight stays exact (see issue_loads).
template <int EPI, int RPW, int NR>
__device__ __forceinline__ void load_residual(const GemvArgs& a, int vr0, int li, int pos, float (&res)[NR]) {
  (void)li;
#pragma unroll
  for (int i = 0; i < NR; i++) res[i] = 0.f;
  if constexpr (EPI == GEMV_EPI_ADD || is_merge(EPI)) {
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int vr = vr0 + i < a.n_vrows ? vr0 + i : a.n_vrows - 1;
      res[i] = a.out[0][vr];
    }
  } else if constexpr (EPI == GEMV_EPI_QKV) {
    (void)pos;
#pragma unroll
    for (int i = 0; i < RPW; i += 2) {
      const int vr = vr0 + i < a.n_vrows ? vr0 + i : a.n_vrows - 2;
      if (a.bias) {
        const float2 b = *reinterpret_cast<const float2*>(a.bias + vr);
        res[RPW + i] = b.x;
        res[RPW + i + 1] = b.y;
      }
    }
  }
}

// QKV: (cos, sin) of each q/k row pair at position pos from the RoPE table
// (TensorMath.ApplyRoPE's angle, TensorMath.cs:418-432; the pair index is the
// row's offset within its head) into res[0..RPW).  Issued once the position
// is known, after x is staged, so the table loads (cache hits) are covered by
// the dot product; v rows (segment 2) read an entry they do not use.
template <int EPI, int RPW, int NR>
__device__ __forceinline__ void load_rope(const GemvArgs& a, int vr0, int pos, float (&res)[NR]) {
  if constexpr (EPI == GEMV_EPI_QKV) {
#pragma unroll
    for (int i = 0; i < RPW; i += 2) {
      const int vr = vr0 + i < a.n_vrows ? vr0 + i : a.n_vrows - 2;
      int seg, r;
      map_row<EPI>(a, vr, seg, r);
      const float2 cs = a.rope[(size_t)pos * (a.head_dim / 2) + (r % a.head_dim) / 2];
      res[i] = cs.x;
      res[i + 1] = cs.y;
    }
  }
}

// pos: the device-side position (QKV), read at kernel start; res: what
// load_residual fetched for these rows.
// QKV (RoPE pairs) and SwiGLU (gate/up pairs) take the rows of a lane two at a
// time and need an even RPW; the store and add forms also take one row.
template <int EPI, int RPW>
__device__ __forceinline__ void epilogue(const GemvArgs& a, int vr0, const float* v, const float* res, int pos) {
  static_assert(RPW % 2 == 0 || (EPI != GEMV_EPI_QKV && EPI != GEMV_EPI_SWIGLU),
                "the QKV and SwiGLU epilogues take rows in pairs");
#pragma unroll
  for (int i = 0; i < RPW; i += 2) {
    const int vr = vr0 + i;
    if (vr >= a.n_vrows) return;
    int seg, r;
    map_row<EPI>(a, vr, seg, r);
    if constexpr (EPI == GEMV_EPI_STORE || EPI == GEMV_EPI_LOGITS) {
      a.out[0][r] = v[i];
      if constexpr (RPW >= 2) {
        if (vr + 1 < a.n_vrows) a.out[0][r + 1] = v[i + 1];
      }
    } else if constexpr (EPI == GEMV_EPI_ADD || is_merge(EPI)) {
      a.out[0][r] = res[i] + v[i];
      if constexpr (RPW >= 2) {
        if (vr + 1 < a.n_vrows) a.out[0][r + 1] = res[i + 1] + v[i + 1];
      }
    } else if constexpr (EPI == GEMV_EPI_SWIGLU) {
      const float g = v[i], u = v[i + 1];
      a.out[0][r] = (g / (1.0f + expf(-g))) * u;
    } else {  // QKV
      float x0 = v[i], x1 = v[i + 1];
      if (a.bias) {  // q/k/v += bias before RoPE (QwenModel.cs:104-125)
        x0 += res[RPW + i];
        x1 += res[RPW + i + 1];
      }
      if (seg < 2) {  // RoPE of the pair (TensorMath.cs:408-458), (cos, sin) from load_rope
        const float c = res[i], s = res[i + 1];
        const float y0 = x0 * c - x1 * s;
        const float y1 = x0 * s + x1 * c;
        x0 = y0;
        x1 = y1;
      }
      if (seg == 0) {
        a.out[0][r] = x0;
        a.out[0][r + 1] = x1;
      } else {
        const size_t off = (size_t)pos * a.kv_dim + r;
        // K or V cache base chosen arithmetically: a select of the two pointer
        // arguments compiles to a scratch table whose load waits on every
        // vector-memory operation in flight
        const uintptr_t kb = reinterpret_cast<uintptr_t>(a.kcache), vb = reinterpret_cast<uintptr_t>(a.vcache);
        const uintptr_t base = vb + ((kb - vb) & (uintptr_t)(0 - (uintptr_t)(seg == 1)));
        if (a.kv_f16) {
          CN_GLOBAL _Float16* dst = (CN_GLOBAL _Float16*)base + off;
          dst[0] = (_Float16)x0;
          dst[1] = (_Float16)x1;
        } else {
          CN_GLOBAL float* dst = (CN_GLOBAL float*)base + off;
          dst[0] = x0;
          dst[1] = x1;
        }
      }
    }
  }
}

}  // namespace
