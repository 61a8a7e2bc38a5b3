// gemv.hip — fused dequant-GEMV for batch-1 decode on gfx950.
//
// Replaces TensorMath.MatVecMulQ4_0 / MatVecMulQ6K / MatVecMulGeneric
// (src/ChatNet.Core/Tensors/TensorMath.cs:548-656) and the fused row dots
// DequantQ4_0.DotProduct (DequantQ4_0.cs:80-149), DequantQ4K.DotProduct
// (DequantQ4K.cs:89-163), DequantQ6K.DotProduct (DequantQ6K.cs:104-188),
// DequantQ8_0.DotProduct and DequantQ5K.DotProduct.
//
// Weights stay in their raw GGUF block layout in HBM.  One lane owns one
// "unit" of a row — two Q4_0 or Q8_0 blocks (64 weights, 36 / 68 B, dword
// aligned), or half a Q4_K / Q5_K / Q6_K super-block (128 weights plus the
// header or scales it needs; Q6_K realigned in registers) — and LPR lanes
// cover a row, so a wave reads each row as one contiguous stretch.  Every lane
// works on RPW rows at once so each x value it reads from LDS feeds RPW rows.
// The input vector is staged in LDS once per workgroup as integer digits (with
// RMSNorm's weight fused in when one is given, TensorMath.RmsNorm
// TensorMath.cs:97-165; the 1/rms factor is applied to the finished sums):
// x is scaled by a power of two per 32- or 16-element group to 19 significant
// bits and split into base-16 digits (Q4_0, short Q4_K rows: signed weight
// nibbles on v_dot8_i32_i4) or base-256 digits (Q8_0, Q5_K, Q6_K, long Q4_K
// rows: weight bytes on v_dot4_i32_i8).  Each group's dot is exact in int32;
// the per-group scales, offsets (q-8, q-32, dmin*m) and 2^-e are applied in
// fp32 once per group.  Partial row sums are reduced across the LPR lanes with
// cross-lane shuffles.
//
// Epilogues (fused into the lane that finishes a row pair):
//   STORE   y[r]  = dot                          (LM head, matmul API)
//   ADD     y[r] += dot                          (O / down + residual, TensorMath.Add :712-733)
//   QKV     RoPE on q/k pairs + K/V cache write  (TensorMath.ApplyRoPE :408-458, LlamaModel.cs:146-153)
//   SWIGLU  h[r] = silu(gate[r]) * up[r]         (TensorMath.SiluElementwiseMul :253-286)
#include <cstring>

#include "device_common.h"
#include "gemv_common.h"
#include "kernels.h"

namespace {

constexpr int QT_Q4_0 = 2, QT_Q8_0 = 8, QT_Q3_K = 11, QT_Q4_K = 12, QT_Q5_K = 13, QT_Q6_K = 14;
// Q6_K rows read in quarter super-blocks (64 weights per lane unit): the
// launch shape of rows of 65..96 half super-blocks (8192 < K <= 12288).
constexpr int QT_Q6_KQ = 114;

template <int QT> struct QTraits;
template <> struct QTraits<QT_Q4_0> {
  static constexpr int UNIT = 64;        // weights per lane unit
  static constexpr int NDW = 9;          // dwords held per unit
  static constexpr int BLOCK_BYTES = 18, BLOCK = 32;
};
// K-quant units are half super-blocks (128 weights): the dwords a lane holds
// are the super-block header or scales plus that half's quants (load_unit).
template <> struct QTraits<QT_Q4_K> {
  static constexpr int UNIT = 128, NDW = 20;
  static constexpr int BLOCK_BYTES = 144, BLOCK = 256;
};
template <> struct QTraits<QT_Q6_K> {
  static constexpr int UNIT = 128, NDW = 27;
  static constexpr int BLOCK_BYTES = 210, BLOCK = 256;
};
template <> struct QTraits<QT_Q6_KQ> {
  static constexpr int UNIT = 64, NDW = 15;
  static constexpr int BLOCK_BYTES = 210, BLOCK = 256;
};
template <> struct QTraits<QT_Q3_K> {
  static constexpr int UNIT = 128, NDW = 16;
  static constexpr int BLOCK_BYTES = 110, BLOCK = 256;
};
template <> struct QTraits<QT_Q8_0> {
  static constexpr int UNIT = 64, NDW = 17;  // two 34-byte blocks
  static constexpr int BLOCK_BYTES = 34, BLOCK = 32;
};
template <> struct QTraits<QT_Q5_K> {
  static constexpr int UNIT = 128, NDW = 24;
  static constexpr int BLOCK_BYTES = 176, BLOCK = 256;
};

// ---------------------------------------------------------------------------
// Q4_0 inputs as signed 4-bit digits.
//
// For the Q4_0 GEMV, x is staged in LDS as integers so that v_dot8_i32_i4 can
// multiply raw weight nibbles exactly: per 32-element block b,
//   s_b = 18 - e_b  with max|x_b| = f * 2^e_b, f in [0.5, 1)   (so |X| <= 2^18)
//   X_j = rint(x_j * 2^s_b) = sum_{d<5} D_{j,d} 16^d,  D in [-8, 7]
// A weight dword XOR 0x88888888 holds (q - 8) as eight signed nibbles, so
//   sum_j (q_j - 8) X_j = Horner over d of dot8(qs ^ 0x88888888, D_d)
// is exact in int32 (|.| <= 32 * 8 * 2^18), and the block contributes
// fp16(d_b) * 2^-s_b * that integer.  X carries 19 significant bits relative
// to the block maximum; the GEMV's normwise deviation from an fp32 dot is
// about 4e-6.
// LDS record of unit u (blocks 2u and 2u+1): 44 dwords,
//   dword blk*20 + d*4 + k: nibble 2i = digit d of element 4k+i, nibble 2i+1 =
//   digit d of element 16+4k+i (the nibble order of qs dword k, and of a Q4_K
//   sub-block's 16 qs bytes, DequantQ4K.cs:59-72);
//   dword 40 + blk = s_b;  dword 42 + blk = sum_j X_j of the block (written
//   for the Q4_K dot, whose per-block min term needs it).  The 44-dword stride
//   keeps 16-byte reads of 16 neighbouring lanes on distinct banks.
// ---------------------------------------------------------------------------
constexpr int XD_UNIT_DW = 44;

// Balanced base-16 digits without carries: with E_d = D_d + 8 in [0, 15],
// sum_d 16^d E_d = X + 0x88888, so the nibbles of (X + 0x88888) are the E_d and
// XOR 8 turns each into D_d = E_d - 8 as a signed nibble.  Valid for
// X in [-0x88888, 0x77777], which |X| <= 2^18 satisfies.

// x (and the RMSNorm weight) of the MAXT work items a thread stages.
// Work item t = (block t/4, dword k = t%4) holds x[32b+4k..+3] and
// x[32b+16+4k..+3]; thread i owns items i, i+256, ...
template <int MAXT, bool NORM>
struct XStage {
  float x[MAXT][8];
  float g[MAXT][8];
};
template <int MAXT>
struct XStage<MAXT, false> {
  float x[MAXT][8];
};

// Issues every load of the staged x before the caller issues its weight
// loads: vector-memory counters retire in order, so loads issued after the
// weight stream could not be consumed before the whole stream had landed.
// Every load is issued unconditionally (threads past the last item re-read
// the last one; stage_digitize ignores them): a load issued on only some paths leaves
// the compiler unable to count the loads after x, and it then waits for all
// of them, weights included.  BS threads stage the K/8 items, item t on
// thread t % BS.
template <int MAXT, bool NORM, int BS, bool MERGE = false>
__device__ __forceinline__ void stage_load(const float* __restrict__ x, const float* __restrict__ norm_w, int K,
                                           XStage<MAXT, NORM>& st, const MergeSrc& ms = MergeSrc{}) {
  const int ntask = K >> 3;
#pragma unroll
  for (int j = 0; j < MAXT; j++) {
    const int t = threadIdx.x + BS * j;
    const bool on = t < ntask;
    const int tc = on ? t : ntask - 1;
    const int b = tc >> 2, k = tc & 3;
    float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo, glo = lo, ghi = lo;
    if constexpr (!MERGE) {  // merged x: stage_merge_load / stage_merge
      lo = *reinterpret_cast<const float4*>(x + 32 * b + 4 * k);
      hi = *reinterpret_cast<const float4*>(x + 32 * b + 16 + 4 * k);
    }
    if constexpr (NORM) {
      glo = *reinterpret_cast<const float4*>(norm_w + 32 * b + 4 * k);
      ghi = *reinterpret_cast<const float4*>(norm_w + 32 * b + 16 + 4 * k);
    }
    st.x[j][0] = lo.x; st.x[j][1] = lo.y; st.x[j][2] = lo.z; st.x[j][3] = lo.w;
    st.x[j][4] = hi.x; st.x[j][5] = hi.y; st.x[j][6] = hi.z; st.x[j][7] = hi.w;
    if constexpr (NORM) {
      st.g[j][0] = glo.x; st.g[j][1] = glo.y; st.g[j][2] = glo.z; st.g[j][3] = glo.w;
      st.g[j][4] = ghi.x; st.g[j][5] = ghi.y; st.g[j][6] = ghi.z; st.g[j][7] = ghi.w;
    }
  }
}

// x of the base-16 staging read from the decode attention's chunk partials
// (ADD_MERGE), in two phases so the weight loads need not wait for them:
// stage_merge_load issues the loads of every chunk's (max, sum) and outputs
// for the thread's items (the two float4 of an item lie in one head: 32-element
// blocks never straddle a head), then, after the caller has issued its weight
// loads, stage_merge combines them as merged_x4 does.
template <int MAXT, int NS>
struct XMerge {
  float2 ml[MAXT][NS];
  float4 lo[MAXT][NS], hi[MAXT][NS];
};

template <int MAXT, int BS, int NS>
__device__ __forceinline__ void stage_merge_load(const MergeSrc& m, int K, XMerge<MAXT, NS>& r) {
  const int ntask = K >> 3;
#pragma unroll
  for (int j = 0; j < MAXT; j++) {
    const int t = threadIdx.x + BS * j;
    const int tc = t < ntask ? t : ntask - 1;
    const int i = 32 * (tc >> 2) + 4 * (tc & 3);  // first element of the item's low float4
    const int h = i / m.hd, d = i - h * m.hd;
    const size_t base = (size_t)h * m.splits;
#pragma unroll
    for (int c = 0; c < NS; c++) {  // chunks past splits re-read the last one, weight 0
      const size_t s = base + (c < m.splits ? c : m.splits - 1);
      r.ml[j][c] = *reinterpret_cast<const float2*>(m.ml + 2 * s);
      r.lo[j][c] = *reinterpret_cast<const float4*>(m.o + s * m.hd + d);
      r.hi[j][c] = *reinterpret_cast<const float4*>(m.o + s * m.hd + d + 16);
    }
  }
}

template <int MAXT, bool NORM, int NS>
__device__ __forceinline__ void stage_merge(const MergeSrc& m, const XMerge<MAXT, NS>& r, XStage<MAXT, NORM>& st) {
#pragma unroll
  for (int j = 0; j < MAXT; j++) {
    float2 ml[NS];
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < NS; c++) {
      ml[c] = r.ml[j][c];
      if (c >= m.s_eff) ml[c].y = 0.f;
      if (ml[c].y > 0.f) M = fmaxf(M, ml[c].x);
    }
    float L = 0.f;
    float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo;
#pragma unroll
    for (int c = 0; c < NS; c++) {
      if (ml[c].y > 0.f) {
        const float f = expf(ml[c].x - M);
        L += ml[c].y * f;
        lo.x += r.lo[j][c].x * f; lo.y += r.lo[j][c].y * f; lo.z += r.lo[j][c].z * f; lo.w += r.lo[j][c].w * f;
        hi.x += r.hi[j][c].x * f; hi.y += r.hi[j][c].y * f; hi.z += r.hi[j][c].z * f; hi.w += r.hi[j][c].w * f;
      }
    }
    st.x[j][0] = lo.x / L; st.x[j][1] = lo.y / L; st.x[j][2] = lo.z / L; st.x[j][3] = lo.w / L;
    st.x[j][4] = hi.x / L; st.x[j][5] = hi.y / L; st.x[j][6] = hi.z / L; st.x[j][7] = hi.w / L;
  }
}

// Writes the digit records of x * norm_w (x alone without NORM).  RMSNorm's
// scale rms = 1/sqrt(sum x^2 / K + eps) (TensorMath.cs:142) is one positive
// factor per token, so it is applied to the finished dot products instead of
// to every element; each wave leaves its share of sum x^2 in red[wave] for the
// caller to combine after its __syncthreads().  The four items of a block sit
// in adjacent lanes and share the block maximum through two xor-shuffles.
template <int MAXT, bool NORM, int BS, bool BSUM = false>
__device__ __forceinline__ void stage_digitize(const XStage<MAXT, NORM>& st, int K, uint32_t* xd, float* red) {
  const int ntask = K >> 3;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < MAXT; j++) {
    const int t = threadIdx.x + BS * j;
    const bool on = t < ntask;
    const int b = t >> 2, k = t & 3;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      v[i] = st.x[j][i];
      ss += on ? v[i] * v[i] : 0.f;  // threads past the last item hold a re-read item
    }
    if constexpr (NORM) {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = v[i] * st.g[j][i];
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1, CN_WAVE));
    m = fmaxf(m, __shfl_xor(m, 2, CN_WAVE));
    int e = 0;
    (void)frexpf(m, &e);
    const int s = m > 0.f ? 18 - e : 0;
    // X + 0x88888 lands in the low 20 bits of a float: 13142152 = 1.5 * 2^23 +
    // 0x88888, and the add rounds ldexp(v, s) (|.| <= 2^18, exact) to the
    // nearest integer exactly as a round-to-nearest-even conversion would.
    uint32_t tl[4], th[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      tl[i] = __float_as_uint(ldexpf(v[i], s) + 13142152.0f);
      th[i] = __float_as_uint(ldexpf(v[4 + i], s) + 13142152.0f);
    }
    // E_i bytes 0..2: digits 0, 2, 4 of the pair (tl_i in the low nibble, th_i
    // in the high one); O_i bytes 0..1: digits 1, 3.  Byte permutes then
    // gather byte d/2 of E (or O) of the four pairs into digit word d, and one
    // XOR per word turns the biased nibbles E = D + 8 into signed digits.
    constexpr uint32_t M = 0x000F0F0Fu;
    uint32_t E[4], O[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      E[i] = (tl[i] & M) | ((th[i] << 4) & ~M);
      O[i] = ((tl[i] >> 4) & M) | (th[i] & ~M);
    }
    const uint32_t ea = __builtin_amdgcn_perm(E[1], E[0], 0x05010400u);  // E0.b0 E1.b0 E0.b1 E1.b1
    const uint32_t eb = __builtin_amdgcn_perm(E[3], E[2], 0x05010400u);
    const uint32_t ec = __builtin_amdgcn_perm(E[1], E[0], 0x00000602u);  // E0.b2 E1.b2
    const uint32_t ed = __builtin_amdgcn_perm(E[3], E[2], 0x00000602u);
    const uint32_t oa = __builtin_amdgcn_perm(O[1], O[0], 0x05010400u);
    const uint32_t ob = __builtin_amdgcn_perm(O[3], O[2], 0x05010400u);
    uint32_t dw[5];
    dw[0] = __builtin_amdgcn_perm(eb, ea, 0x05040100u) ^ 0x88888888u;
    dw[1] = __builtin_amdgcn_perm(ob, oa, 0x05040100u) ^ 0x88888888u;
    dw[2] = __builtin_amdgcn_perm(eb, ea, 0x07060302u) ^ 0x88888888u;
    dw[3] = __builtin_amdgcn_perm(ob, oa, 0x07060302u) ^ 0x88888888u;
    dw[4] = __builtin_amdgcn_perm(ed, ec, 0x05040100u) ^ 0x88888888u;
    int bs = 0;
    if constexpr (BSUM) {
      // X_i = (low 20 bits of tl/th) - 0x88888; the block sum over its 4 items
#pragma unroll
      for (int i = 0; i < 4; i++) bs += (int)(tl[i] & 0xFFFFFu) + (int)(th[i] & 0xFFFFFu) - 2 * 0x88888;
      bs += __shfl_xor(bs, 1, CN_WAVE);
      bs += __shfl_xor(bs, 2, CN_WAVE);
    }
    if (on) {
      uint32_t* rec = xd + (b >> 1) * XD_UNIT_DW;
      const int blk = b & 1;
#pragma unroll
      for (int d = 0; d < 5; d++) rec[blk * 20 + d * 4 + k] = dw[d];
      if (k == 0) {
        rec[40 + blk] = (uint32_t)s;
        if constexpr (BSUM) rec[42 + blk] = (uint32_t)bs;
      }
    }
  }
  ss = cn_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
}

// ---------------------------------------------------------------------------
// Q6_K inputs as signed base-256 digits (v_dot4_i32_i8).
//
// Per 16-element group g (the span of one Q6_K scale):
//   s_g = 18 - e_g  with max|x_g| = f * 2^e_g, f in [0.5, 1)   (so |X| <= 2^18)
//   X_j = rint(x_j * 2^s_g) = sum_{d<3} D_{j,d} 256^d,  D in [-128, 127]
// The 6-bit weights q in [0, 63] are non-negative int8s, so
//   sum_j q_j X_j = Horner over d of dot4(q bytes, D_d bytes)
// is exact in int32 (|.| <= 16 * 63 * 2^18), and the group contributes
// sc_g * 2^-s_g * (that - 32 * sum_j X_j).
// LDS record of unit u (128 elements, half a super-block): XD6_UNIT_DW dwords,
// local group g at dword 16g: dwords 4d..4d+3 = digit plane d (byte b of dword
// k is the digit of element 128u + 16g + 4k + b), dword 12 = sum_j X_j,
// dword 13 = s_g.  The 132-dword unit stride puts the 16-byte reads of
// neighbouring lanes (different units, same group) on different banks.
// ---------------------------------------------------------------------------
constexpr int XD6_UNIT_DW = 132;

template <int MAXT, bool NORM>
struct XStage16 {
  float x[MAXT][16];
  float g[MAXT][16];
};
template <int MAXT>
struct XStage16<MAXT, false> {
  float x[MAXT][16];
};

// Group t of x (and of the RMSNorm weight) on thread t % BS, loads issued
// before the caller's weight loads (see stage_load).
template <int MAXT, bool NORM, int BS, bool MERGE = false, int NS = kFoldMaxSplits>
__device__ __forceinline__ void stage_load16(const float* __restrict__ x, const float* __restrict__ norm_w, int K,
                                             XStage16<MAXT, NORM>& st, const MergeSrc& ms = MergeSrc{}) {
  const int ngroups = K >> 4;
#pragma unroll
  for (int j = 0; j < MAXT; j++) {
    const int t = threadIdx.x + BS * j;
    const bool on = t < ngroups;
    const int tc = on ? t : ngroups - 1;  // loads issued unconditionally (see stage_load)
    MergeW<NS> mw{};
    int mh = 0, md = 0;
    if constexpr (MERGE) {  // the group's 16 elements lie in one head
      mh = (16 * tc) / ms.hd;
      md = 16 * tc - mh * ms.hd;
      mw = merge_weights<NS>(ms, mh);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float4 v, g = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (MERGE) v = merge_apply(ms, mw, mh, md + 4 * c);
      else v = *reinterpret_cast<const float4*>(x + 16 * tc + 4 * c);
      if constexpr (NORM) g = *reinterpret_cast<const float4*>(norm_w + 16 * tc + 4 * c);
      st.x[j][4 * c + 0] = v.x; st.x[j][4 * c + 1] = v.y; st.x[j][4 * c + 2] = v.z; st.x[j][4 * c + 3] = v.w;
      if constexpr (NORM) {
        st.g[j][4 * c + 0] = g.x; st.g[j][4 * c + 1] = g.y; st.g[j][4 * c + 2] = g.z; st.g[j][4 * c + 3] = g.w;
      }
    }
  }
}

// Writes the base-256 digit records of x * norm_w (x alone without NORM) and,
// as stage_digitize, leaves each wave's share of sum x^2 in red[wave].
// TR (Q3_K): record dword w, byte b holds element 4b + w of the group instead
// of element 4w + b, the order in which Q3_K's 2-bit fields come out of a qs
// dword (shift by 2w, mask 0x03030303).
template <int MAXT, bool NORM, int BS, bool TR = false>
__device__ __forceinline__ void stage_digitize16(const XStage16<MAXT, NORM>& st, int K, uint32_t* xd, float* red) {
  const int ngroups = K >> 4;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < MAXT; j++) {
    const int t = threadIdx.x + BS * j;
    float v[16];
    const bool on = t < ngroups;  // threads past the last group hold a re-read group
#pragma unroll
    for (int i = 0; i < 16; i++) {
      v[i] = st.x[j][i];
      ss += on ? v[i] * v[i] : 0.f;
    }
    if constexpr (NORM) {
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = v[i] * st.g[j][i];
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
    int e = 0;
    (void)frexpf(m, &e);
    const int sc = m > 0.f ? 18 - e : 0;
    // U = X + 0x808080 in [0x7C8080, 0x848080]: its bytes 0..2 are D_d + 128
    uint32_t U[16];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int X = (int)rintf(ldexpf(v[i], sc));
      sum += X;
      U[i] = (uint32_t)(X + 0x808080);
    }
    if (on) {
      uint32_t* rec = xd + (t >> 3) * XD6_UNIT_DW + 16 * (t & 7);
      uint32_t P[3][4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        // the four elements of record dword k, in byte order
        const uint32_t u0 = U[TR ? k : 4 * k], u1 = U[TR ? 4 + k : 4 * k + 1];
        const uint32_t u2 = U[TR ? 8 + k : 4 * k + 2], u3 = U[TR ? 12 + k : 4 * k + 3];
        const uint32_t a01 = __builtin_amdgcn_perm(u1, u0, 0x05010400u);  // U0.b0 U1.b0 U0.b1 U1.b1
        const uint32_t a23 = __builtin_amdgcn_perm(u3, u2, 0x05010400u);
        const uint32_t c01 = __builtin_amdgcn_perm(u1, u0, 0x00000602u);  // U0.b2 U1.b2
        const uint32_t c23 = __builtin_amdgcn_perm(u3, u2, 0x00000602u);
        P[0][k] = __builtin_amdgcn_perm(a23, a01, 0x05040100u) ^ 0x80808080u;
        P[1][k] = __builtin_amdgcn_perm(a23, a01, 0x07060302u) ^ 0x80808080u;
        P[2][k] = __builtin_amdgcn_perm(c23, c01, 0x05040100u) ^ 0x80808080u;
      }
#pragma unroll
      for (int d = 0; d < 3; d++)
        *reinterpret_cast<uint4*>(rec + 4 * d) = make_uint4(P[d][0], P[d][1], P[d][2], P[d][3]);
      rec[12] = (uint32_t)sum;
      rec[13] = (uint32_t)sc;
    }
  }
  ss = cn_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
}

// ---------------------------------------------------------------------------
// Unit loads
// ---------------------------------------------------------------------------
template <int QT>
__device__ __forceinline__ void load_unit(const cn_gbyte* row, int u, uint32_t* w);

template <>
__device__ __forceinline__ void load_unit<QT_Q4_0>(const cn_gbyte* row, int u, uint32_t* w) {
  const CN_GLOBAL uint32_t* p = (const CN_GLOBAL uint32_t*)(row + (size_t)u * 36);
#pragma unroll
  for (int k = 0; k < 9; k++) w[k] = p[k];
}

__device__ __forceinline__ void load_u32x4(const cn_gbyte* p, uint32_t* w) {
  const cn_u32x4 t = *(const CN_GLOBAL cn_u32x4*)p;
  w[0] = t.x;
  w[1] = t.y;
  w[2] = t.z;
  w[3] = t.w;
}

// Half h = u & 1 of Q4_K super-block u >> 1 (144 bytes, 16-byte aligned):
// w[0..3] = d, dmin and the 12 scale bytes, w[4..19] = qs[64h .. 64h+63].
template <>
__device__ __forceinline__ void load_unit<QT_Q4_K>(const cn_gbyte* row, int u, uint32_t* w) {
  const cn_gbyte* sb = row + (size_t)(u >> 1) * 144;
  const int h = u & 1;
  load_u32x4(sb, w);
#pragma unroll
  for (int k = 0; k < 4; k++) load_u32x4(sb + 16 + 64 * h + 16 * k, w + 4 + 4 * k);
}

// Two Q8_0 blocks, 68 bytes: rows hold whole pairs (K % 64 == 0), so a unit
// starts on a 4-byte boundary.
template <>
__device__ __forceinline__ void load_unit<QT_Q8_0>(const cn_gbyte* row, int u, uint32_t* w) {
  const CN_GLOBAL uint32_t* p = (const CN_GLOBAL uint32_t*)(row + (size_t)u * 68);
#pragma unroll
  for (int k = 0; k < 17; k++) w[k] = p[k];
}

// Half h = u & 1 of Q5_K super-block u >> 1 (176 bytes, 16-byte aligned):
// w[0..3] = d, dmin and the scales, w[4..7] = qh[16h .. 16h+15] (the fifth
// bits of elements 128h ..), w[8..23] = qs[64h .. 64h+63].
template <>
__device__ __forceinline__ void load_unit<QT_Q5_K>(const cn_gbyte* row, int u, uint32_t* w) {
  const cn_gbyte* sb = row + (size_t)(u >> 1) * 176;
  const int h = u & 1;
  load_u32x4(sb, w);
  load_u32x4(sb + 16 + 16 * h, w + 4);
#pragma unroll
  for (int k = 0; k < 4; k++) load_u32x4(sb + 48 + 64 * h + 16 * k, w + 8 + 4 * k);
}

// Half h = u & 1 of Q6_K super-block u >> 1 (210 bytes, so super-blocks start
// on 2-byte boundaries): w[0..15] = ql[64h .. 64h+63], w[16..23] = qh[32h ..
// 32h+31], w[24..25] = scales[8h .. 8h+7], w[26] = d (low half).  Each piece
// is read as the dword-aligned window that covers it (one dword more than the
// piece) and realigned by sh = 0 or 2 bytes, the same for every piece of the
// super-block, so the loads do not diverge.  The windows of ql and qh end
// inside the next piece; the scales' window needs its third dword only when
// sh = 2 (it then ends at byte 209), and d is a 16-bit load, so nothing past
// the super-block is read.
template <>
__device__ __forceinline__ void load_unit<QT_Q6_K>(const cn_gbyte* row, int u, uint32_t* w) {
  const cn_gbyte* sb = row + (size_t)(u >> 1) * 210;
  const int h = u & 1;
  const uintptr_t base = reinterpret_cast<uintptr_t>(sb);
  const uint32_t sh = (uint32_t)(base & 3);  // 0 or 2
  const CN_GLOBAL uint32_t* q = (const CN_GLOBAL uint32_t*)(base & ~(uintptr_t)3);
  uint32_t r[17], t[9], c[3];
#pragma unroll
  for (int k = 0; k < 17; k++) r[k] = q[16 * h + k];
#pragma unroll
  for (int k = 0; k < 9; k++) t[k] = q[32 + 8 * h + k];
  c[0] = q[48 + 2 * h];
  c[1] = q[49 + 2 * h];
  c[2] = sh ? q[50 + 2 * h] : 0u;
#pragma unroll
  for (int k = 0; k < 16; k++) w[k] = __builtin_amdgcn_alignbyte(r[k + 1], r[k], sh);
#pragma unroll
  for (int k = 0; k < 8; k++) w[16 + k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], sh);
  w[24] = __builtin_amdgcn_alignbyte(c[1], c[0], sh);
  w[25] = __builtin_amdgcn_alignbyte(c[2], c[1], sh);
  w[26] = *(const CN_GLOBAL uint16_t*)(sb + 208);
}

// Quarter q = u & 1 of half h = (u >> 1) & 1 of Q6_K super-block u >> 2: the
// 64 elements 128h + l + 32i (l in [16q, 16q + 16), i < 4).  w[0..3] =
// ql[64h + 16q .. +15] (low nibbles: i = 0, high: i = 2), w[4..7] =
// ql[64h + 32 + 16q .. +15] (i = 1, 3), w[8..11] = qh[32h + 16q .. +15] (bits
// 2i), w[12..13] = the half's 8 scale bytes (group q + 2i), w[14] = d.  Each
// piece is read as its dword-aligned window and realigned as load_unit<Q6_K>
// does; every window lies inside the super-block or the bytes before it.
template <>
__device__ __forceinline__ void load_unit<QT_Q6_KQ>(const cn_gbyte* row, int u, uint32_t* w) {
  const cn_gbyte* sb = row + (size_t)(u >> 2) * 210;
  const int h = (u >> 1) & 1, q = u & 1;
  const uintptr_t base = reinterpret_cast<uintptr_t>(sb);
  const uint32_t sh = (uint32_t)(base & 3);  // 0 or 2
  const CN_GLOBAL uint32_t* p = (const CN_GLOBAL uint32_t*)(base & ~(uintptr_t)3);
  uint32_t a[5], b[5], c[5], e[3];
#pragma unroll
  for (int k = 0; k < 5; k++) {
    a[k] = p[16 * h + 4 * q + k];
    b[k] = p[16 * h + 8 + 4 * q + k];
    c[k] = p[32 + 8 * h + 4 * q + k];
  }
  e[0] = p[48 + 2 * h];
  e[1] = p[49 + 2 * h];
  e[2] = sh ? p[50 + 2 * h] : 0u;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    w[k] = __builtin_amdgcn_alignbyte(a[k + 1], a[k], sh);
    w[4 + k] = __builtin_amdgcn_alignbyte(b[k + 1], b[k], sh);
    w[8 + k] = __builtin_amdgcn_alignbyte(c[k + 1], c[k], sh);
  }
  w[12] = __builtin_amdgcn_alignbyte(e[1], e[0], sh);
  w[13] = __builtin_amdgcn_alignbyte(e[2], e[1], sh);
  w[14] = *(const CN_GLOBAL uint16_t*)(sb + 208);
}

// Q3_K half super-block h = u & 1 (DequantQ3K.cs: hmask[32] @0, qs[64] @32,
// scales[12] @96, fp16 d @108; 110 bytes, so super-blocks start on 2-byte
// boundaries): w[0..7] = qs[32h .. 32h+31], w[8..11] = hmask[16h .. 16h+15],
// w[12..14] = the 12 scale bytes, w[15] = d (low half).  As for Q6_K, each
// piece is read as the dword-aligned window that covers it and realigned by
// sh = 0 or 2 bytes; the qs and hmask windows end inside the super-block (at
// byte 99 at most), the scales' window takes its fourth dword only when sh = 2
// (it then ends at byte 109), and d is a 16-bit load, so nothing past the
// super-block is read.
template <>
__device__ __forceinline__ void load_unit<QT_Q3_K>(const cn_gbyte* row, int u, uint32_t* w) {
  const cn_gbyte* sb = row + (size_t)(u >> 1) * 110;
  const int h = u & 1;
  const uintptr_t base = reinterpret_cast<uintptr_t>(sb);
  const uint32_t sh = (uint32_t)(base & 3);  // 0 or 2
  const CN_GLOBAL uint32_t* q = (const CN_GLOBAL uint32_t*)(base & ~(uintptr_t)3);
  uint32_t r[9], t[5], c[4];
#pragma unroll
  for (int k = 0; k < 9; k++) r[k] = q[8 + 8 * h + k];
#pragma unroll
  for (int k = 0; k < 5; k++) t[k] = q[4 * h + k];
#pragma unroll
  for (int k = 0; k < 3; k++) c[k] = q[24 + k];
  c[3] = sh ? q[27] : 0u;
#pragma unroll
  for (int k = 0; k < 8; k++) w[k] = __builtin_amdgcn_alignbyte(r[k + 1], r[k], sh);
#pragma unroll
  for (int k = 0; k < 4; k++) w[8 + k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], sh);
#pragma unroll
  for (int k = 0; k < 3; k++) w[12 + k] = __builtin_amdgcn_alignbyte(c[k + 1], c[k], sh);
  w[15] = *(const CN_GLOBAL uint16_t*)(sb + 108);
}

// ---------------------------------------------------------------------------
// Unit dot products for RPW rows sharing the same x slice.
// xs: LDS (padded) already offset to the unit's first element; sx: block sums.
// ---------------------------------------------------------------------------

// Q4_0 unit against the digit record xd (see stage_digitize): block A's qs
// (pair bytes 2..17) is realigned with alignbyte, block B's (bytes 20..35)
// is dword aligned.
template <int RPW>
__device__ __forceinline__ void dot_q4_0_digits(const uint32_t (*w)[9], const uint32_t (&X)[40], int sA, int sB,
                                                float* acc) {
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    uint32_t qa[4], qb[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      qa[k] = __builtin_amdgcn_alignbyte(w[i][k + 1], w[i][k], 2) ^ 0x88888888u;
      qb[k] = w[i][5 + k] ^ 0x88888888u;
    }
    int ta = 0, tb = 0;
#pragma unroll
    for (int d = 4; d >= 0; d--) {
      if (d < 4) {
        ta <<= 4;
        tb <<= 4;
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        ta = __builtin_amdgcn_sdot8((int)qa[k], (int)X[d * 4 + k], ta, false);
        tb = __builtin_amdgcn_sdot8((int)qb[k], (int)X[20 + d * 4 + k], tb, false);
      }
    }
    const float da = ldexpf(cn_h2f(w[i][0]), -sA);
    const float db = ldexpf(cn_h2f(w[i][4] >> 16), -sB);
    acc[i] += (float)ta * da + (float)tb * db;
  }
}

template <int RPW>
__device__ __forceinline__ void dot_unit_q4_0_dig(const uint32_t (*w)[9], const uint32_t* xd, float* acc) {
  uint32_t X[40];
#pragma unroll
  for (int c = 0; c < 10; c++) {
    const uint4 t = *reinterpret_cast<const uint4*>(xd + 4 * c);
    X[4 * c + 0] = t.x; X[4 * c + 1] = t.y; X[4 * c + 2] = t.z; X[4 * c + 3] = t.w;
  }
  const uint2 se = *reinterpret_cast<const uint2*>(xd + 40);
  dot_q4_0_digits<RPW>(w, X, (int)se.x, (int)se.y, acc);
}

// d*sc and dmin*m of sub-blocks 4h .. 4h+3 of a Q4_K / Q5_K super-block from
// its header dwords (get_scale_min_k4, DequantQ4K.cs:218-241): sub-blocks 0..3
// take the low six bits of scale bytes 0..3 / 4..7, sub-blocks 4..7 a nibble
// of bytes 8..11 with the top two bits of bytes 0..3 / 4..7 above it.
__device__ __forceinline__ void k4_scales_half(const uint32_t* hdr, int h, float (&dsc)[4], float (&dmm)[4]) {
  const float d = cn_h2f(hdr[0]), dmin = cn_h2f(hdr[0] >> 16);
  const uint32_t q0 = hdr[1], q1 = hdr[2], q2 = hdr[3];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t b8 = (q2 >> (8 * j)) & 0xFF;
    const int sc_lo = (q0 >> (8 * j)) & 63, m_lo = (q1 >> (8 * j)) & 63;
    const int sc_hi = (b8 & 0xF) | (((q0 >> (8 * j + 6)) & 3) << 4);
    const int m_hi = (b8 >> 4) | (((q1 >> (8 * j + 6)) & 3) << 4);
    dsc[j] = d * (float)(h ? sc_hi : sc_lo);
    dmm[j] = dmin * (float)(h ? m_hi : m_lo);
  }
}

// Half h of a Q4_K super-block (reference order, DequantQ4K.cs:59-72) against
// the digit records of its 4 blocks (2 records).  Local sub-block s's qs dwords
// XOR 0x88888888 are (q - 8) as signed nibbles in the digit records' nibble
// order, so with T_s = sum_j (q_j - 8) X_j from the Horner sum of sdot8 over
// the 5 digits,
//   sum_j q_j X_j = T_s + 8 SX_s   (SX_s = sum_j X_j, exact in int32),
// and the sub-block contributes 2^-e_s (d sc_s (T_s + 8 SX_s) - dmin m_s SX_s):
// d sc q - dmin m per weight against x rounded to its digits, as the Q4_0
// digit dot.
template <int RPW>
__device__ __forceinline__ void dot_unit_q4_k_dig(const uint32_t (*w)[20], const uint32_t* xd, int h, float* acc) {
  float dsc[RPW][4], dmm[RPW][4];
#pragma unroll
  for (int i = 0; i < RPW; i++) k4_scales_half(w[i], h, dsc[i], dmm[i]);
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const uint32_t* rec = xd + (s >> 1) * XD_UNIT_DW;
    const int blk = s & 1;
    uint32_t X[20];
#pragma unroll
    for (int c = 0; c < 5; c++) {
      const uint4 t = *reinterpret_cast<const uint4*>(rec + blk * 20 + 4 * c);
      X[4 * c + 0] = t.x; X[4 * c + 1] = t.y; X[4 * c + 2] = t.z; X[4 * c + 3] = t.w;
    }
    const int e = (int)rec[40 + blk];
    const int sx = (int)rec[42 + blk];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      int t = 0;
#pragma unroll
      for (int dg = 4; dg >= 0; dg--) {
        if (dg < 4) t <<= 4;
#pragma unroll
        for (int k = 0; k < 4; k++)
          t = __builtin_amdgcn_sdot8((int)(w[i][4 + 4 * s + k] ^ 0x88888888u), (int)X[dg * 4 + k], t, false);
      }
      acc[i] += ldexpf(dsc[i][s] * (float)(t + 8 * sx) - dmm[i][s] * (float)sx, -e);
    }
  }
}

// Q6_K super-block (DequantQ6K.cs:53-83): for half h and l < 32,
//   q1 = ql[64h+l]&15 | (qh[32h+l]&3)<<4          -> element 128h+l,    scale sc[8h+l/16]
//   q2 = ql[64h+l+32]&15 | ((qh>>2)&3)<<4         -> element 128h+32+l, scale sc[8h+l/16+2]
//   q3 = ql[64h+l]>>4 | ((qh>>4)&3)<<4            -> element 128h+64+l, scale sc[8h+l/16+4]
//   q4 = ql[64h+l+32]>>4 | ((qh>>6)&3)<<4         -> element 128h+96+l, scale sc[8h+l/16+6]
// value = d*sc*(q-32): the 16 elements of group g = 8h + 2*qi + lb are l in
// [16lb, 16lb+16) of q_{qi+1}; their q bytes, assembled four at a time in
// element order, meet the digit planes of stage_digitize16 on v_dot4_i32_i8.
template <int RPW>
__device__ __forceinline__ void dot_unit_q6_k_dig(const uint32_t (*w)[27], const uint32_t* xd, float* acc) {
  float part[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) part[i] = 0.f;
#pragma unroll
  for (int qi = 0; qi < 4; qi++) {
#pragma unroll
    for (int lb = 0; lb < 2; lb++) {
      const int g = 2 * qi + lb;  // local group: scale 8h + g of the super-block
      const uint32_t* rec = xd + 16 * g;
      uint32_t D[3][4];
#pragma unroll
      for (int d = 0; d < 3; d++) {
        const uint4 t = *reinterpret_cast<const uint4*>(rec + 4 * d);
        D[d][0] = t.x; D[d][1] = t.y; D[d][2] = t.z; D[d][3] = t.w;
      }
      const int xsum = (int)rec[12];
      const int e = (int)rec[13];
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int l = 16 * lb + 4 * k;
          const uint32_t qlw = w[i][(l + ((qi & 1) ? 32 : 0)) >> 2];
          const uint32_t qhw = w[i][16 + (l >> 2)];
          const uint32_t nib = (qi < 2) ? (qlw & 0x0F0F0F0Fu) : ((qlw >> 4) & 0x0F0F0F0Fu);
          q[k] = nib | (((qhw >> (2 * qi)) & 0x03030303u) << 4);
        }
        int t = 0;
#pragma unroll
        for (int d = 2; d >= 0; d--) {
          if (d < 2) t <<= 8;
#pragma unroll
          for (int k = 0; k < 4; k++) t = __builtin_amdgcn_sdot4((int)q[k], (int)D[d][k], t, false);
        }
        const int8_t scv = (int8_t)((w[i][24 + (g >> 2)] >> (8 * (g & 3))) & 0xFF);
        part[i] += ldexpf((float)(t - 32 * xsum) * (float)scv, -e);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) acc[i] += cn_h2f(w[i][26]) * part[i];
}

// Q6_K quarter q of a half super-block (load_unit<QT_Q6_KQ>) against the
// half's digit records (groups q, q + 2, q + 4, q + 6): dot_unit_q6_k_dig's
// arithmetic for those four groups.
template <int RPW>
__device__ __forceinline__ void dot_unit_q6_kq_dig(const uint32_t (*w)[15], const uint32_t* xd, int q, float* acc) {
  float part[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) part[i] = 0.f;
#pragma unroll
  for (int qi = 0; qi < 4; qi++) {
    const int g = 2 * qi + q;  // local group: scale 8h + g of the super-block
    const uint32_t* rec = xd + 16 * g;
    uint32_t D[3][4];
#pragma unroll
    for (int d = 0; d < 3; d++) {
      const uint4 t = *reinterpret_cast<const uint4*>(rec + 4 * d);
      D[d][0] = t.x; D[d][1] = t.y; D[d][2] = t.z; D[d][3] = t.w;
    }
    const int xsum = (int)rec[12];
    const int e = (int)rec[13];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      uint32_t qv[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t qlw = (qi & 1) ? w[i][4 + k] : w[i][k];
        const uint32_t nib = (qi < 2) ? (qlw & 0x0F0F0F0Fu) : ((qlw >> 4) & 0x0F0F0F0Fu);
        qv[k] = nib | (((w[i][8 + k] >> (2 * qi)) & 0x03030303u) << 4);
      }
      int t = 0;
#pragma unroll
      for (int d = 2; d >= 0; d--) {
        if (d < 2) t <<= 8;
#pragma unroll
        for (int k = 0; k < 4; k++) t = __builtin_amdgcn_sdot4((int)qv[k], (int)D[d][k], t, false);
      }
      const int8_t scv = (int8_t)((w[i][12 + (g >> 2)] >> (8 * (g & 3))) & 0xFF);
      part[i] += ldexpf((float)(t - 32 * xsum) * (float)scv, -e);
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) acc[i] += cn_h2f(w[i][14]) * part[i];
}

// Q3_K half super-block h (DequantQ3K.cs:35-70, DecodeScales :122-150): element
// l of the half is q3 = (qs byte l/4 >> 2(l%4)) & 3 | (hmask bit l) << 2,
// value d*sc*(q3 - 4) with sc the 6-bit scale of group 8h + l/16 (low nibble
// of byte i or high nibble of byte i-8, two bits of byte 8 + i%4 above it,
// minus 32).  Group g's qs are dword g; shifted by 2w and masked they give the
// 2-bit fields of elements 4b + w in bytes b, which meet the transposed digit
// records (stage_digitize16 with TR).  Its 16 hmask bits are spread one nibble
// per byte (bit 4b + w -> bit 8b + w) and bit w of each byte moved to bit 2.
template <int RPW>
__device__ __forceinline__ void dot_unit_q3_k_dig(const uint32_t (*w)[16], const uint32_t* xd, int h, float* acc) {
  float part[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) part[i] = 0.f;
#pragma unroll
  for (int g = 0; g < 8; g++) {
    const uint32_t* rec = xd + 16 * g;
    uint32_t D[3][4];
#pragma unroll
    for (int d = 0; d < 3; d++) {
      const uint4 t = *reinterpret_cast<const uint4*>(rec + 4 * d);
      D[d][0] = t.x; D[d][1] = t.y; D[d][2] = t.z; D[d][3] = t.w;
    }
    const int xsum = (int)rec[12];
    const int e = (int)rec[13];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const uint32_t qw = w[i][g];
      uint32_t hs = (w[i][8 + (g >> 1)] >> (16 * (g & 1))) & 0xFFFFu;
      hs = (hs | (hs << 8)) & 0x00FF00FFu;
      hs = (hs | (hs << 4)) & 0x0F0F0F0Fu;
      uint32_t q[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t hb = k < 3 ? (hs << (2 - k)) : (hs >> 1);
        q[k] = ((qw >> (2 * k)) & 0x03030303u) | (hb & 0x04040404u);
      }
      int t = 0;
#pragma unroll
      for (int d = 2; d >= 0; d--) {
        if (d < 2) t <<= 8;
#pragma unroll
        for (int k = 0; k < 4; k++) t = __builtin_amdgcn_sdot4((int)q[k], (int)D[d][k], t, false);
      }
      const uint32_t lob = (w[i][12 + (g >> 2)] >> (8 * (g & 3))) >> (4 * h);
      const uint32_t hib = w[i][14] >> (8 * (g & 3) + 4 * h + 2 * (g >> 2));
      const int scv = (int)((lob & 15u) | ((hib & 3u) << 4)) - 32;
      part[i] += ldexpf((float)(t - 4 * xsum) * (float)scv, -e);
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) acc[i] += cn_h2f(w[i][15]) * part[i];
}

// Q8_0 pair of blocks (DequantQ8_0.cs:51-90) against the base-256 digit
// records of its four 16-element groups: block A is unit bytes 0..33 (d, then
// 32 int8; its qs realigned with alignbyte), block B bytes 34..67 (d in the
// high half of dword 8, qs in dwords 9..16).  The int8 weights meet the x
// digits directly on v_dot4_i32_i8: t_g = sum_j q_j X_j is exact
// (|.| <= 16 * 128 * 2^18) and the group contributes d * 2^-e_g * t_g.
template <int RPW>
__device__ __forceinline__ void dot_unit_q8_0_dig8(const uint32_t (*w)[17], const uint32_t* xd, float* acc) {
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int b = g >> 1;
    const uint32_t* rec = xd + 16 * g;
    uint32_t D[3][4];
#pragma unroll
    for (int d = 0; d < 3; d++) {
      const uint4 t = *reinterpret_cast<const uint4*>(rec + 4 * d);
      D[d][0] = t.x; D[d][1] = t.y; D[d][2] = t.z; D[d][3] = t.w;
    }
    const int e = (int)rec[13];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      int t = 0;
#pragma unroll
      for (int dg = 2; dg >= 0; dg--) {
        if (dg < 2) t <<= 8;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int kk = 4 * (g & 1) + k;  // qs dword of the block
          const uint32_t q = b == 0 ? __builtin_amdgcn_alignbyte(w[i][kk + 1], w[i][kk], 2) : w[i][9 + kk];
          t = __builtin_amdgcn_sdot4((int)q, (int)D[dg][k], t, false);
        }
      }
      const float d = b == 0 ? cn_h2f(w[i][0]) : cn_h2f(w[i][8] >> 16);
      acc[i] += d * ldexpf((float)t, -e);
    }
  }
}

// Q4_K / Q5_K super-block against the base-256 digit record of
// stage_digitize16.  Scales and nibble order of Q4_K (DequantQ4K.cs:59-72):
// sub-block s uses qs[16s..16s+15], low nibbles -> elements 32s+0..15, high ->
// 32s+16..31, so digit group g = 2s + hh takes the low (hh = 0) or high nibbles
// of those 16 bytes, four elements per qs dword in element order.  Q5_K
// (DequantQ5K.cs:37-88) adds qh[32] at byte 16 whose bit e%8 of byte e/8 is bit
// 4 of element e: bits 16hh + 4k .. +3 of dword 4+s for the four elements of
// qs dword k, spread into byte lanes (t * 0x00204081 puts bit b of t at bit
// 8b) above the nibbles.  With t_g = sum_j q_j X_j (exact, |.| <= 16*31*2^18)
// the group contributes 2^-e_g (d sc_s t_g - dmin m_s SX_g).
template <int QT, int RPW>
__device__ __forceinline__ void dot_unit_k45_dig8(const uint32_t (*w)[QTraits<QT>::NDW], const uint32_t* xd, int h,
                                                  float* acc) {
  constexpr int QS = QT == QT_Q5_K ? 8 : 4;  // first qs dword of the half
  float dsc[RPW][4], dmm[RPW][4];
#pragma unroll
  for (int i = 0; i < RPW; i++) k4_scales_half(w[i], h, dsc[i], dmm[i]);
#pragma unroll
  for (int g = 0; g < 8; g++) {
    const int sb = g >> 1, hh = g & 1;  // local sub-block, low / high nibbles
    const uint32_t* rec = xd + 16 * g;
    uint32_t D[3][4];
#pragma unroll
    for (int d = 0; d < 3; d++) {
      const uint4 t = *reinterpret_cast<const uint4*>(rec + 4 * d);
      D[d][0] = t.x; D[d][1] = t.y; D[d][2] = t.z; D[d][3] = t.w;
    }
    const int xsum = (int)rec[12];
    const int e = (int)rec[13];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      uint32_t q[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t dw = w[i][QS + 4 * sb + k];
        uint32_t v = hh ? ((dw >> 4) & 0x0F0F0F0Fu) : (dw & 0x0F0F0F0Fu);
        if constexpr (QT == QT_Q5_K) {
          const uint32_t t4 = (w[i][4 + sb] >> (16 * hh + 4 * k)) & 0xFu;
          v |= ((t4 * 0x00204081u) & 0x01010101u) << 4;
        }
        q[k] = v;
      }
      int t = 0;
#pragma unroll
      for (int d = 2; d >= 0; d--) {
        if (d < 2) t <<= 8;
#pragma unroll
        for (int k = 0; k < 4; k++) t = __builtin_amdgcn_sdot4((int)q[k], (int)D[d][k], t, false);
      }
      acc[i] += ldexpf(dsc[i][sb] * (float)t - dmm[i][sb] * (float)xsum, -e);
    }
  }
}

// Issues the loads of one wave iteration: RPW rows x NU units per lane.
// Every load is issued (a row past n_vrows re-reads the last row, a unit past
// the row's end the last unit) so the loads are straight-line code: the
// caller discards those rows (the epilogue skips them) and units (the dot
// skips them), and the compiler can count exactly how many loads follow the
// staged x (a load on a conditional path makes it wait for all of them).
template <int QT, int RPW, int LPR, int NU, int EPI>
__device__ __forceinline__ void issue_loads(const GemvArgs& a, int it, int sub, int li, int nunits, size_t bpr,
                                            uint32_t (&w)[RPW][NU][QTraits<QT>::NDW]) {
  constexpr int RW = RPW * (CN_WAVE / LPR);
  const int vr0 = it * RW + sub * RPW;
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const int vr = vr0 + i < a.n_vrows ? vr0 + i : a.n_vrows - 1;
    int seg, r;
    map_row<EPI>(a, vr, seg, r);
    const cn_gbyte* rp = seg_w(a, seg) + (size_t)r * bpr;
#pragma unroll
    for (int n = 0; n < NU; n++) {
      const int u = li + LPR * n;
      load_unit<QT>(rp, u < nunits ? u : nunits - 1, w[i][n]);
    }
  }
}

// One launch streams n_vrows rows.  A wave iteration covers RW = RPW*(64/LPR)
// rows; every lane holds RPW rows x NU units in registers.  The first
// iteration's loads are issued before x is staged, so HBM latency overlaps the
// prologue, and each next iteration's loads are issued before the current
// reduction and epilogue.  BS threads per workgroup (Q4_0: 256, 512 or 1024;
// K-quants 256): the launch picks BS so that one workgroup per CU holds every
// row of the launch in flight where the register budget allows.
template <int QT, int RPW, int LPR, int NU, int EPI, int BS>
__global__ __launch_bounds__(BS) void gemv_kernel(GemvArgs a) {
  using T = QTraits<QT>;
  static_assert(QT == QT_Q4_0 || BS == CN_BLOCK, "K-quant GEMVs run 256-thread workgroups");
  constexpr int NWV = BS / CN_WAVE;
  constexpr int UNIT = T::UNIT;
  constexpr int RW = RPW * (CN_WAVE / LPR);
  extern __shared__ float smem[];
  const int K = a.K;
  const int nunits = K / UNIT;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, li = lane % LPR;
  const int n_iters = (a.n_vrows + RW - 1) / RW;
  const size_t bpr = (size_t)(K / T::BLOCK) * T::BLOCK_BYTES;
  const int wstride = gridDim.x * NWV;
  int it = blockIdx.x * NWV + wave;

  uint32_t w[RPW][NU][T::NDW];
  constexpr int NR = res_count<EPI, RPW>();
  float res[NR];
  // The stop flag and the position are read as vector loads issued ahead of
  // x and consumed late (after staging, in the epilogue), so no scalar wait
  // for them stalls the loads at the start.
  constexpr bool MERGE = is_merge(EPI);
  constexpr int NS = merge_slots(EPI);
  const int stop_v = cn_load_late(stop_flag(a));
  const int pos_v = (EPI == GEMV_EPI_QKV || MERGE) ? cn_load_late(a.pos) : 0;
  constexpr bool kDig8 =
      QT == QT_Q8_0 || QT == QT_Q3_K || QT == QT_Q6_K || QT == QT_Q6_KQ || QT == QT_Q5_K || (QT == QT_Q4_K && LPR > 32);
  MergeSrc ms{};
  if constexpr (MERGE) {
    ms.o = a.part_o;
    ms.ml = a.part_ml;
    ms.hd = a.head_dim;
    ms.splits = a.msplits;
    // the base-256 staging merges while it loads: it needs the position now
    if constexpr (kDig8)
      ms.s_eff = min(a.msplits, (__builtin_amdgcn_readfirstlane(pos_v) + a.mchunk) / a.mchunk);
  }

  // ---- prologue: stage x (optionally RMS-normalised) into LDS ----
  // Integer digit paths: base-16 digits on v_dot8_i32_i4 for Q4_0 and for Q4_K
  // up to K = 4096 (the register budget of the staged x at 16 items per
  // half-super-block lane); base-256 digits on v_dot4_i32_i8 for Q8_0, Q6_K,
  // Q5_K and the longer Q4_K rows.
  {
    constexpr bool NORM = EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_SWIGLU || EPI == GEMV_EPI_LOGITS;
    uint32_t* xd = reinterpret_cast<uint32_t*>(smem);
    float* xred;
    if constexpr (kDig8) {
      // groups per thread: K <= UNIT * LPR * NU, so K/16 <= (UNIT/16) * LPR * NU groups over BS threads
      constexpr int MAXT = ((UNIT / 16) * LPR * NU + BS - 1) / BS;
      XStage16<MAXT, NORM> st;
      stage_load16<MAXT, NORM, BS, MERGE, NS>(a.x, a.norm_w, K, st, ms);
      // Two units per lane: the staged x would sit beside twice the weight
      // registers (2 waves per SIMD), so it is digitized before the weight
      // loads are issued.
      constexpr bool kLate = NU >= 2;
      if constexpr (!kLate) {
        issue_loads<QT, RPW, LPR, NU, EPI>(a, it, sub, li, nunits, bpr, w);
        load_residual<EPI, RPW, NR>(a, it * RW + sub * RPW, li, 0, res);
      }
      xred = reinterpret_cast<float*>(smem) + (size_t)((K + 127) >> 7) * XD6_UNIT_DW;
      stage_digitize16<MAXT, NORM, BS, QT == QT_Q3_K>(st, K, xd, xred);
      if constexpr (kLate) {
        issue_loads<QT, RPW, LPR, NU, EPI>(a, it, sub, li, nunits, bpr, w);
        load_residual<EPI, RPW, NR>(a, it * RW + sub * RPW, li, 0, res);
      }
    } else {
      // items per thread: K <= UNIT * LPR * NU, so K/8 <= (UNIT/8) * LPR * NU items over BS threads
      constexpr int MAXT = ((UNIT / 8) * LPR * NU + BS - 1) / BS;
      XStage<MAXT, NORM> st;
      stage_load<MAXT, NORM, BS, MERGE>(a.x, a.norm_w, K, st, ms);
      XMerge<MERGE ? MAXT : 1, MERGE ? NS : 1> mr;
      if constexpr (MERGE) stage_merge_load<MAXT, BS, NS>(ms, K, mr);
      // rows past n_vrows are loaded (re-reading the last row) and skipped
      issue_loads<QT, RPW, LPR, NU, EPI>(a, it, sub, li, nunits, bpr, w);
      load_residual<EPI, RPW, NR>(a, it * RW + sub * RPW, li, 0, res);
      if constexpr (MERGE) {
        // chunks below pos + 1 (the position arrives with the partials)
        ms.s_eff = min(a.msplits, (__builtin_amdgcn_readfirstlane(pos_v) + a.mchunk) / a.mchunk);
        stage_merge<MAXT, NORM, NS>(ms, mr, st);
      }
      xred = reinterpret_cast<float*>(smem) + (size_t)(K >> 6) * XD_UNIT_DW;
      stage_digitize<MAXT, NORM, BS, QT == QT_Q4_K>(st, K, xd, xred);
    }
    __syncthreads();
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NWV; v++) ss += xred[v];
    const float rms = NORM ? 1.0f / sqrtf(ss / (float)K + a.eps) : 1.0f;
    if (__builtin_amdgcn_readfirstlane(stop_v)) return;
    const int pos = __builtin_amdgcn_readfirstlane(pos_v);
    while (it < n_iters) {
      load_rope<EPI, RPW, NR>(a, it * RW + sub * RPW, pos, res);
      float acc[RPW];
#pragma unroll
      for (int i = 0; i < RPW; i++) acc[i] = 0.f;
#pragma unroll
      for (int n = 0; n < NU; n++) {
        const int u = li + LPR * n;
        if (u < nunits) {
          uint32_t wu[RPW][T::NDW];
#pragma unroll
          for (int i = 0; i < RPW; i++)
#pragma unroll
            for (int k = 0; k < T::NDW; k++) wu[i][k] = w[i][n][k];
          if constexpr (QT == QT_Q4_0) dot_unit_q4_0_dig<RPW>(wu, xd + u * XD_UNIT_DW, acc);
          else if constexpr (QT == QT_Q8_0) dot_unit_q8_0_dig8<RPW>(wu, xd + (u >> 1) * XD6_UNIT_DW + 64 * (u & 1), acc);
          else if constexpr (QT == QT_Q6_K) dot_unit_q6_k_dig<RPW>(wu, xd + u * XD6_UNIT_DW, acc);
          else if constexpr (QT == QT_Q6_KQ) dot_unit_q6_kq_dig<RPW>(wu, xd + (u >> 1) * XD6_UNIT_DW, u & 1, acc);
          else if constexpr (QT == QT_Q3_K) dot_unit_q3_k_dig<RPW>(wu, xd + u * XD6_UNIT_DW, u & 1, acc);
          else if constexpr (kDig8) dot_unit_k45_dig8<QT, RPW>(wu, xd + u * XD6_UNIT_DW, u & 1, acc);
          else dot_unit_q4_k_dig<RPW>(wu, xd + 2 * u * XD_UNIT_DW, u & 1, acc);
        }
      }
      const int cur = it;
      float res_cur[NR];
#pragma unroll
      for (int i = 0; i < NR; i++) res_cur[i] = res[i];
      it += wstride;
      if (it < n_iters) {
        issue_loads<QT, RPW, LPR, NU, EPI>(a, it, sub, li, nunits, bpr, w);
        load_residual<EPI, RPW, NR>(a, it * RW + sub * RPW, li, 0, res);
      }
#pragma unroll
      for (int i = 0; i < RPW; i++) {
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) acc[i] += __shfl_xor(acc[i], off, CN_WAVE);
        acc[i] *= rms;
      }
      if (li == 0) epilogue<EPI, RPW>(a, cur * RW + sub * RPW, acc, res_cur, pos);
    }
  }
}

// Several columns of x against the same Q4_0 rows (chatnet_matmul with
// 2 <= N <= 16): gemv_kernel's digit path with the digit records of ncols
// columns staged in LDS (column c at c * cstride dwords) and each lane's units,
// loaded once, dotted with every column.  y[c * M + row] = dot(W[row], x[c]) in
// gemv_kernel's exact arithmetic (the same records, the same reduction order),
// so a column's result equals the single-column GEMV's bit for bit wherever
// that runs gemv_kernel (not gemv_ks_kernel's two-wave K split, 4096 < K <= 8192,
// which sums in another order).
template <int NC, int RPW, int LPR, int NU, int BS>
__global__ __launch_bounds__(BS) void gemv_cols_kernel(GemvArgs a, int ncols) {
  using T = QTraits<QT_Q4_0>;
  constexpr int NWV = BS / CN_WAVE;
  constexpr int RW = RPW * (CN_WAVE / LPR);
  constexpr int MAXT = ((T::UNIT / 8) * LPR * NU + BS - 1) / BS;
  // columns whose x loads are issued together before any is digitized
  constexpr int CB = MAXT <= 1 ? 8 : (MAXT <= 2 ? 4 : 2);
  extern __shared__ float smem[];
  const int K = a.K, M = a.n_vrows;
  const int nunits = K / T::UNIT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, li = lane % LPR;
  const int n_iters = (M + RW - 1) / RW;
  const size_t bpr = (size_t)(K / T::BLOCK) * T::BLOCK_BYTES;
  const int wstride = gridDim.x * NWV;
  const int cstride = nunits * XD_UNIT_DW;
  int it = blockIdx.x * NWV + wave;
  uint32_t* xd = reinterpret_cast<uint32_t*>(smem);
  float* red = smem + (size_t)NC * cstride;  // sums of squares, unused

  uint32_t w[RPW][NU][T::NDW];
  issue_loads<QT_Q4_0, RPW, LPR, NU, GEMV_EPI_STORE>(a, it, sub, li, nunits, bpr, w);
  for (int c0 = 0; c0 < ncols; c0 += CB) {
    XStage<MAXT, false> st[CB];
#pragma unroll
    for (int j = 0; j < CB; j++)  // columns past ncols re-read the last
      stage_load<MAXT, false, BS>(a.x + (size_t)min(c0 + j, ncols - 1) * K, nullptr, K, st[j]);
#pragma unroll
    for (int j = 0; j < CB; j++)
      if (c0 + j < ncols) stage_digitize<MAXT, false, BS>(st[j], K, xd + (size_t)(c0 + j) * cstride, red);
  }
  __syncthreads();
  while (it < n_iters) {
    float acc[NC][RPW];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int i = 0; i < RPW; i++) acc[c][i] = 0.f;
#pragma unroll
    for (int n = 0; n < NU; n++) {
      const int u = li + LPR * n;
      if (u < nunits) {
        uint32_t wu[RPW][T::NDW];
#pragma unroll
        for (int i = 0; i < RPW; i++)
#pragma unroll
          for (int k = 0; k < T::NDW; k++) wu[i][k] = w[i][n][k];
#pragma unroll
        for (int c = 0; c < NC; c++)
          if (c < ncols) dot_unit_q4_0_dig<RPW>(wu, xd + (size_t)c * cstride + u * XD_UNIT_DW, acc[c]);
      }
    }
    const int cur = it;
    it += wstride;
    if (it < n_iters) issue_loads<QT_Q4_0, RPW, LPR, NU, GEMV_EPI_STORE>(a, it, sub, li, nunits, bpr, w);
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int i = 0; i < RPW; i++)
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) acc[c][i] += __shfl_xor(acc[c][i], off, CN_WAVE);
    if (li == 0) {
#pragma unroll
      for (int c = 0; c < NC; c++)
#pragma unroll
        for (int i = 0; i < RPW; i++) {
          const int row = cur * RW + sub * RPW + i;
          if (c < ncols && row < M) a.out[0][(size_t)c * M + row] = acc[c][i];
        }
    }
  }
}

template <int NC, int RPW, int LPR, int NU>
hipError_t launch_cols_k(const GemvArgs& a, int ncols, int num_cus, hipStream_t st) {
  constexpr int BS = 512, RW = RPW * (CN_WAVE / LPR);
  const size_t smem = ((size_t)NC * (a.K / 64) * XD_UNIT_DW + 16) * sizeof(float);
  const auto kern = &gemv_cols_kernel<NC, RPW, LPR, NU, BS>;
  static std::atomic<uint64_t> lds_done{0};
  const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(kern), lds_done);
  if (e != hipSuccess) return e;
  const int per_cu = (int)((160 * 1024) / smem) < 2 ? 1 : 2;
  const int waves = (a.n_vrows + RW - 1) / RW;
  int grid = (waves + BS / CN_WAVE - 1) / (BS / CN_WAVE);
  if (grid > per_cu * num_cus) grid = per_cu * num_cus;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(BS), smem, st, a, ncols);
  return hipGetLastError();
}

// Two rows per lane while that still gives every CU a workgroup, else one.
template <int NC, int LPR, int NU>
hipError_t launch_cols_rows(const GemvArgs& a, int ncols, int num_cus, hipStream_t st) {
  if constexpr (NU <= 2) {
    const int wg2 = (a.n_vrows + 2 * (CN_WAVE / LPR) * 8 - 1) / (2 * (CN_WAVE / LPR) * 8);
    if (wg2 >= num_cus) return launch_cols_k<NC, 2, LPR, NU>(a, ncols, num_cus, st);
  }
  return launch_cols_k<NC, 1, LPR, NU>(a, ncols, num_cus, st);
}

template <int NC>
hipError_t launch_cols_nc(const GemvArgs& a, int ncols, int num_cus, hipStream_t st) {
  const int nunits = a.K / 64;
  if (nunits <= 32) return launch_cols_rows<NC, 32, 1>(a, ncols, num_cus, st);
  if (nunits <= 64) return launch_cols_rows<NC, 64, 1>(a, ncols, num_cus, st);
  if (nunits <= 128) return launch_cols_rows<NC, 64, 2>(a, ncols, num_cus, st);
  if (nunits <= 192) return launch_cols_rows<NC, 64, 3>(a, ncols, num_cus, st);
  return launch_cols_rows<NC, 64, 4>(a, ncols, num_cus, st);
}

template <int QT>
size_t gemv_smem_bytes(int K) {
  using T = QTraits<QT>;
  const int nunits = K / T::UNIT;
  // digit records (base 16: Q4_0, Q4_K up to 32 half super-blocks per row;
  // base 256 per 128 elements otherwise) + one float per wave
  if (QT == QT_Q4_0 || (QT == QT_Q4_K && nunits <= 32)) return ((size_t)(K >> 6) * XD_UNIT_DW + 16) * sizeof(uint32_t);
  return ((size_t)((K + 127) >> 7) * XD6_UNIT_DW + 16) * sizeof(uint32_t);
}

// Launch shape of one GEMV: lanes per row, units per lane, rows per lane,
// threads per workgroup and workgroups.
struct GemvShape {
  int lpr, nu, rpw, bs, grid;
};

// Q4_0: the (LPR, NU) pair that wastes the fewest lanes (NU <= 4, ties to the
// wider LPR).  Rows per lane: the smallest of 2, 4, 8 (register budget
// permitting) whose waves would all be resident at once (20, 16 and 12 waves
// per CU assumed for 2, 4 and 8 rows).  256-thread workgroups, at most two per
// CU, with further rows taken by a grid-stride loop; when 512-thread
// workgroups bring the launch to one workgroup per CU they are used instead,
// so x is staged once per CU (measured on 4096x4096 and 4096x11008: 4.85 ->
// 4.52 us and 10.1 -> 9.1 us).  Single-round shapes with more rows per lane,
// and 1024- or 128-thread workgroups, measured slower on every decode GEMV of
// the 1.1B and 7B shapes.
// K-quants: one super-block per lane (NU = 1), 2 rows, LPR the smallest power
// of two covering the row (min 16), 256 threads, at most two workgroups per CU.
// Q8_0: Q4_0's (LPR, NU) with 2 rows per lane and 256 threads.
template <int QT>
GemvShape pick_shape(int K, int n_vrows, int num_cus, bool allow8, bool isolated, bool paired) {
  using T = QTraits<QT>;
  const int nunits = K / T::UNIT;
  GemvShape s{64, 1, 2, CN_BLOCK, 1};
  if (QT == QT_Q8_0) {  // Q4_0's (LPR, NU) rule, two rows per lane
    double best = -1.0;
    for (int lpr = 64; lpr >= 32; lpr >>= 1)
      for (int nu = 1; nu <= 4; nu++) {
        if (lpr * nu < nunits) continue;
        const double eff = (double)nunits / (double)(lpr * nu);
        if (eff > best + 1e-9) { best = eff; s.lpr = lpr; s.nu = nu; }
        break;
      }
    if (best < 0) { s.lpr = 64; s.nu = 4; }
  } else if (QT == QT_Q4_0) {
    double best = -1.0;
    for (int lpr = 64; lpr >= 32; lpr >>= 1)
      for (int nu = 1; nu <= 4; nu++) {
        if (lpr * nu < nunits) continue;
        const double eff = (double)nunits / (double)(lpr * nu);
        if (eff > best + 1e-9) { best = eff; s.lpr = lpr; s.nu = nu; }
        break;  // larger nu only adds idle lanes
      }
    if (best < 0) { s.lpr = 64; s.nu = 4; }
    const int max_rpw = s.nu == 1 ? (allow8 ? 8 : 4) : (s.nu == 2 ? 4 : 2);
    const int resident[9] = {0, 0, 20, 0, 16, 0, 0, 0, 12};
    s.rpw = max_rpw;
    for (int rpw = 2; rpw <= max_rpw; rpw *= 2) {
      const int rw = rpw * (64 / s.lpr);
      if ((n_vrows + rw - 1) / rw <= num_cus * resident[rpw]) {
        s.rpw = rpw;
        break;
      }
    }
  } else {  // K-quants: half super-blocks, up to 128 per row (K <= 16384)
    s.rpw = 2;
    s.lpr = nunits <= 16 ? 16 : (nunits <= 32 ? 32 : 64);
    s.nu = (nunits + s.lpr - 1) / s.lpr;
    if (QT == QT_Q5_K && nunits > 64 && nunits <= 96 && !paired) {
      // 65..96 half super-blocks (8192 < K <= 12288, the 7B down projection):
      // 32 lanes x 3 units fill 96 slots where 64 x 2 would leave a third idle;
      // one row per lane keeps the three units' registers in budget (4096 x
      // 11008 cold: 13.6 -> 12.0 us; Q6_K measured 14.9 -> 15.3, so it keeps
      // 64 x 2)
      s.rpw = 1;
      s.lpr = 32;
      s.nu = 3;
    }
  }
  if (QT == QT_Q4_0 && s.nu == 3 && !paired) {
    // Rows of 129..192 units (8192 < K <= 12288): one row per lane, so the
    // launch has twice the waves and each finishes its three units sooner
    // (7B down projection 4096x11008 in the decode graph: 723 -> 730 tok/s),
    // in 512-thread workgroups at most two per CU.
    s.rpw = 1;
    s.bs = 512;
    const int waves1 = (n_vrows + (64 / s.lpr) - 1) / (64 / s.lpr);
    s.grid = (waves1 + 7) / 8;
    if (s.grid > 2 * num_cus) s.grid = 2 * num_cus;
    return s;
  }
  if (QT == QT_Q4_0) {
    // Launches that reach 16 waves per CU at two rows per lane run that way, in
    // 512-thread workgroups at most two per CU: more waves in flight beat fewer
    // wider ones (7B QKV and gate/up each +3.4 % decode tok/s, the stand-alone
    // 11008x4096 product 7.9 -> 7.2 us).  Smaller stand-alone products (nothing
    // fused) also take two rows per lane, in 256-thread workgroups at most three
    // per CU; smaller fused launches keep the rule above, measured in the
    // TinyLlama decode graph.
    const int rw2 = 2 * (64 / s.lpr);
    const int waves2 = (n_vrows + rw2 - 1) / rw2;
    if (waves2 >= 16 * num_cus) {
      s.rpw = 2;
      s.bs = 512;
      s.grid = (waves2 + 7) / 8;
      if (s.grid > 2 * num_cus) s.grid = 2 * num_cus;
      return s;
    }
    if (isolated) {
      s.rpw = 2;
      s.grid = (waves2 + 3) / 4;
      if (s.grid > 3 * num_cus) s.grid = 3 * num_cus;
      return s;
    }
  }
  const int rw = s.rpw * (64 / s.lpr);
  const int waves = (n_vrows + rw - 1) / rw;
  s.grid = (waves + 3) / 4;
  if (QT == QT_Q4_0 && s.grid > num_cus && (waves + 7) / 8 <= num_cus) {
    s.bs = 512;
    s.grid = (waves + 7) / 8;
  }
  // one-unit Q6_K lanes (<= 128 VGPRs) run best at four 256-thread workgroups
  // per CU (32000x4096 29.2 -> 28.0 us), two-unit K-quant lanes (~160 VGPRs,
  // x digitized before the weight loads) at three, Q4_K and Q5_K one-unit
  // lanes at two
  const bool kq = QT == QT_Q3_K || QT == QT_Q4_K || QT == QT_Q5_K || QT == QT_Q6_K || QT == QT_Q6_KQ;
  const int per_cu = (QT == QT_Q6_K || QT == QT_Q3_K) && s.nu == 1 ? 4 : (kq && s.nu >= 2 ? 3 : 2);
  if (s.grid > per_cu * num_cus) s.grid = per_cu * num_cus;
  if (s.grid < 1) s.grid = 1;
  return s;
}

// One instantiation's launch.  The base-256 digit records of rows longer than
// 15872 take more than 64 KB of LDS, which must be allowed explicitly (once
// per kernel and device, for the CU's whole LDS).
template <int QT, int RPW, int LPR, int NU, int EPI, int BS>
hipError_t launch_one(const GemvArgs& a, int grid, size_t smem, hipStream_t st) {
  const auto kern = &gemv_kernel<QT, RPW, LPR, NU, EPI, BS>;
  if (smem > 65536) {
    static std::atomic<uint64_t> lds_done{0};
    const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(kern), lds_done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(BS), smem, st, a);
  return hipGetLastError();
}

template <int QT, int RPW, int NU, int EPI, int BS>
hipError_t launch_k(const GemvArgs& a, int lpr, int grid, size_t smem, hipStream_t st) {
  if constexpr (QT != QT_Q4_0) {
    if (lpr == 16) return launch_one<QT, RPW, 16, NU, EPI, BS>(a, grid, smem, st);
  }
  if (lpr == 32) return launch_one<QT, RPW, 32, NU, EPI, BS>(a, grid, smem, st);
  return launch_one<QT, RPW, 64, NU, EPI, BS>(a, grid, smem, st);
}

template <int QT, int RPW, int NU, int EPI>
hipError_t launch_bs(const GemvArgs& a, const GemvShape& s, size_t smem, hipStream_t st) {
  if (s.bs == 512) return launch_k<QT, RPW, NU, EPI, 512>(a, s.lpr, s.grid, smem, st);
  return launch_k<QT, RPW, NU, EPI, 256>(a, s.lpr, s.grid, smem, st);
}


// Q4_0 rows of 65..128 units (4096 < K <= 8192) with a store or residual-add
// epilogue: the row's K is split over KS waves of a workgroup, one 36-byte
// unit per lane, so the launch has as many waves in flight as a 4096-wide
// product of the same bytes instead of three units per lane at a third of
// the waves.  The KS partial sums of a row group meet in LDS; the first wave
// adds them in ks order and runs the epilogue.  Every wave of a workgroup runs
// the same number of loop iterations (base is per workgroup, the work is
// predicated), so the barriers always match.
template <int RPW, int KS, int EPI, int BS>
__global__ __launch_bounds__(BS) void gemv_ks_kernel(GemvArgs a) {
  static_assert(EPI == GEMV_EPI_STORE || EPI == GEMV_EPI_ADD, "K split for store / residual add only");
  constexpr int NWV = BS / CN_WAVE;
  static_assert(NWV % KS == 0, "whole row groups per workgroup");
  constexpr int NRG = NWV / KS;  // row groups per workgroup
  constexpr int NR = res_count<EPI, RPW>();
  extern __shared__ float smem[];
  const int K = a.K;
  const int nunits = K >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave / KS, ks = wave % KS;
  const int u = ks * CN_WAVE + lane;  // this lane's unit
  const int n_iters = (a.n_vrows + RPW - 1) / RPW;
  const size_t bpr = (size_t)nunits * 36;
  const int gstride = gridDim.x * NRG;
  int base = blockIdx.x * NRG;
  int it = base + rg;

  uint32_t w[RPW][9];
  float res[NR];
  const int stop_v = cn_load_late(stop_flag(a));  // consumed after staging
  auto load = [&](int itn) {  // straight-line loads, as issue_loads
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int vr = itn * RPW + i < a.n_vrows ? itn * RPW + i : a.n_vrows - 1;
      load_unit<QT_Q4_0>((const cn_gbyte*)a.w[0] + (size_t)vr * bpr, u < nunits ? u : nunits - 1, w[i]);
    }
  };
  // items per thread: K/8 <= 8 * 64 * KS items over BS = 64 * KS * NRG threads
  constexpr int MAXT = (8 * CN_WAVE * KS + BS - 1) / BS;
  XStage<MAXT, false> st;
  stage_load<MAXT, false, BS>(a.x, nullptr, K, st);
  load(it);
  load_residual<EPI, RPW, NR>(a, it * RPW, lane, 0, res);
  uint32_t* xd = reinterpret_cast<uint32_t*>(smem);
  float* xred = smem + (size_t)nunits * XD_UNIT_DW;
  float* part = xred + 16;  // [NRG][KS-1][RPW]
  stage_digitize<MAXT, false, BS>(st, K, xd, xred);
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(stop_v)) return;
  while (base < n_iters) {
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[i] = 0.f;
    if (u < nunits) dot_unit_q4_0_dig<RPW>(w, xd + u * XD_UNIT_DW, acc);
    const int cur = it;
    float res_cur[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) res_cur[i] = res[i];
    base += gstride;
    it += gstride;
    if (base < n_iters) {
      load(it);
      load_residual<EPI, RPW, NR>(a, it * RPW, lane, 0, res);
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
#pragma unroll
      for (int off = CN_WAVE / 2; off > 0; off >>= 1) acc[i] += __shfl_xor(acc[i], off, CN_WAVE);
    }
    if (ks > 0 && lane == 0) {
#pragma unroll
      for (int i = 0; i < RPW; i++) part[(rg * (KS - 1) + ks - 1) * RPW + i] = acc[i];
    }
    __syncthreads();
    if (ks == 0 && lane == 0 && cur < n_iters) {
#pragma unroll
      for (int k = 1; k < KS; k++)
#pragma unroll
        for (int i = 0; i < RPW; i++) acc[i] += part[(rg * (KS - 1) + k - 1) * RPW + i];
      epilogue<EPI, RPW>(a, cur * RPW, acc, res_cur, 0);
    }
    __syncthreads();
  }
}

template <int KS, int EPI, int RPW = 2>
hipError_t launch_ks(const GemvArgs& a, hipStream_t st) {
  constexpr int NRG = 2, BS = CN_WAVE * KS * NRG;
  const int n_iters = (a.n_vrows + RPW - 1) / RPW;
  const int grid = (n_iters + NRG - 1) / NRG;
  const size_t smem = ((size_t)(a.K >> 6) * XD_UNIT_DW + 16 + NRG * (KS - 1) * RPW) * sizeof(float);
  hipLaunchKernelGGL((gemv_ks_kernel<RPW, KS, EPI, BS>), dim3(grid), dim3(BS), smem, st, a);
  return hipGetLastError();
}

template <int QT, int EPI>
hipError_t launch_qt(const GemvArgs& a, int num_cus, hipStream_t st) {
  if constexpr (QT == QT_Q6_K && (EPI == GEMV_EPI_STORE || EPI == GEMV_EPI_ADD)) {
    // Rows of 65..96 half super-blocks (the 7B down projection, 86): 64 lanes
    // x 2 half super-blocks leave a third of the slots idle, 64 lanes x 3
    // quarters a tenth
    const int halves = a.K / 128;
    if (halves > 64 && halves <= 96) return launch_qt<QT_Q6_KQ, EPI>(a, num_cus, st);
  }
  // 8 rows per lane only for the norm-fused epilogues (the wide QKV, gate/up
  // and LM-head launches); hipcc 7.2 fails to compile the 8-row STORE/ADD forms.
  constexpr bool kAllow8 = EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_SWIGLU || EPI == GEMV_EPI_LOGITS;
  if constexpr (QT == QT_Q4_0 && (EPI == GEMV_EPI_STORE || EPI == GEMV_EPI_ADD)) {
    // 4096 < K <= 8192: K split over two waves (TinyLlama's down projection
    // 2048x5632: 6.05 -> 5.70 us).  Longer rows keep three or four units per
    // lane: split three ways, the 7B down projection lost 5 % of decode at two
    // rows per lane (1024 six-wave workgroups, not all resident) and 2 % at
    // four.
    const int nunits = a.K >> 6;
    if (nunits > 64 && nunits <= 128) return launch_ks<2, EPI>(a, st);
  }
  // the QKV and SwiGLU epilogues take a lane's rows in pairs: never one row per lane
  constexpr bool kPaired = EPI == GEMV_EPI_QKV || EPI == GEMV_EPI_SWIGLU;
  const GemvShape s = pick_shape<QT>(a.K, a.n_vrows, num_cus, kAllow8, EPI == GEMV_EPI_STORE, kPaired);
  const size_t smem = gemv_smem_bytes<QT>(a.K);
  if constexpr (QT == QT_Q4_0) {
    if (s.nu == 1) {
      if constexpr (kAllow8) {
        if (s.rpw == 8) return launch_bs<QT, 8, 1, EPI>(a, s, smem, st);
      }
      if (s.rpw == 4) return launch_bs<QT, 4, 1, EPI>(a, s, smem, st);
      return launch_bs<QT, 2, 1, EPI>(a, s, smem, st);
    }
    if (s.nu == 2) {
      if (s.rpw == 4) return launch_bs<QT, 4, 2, EPI>(a, s, smem, st);
      return launch_bs<QT, 2, 2, EPI>(a, s, smem, st);
    }
    if (s.nu == 3) {
      if constexpr (kPaired) return launch_bs<QT, 2, 3, EPI>(a, s, smem, st);
      else return launch_bs<QT, 1, 3, EPI>(a, s, smem, st);
    }
    return launch_bs<QT, 2, 4, EPI>(a, s, smem, st);
  } else if constexpr (QT == QT_Q8_0) {
    if (s.nu == 1) return launch_k<QT, 2, 1, EPI, CN_BLOCK>(a, s.lpr, s.grid, smem, st);
    if (s.nu == 2) return launch_k<QT, 2, 2, EPI, CN_BLOCK>(a, s.lpr, s.grid, smem, st);
    if (s.nu == 3) return launch_k<QT, 2, 3, EPI, CN_BLOCK>(a, s.lpr, s.grid, smem, st);
    return launch_k<QT, 2, 4, EPI, CN_BLOCK>(a, s.lpr, s.grid, smem, st);
  } else if constexpr (QT == QT_Q6_KQ) {
    return launch_one<QT, 2, 64, 3, EPI, CN_BLOCK>(a, s.grid, smem, st);  // 129..192 quarters per row
  } else {
    if (s.nu == 1) return launch_k<QT, 2, 1, EPI, CN_BLOCK>(a, s.lpr, s.grid, smem, st);
    if constexpr (QT == QT_Q5_K && !kPaired) {
      if (s.nu == 3) return launch_one<QT, 1, 32, 3, EPI, CN_BLOCK>(a, s.grid, smem, st);
    }
    return launch_k<QT, 2, 2, EPI, CN_BLOCK>(a, s.lpr, s.grid, smem, st);
  }
}

template <int EPI>
hipError_t launch_epi(int qtype, const GemvArgs& a, int num_cus, hipStream_t st) {
  switch (qtype) {
    case QT_Q4_0: return launch_qt<QT_Q4_0, EPI>(a, num_cus, st);
    case QT_Q4_K: return launch_qt<QT_Q4_K, EPI>(a, num_cus, st);
    case QT_Q6_K: return launch_qt<QT_Q6_K, EPI>(a, num_cus, st);
    case QT_Q3_K: return launch_qt<QT_Q3_K, EPI>(a, num_cus, st);
    case QT_Q8_0: return launch_qt<QT_Q8_0, EPI>(a, num_cus, st);
    case QT_Q5_K: return launch_qt<QT_Q5_K, EPI>(a, num_cus, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

size_t gemv_lds_bytes(int qtype, int K) {
  switch (qtype) {
    case QT_Q4_0: return gemv_smem_bytes<QT_Q4_0>(K);
    case QT_Q4_K: return gemv_smem_bytes<QT_Q4_K>(K);
    case QT_Q6_K: return gemv_smem_bytes<QT_Q6_K>(K);
    case QT_Q3_K: return gemv_smem_bytes<QT_Q3_K>(K);
    case QT_Q8_0: return gemv_smem_bytes<QT_Q8_0>(K);
    case QT_Q5_K: return gemv_smem_bytes<QT_Q5_K>(K);
    default: return 0;
  }
}

// The launch shapes cover rows of up to 256 lanes x units: K <= 16384.
bool gemv_supports(int qtype, int K) {
  switch (qtype) {
    case 0:  // F32 and F16 rows (gemv_float.hip): K floats of x in LDS
    case 1:
    case QT_Q4_0:
    case QT_Q8_0: return K > 0 && K % 64 == 0 && K <= 16384;
    case QT_Q3_K:
    case QT_Q4_K:
    case QT_Q5_K:
    case QT_Q6_K: return K > 0 && K % 256 == 0 && K <= 16384;
    // served as packed units (gemv_launch with kGemvPacked)
    case 3:   // Q4_1
    case 6:   // Q5_0
    case 7: return K > 0 && K % 64 == 0 && K <= 16384;  // Q5_1
    case 20: return K > 0 && K % 64 == 0 && K <= 16384;  // IQ4_NL
    case 10:  // Q2_K
    case 15:  // Q8_K
    case 16:  // IQ2_XXS
    case 17:  // IQ2_XS
    case 18:  // IQ3_XXS
    case 19:  // IQ1_S
    case 21:  // IQ3_S
    case 22:  // IQ2_S
    case 23:  // IQ4_XS
    case 29: return K > 0 && K % 256 == 0 && K <= 16384;  // IQ1_M
    default: return false;
  }
}

int gemv_cols_max(int K) {
  if (K <= 0 || K % 64 != 0 || K > 16384) return 0;
  const size_t per_col = (size_t)(K / 64) * XD_UNIT_DW * sizeof(float);
  const int n = (int)((150 * 1024) / per_col);
  return n >= 16 ? 16 : (n >= 8 ? 8 : (n >= 4 ? 4 : (n >= 2 ? 2 : 1)));
}

hipError_t gemv_cols_launch(const void* w, const float* x, float* y, int M, int K, int N, int num_cus,
                            hipStream_t st) {
  const int g = gemv_cols_max(K);
  if (g < 2 || M <= 0 || N < 1 || !w || !x || !y) return hipErrorInvalidValue;
  for (int c0 = 0; c0 < N; c0 += g) {
    const int nc = N - c0 < g ? N - c0 : g;
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    a.w[0] = a.w[1] = a.w[2] = static_cast<const uint8_t*>(w);
    a.seg_rows[0] = M;
    a.n_vrows = M;
    a.K = K;
    a.x = x + (size_t)c0 * K;
    a.out[0] = y + (size_t)c0 * M;
    hipError_t e;
    if (nc <= 2) e = launch_cols_nc<2>(a, nc, num_cus, st);
    else if (nc <= 4) e = launch_cols_nc<4>(a, nc, num_cus, st);
    else if (nc <= 8) e = launch_cols_nc<8>(a, nc, num_cus, st);
    else e = launch_cols_nc<16>(a, nc, num_cus, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool gemv_needs_pack(int qtype) {
  return qtype == 3 || qtype == 6 || qtype == 7 || qtype == 10 || qtype == 15 || (qtype >= 16 && qtype <= 23) ||
         qtype == 29;
}

hipError_t gemv_launch(int qtype, int epi, const GemvArgs& a, int num_cus, hipStream_t st) {
  if (qtype == 0 || qtype == 1 || qtype == kGemvPacked) return gemv_float_launch(qtype, epi, a, num_cus, st);
  if (qtype != QT_Q4_0 && qtype != QT_Q8_0 && qtype != QT_Q3_K && qtype != QT_Q4_K && qtype != QT_Q5_K &&
      qtype != QT_Q6_K)
    return hipErrorInvalidValue;  // the packed-unit types are launched as kGemvPacked
  switch (epi) {
    case GEMV_EPI_STORE: return launch_epi<GEMV_EPI_STORE>(qtype, a, num_cus, st);
    case GEMV_EPI_ADD: return launch_epi<GEMV_EPI_ADD>(qtype, a, num_cus, st);
    case GEMV_EPI_QKV: return launch_epi<GEMV_EPI_QKV>(qtype, a, num_cus, st);
    case GEMV_EPI_SWIGLU: return launch_epi<GEMV_EPI_SWIGLU>(qtype, a, num_cus, st);
    case GEMV_EPI_LOGITS: return launch_epi<GEMV_EPI_LOGITS>(qtype, a, num_cus, st);
    case GEMV_EPI_ADD_MERGE:
      if (a.msplits < 2 || a.msplits > kFoldMaxSplits || a.mchunk < 1 || a.head_dim % 32 != 0)
        return hipErrorInvalidValue;
      if (merge_epi(a.msplits) == kEpiMerge2) return launch_epi<kEpiMerge2>(qtype, a, num_cus, st);
      if (merge_epi(a.msplits) == kEpiMerge4) return launch_epi<kEpiMerge4>(qtype, a, num_cus, st);
      return launch_epi<GEMV_EPI_ADD_MERGE>(qtype, a, num_cus, st);
    default: return hipErrorInvalidValue;
  }
}
