// gemm.hip — quantized-weight GEMM on the bf16 matrix cores of gfx950 (N > 1).
//
// y[n][m] = sum_k W[m][k] * x[n][k] for a batch of N inputs: the batched form
// of TensorMath.MatVecMulQ4_0 (src/ChatNet.Core/Tensors/TensorMath.cs:548-578)
// that a multi-token LlamaModel.Forward span (LlamaModel.cs:93-238) needs.
//
// Operands: W stays in its raw Q4_0 blocks in HBM; x arrives as bf16 [N][K]
// (converted, or RMS-normalised and converted, by the producer kernel).
// Each Q4_0 block (32 weights along K) is exactly the K extent of one
// v_mfma_f32_16x16x32_bf16, so a wave dequantizes a block of 16 rows straight
// into the MFMA A operand in registers: lane l holds row l%16 and the 8
// consecutive k in [8g, 8g+8), g = l/16, which are the low (g < 2) or high
// (g >= 2) nibbles of qs[8(g&1) .. 8(g&1)+7].  Each value is d*(q-8) computed
// exactly in fp32 (one fma) and rounded once to bf16.  W needs no LDS: every
// W element is used by exactly one wave.  The x tile (BN columns x KC of K) is
// shared by the 4 waves through LDS, double-buffered; the next chunk's x and W
// loads are issued before the current chunk's MFMAs.  Accumulation is fp32.
//
// Tiles: a workgroup owns BM = 64*MT rows (16*MT per wave) x BN = 16*NT
// columns; when that leaves the chip under-filled the K range is split and
// the partial tiles are summed by gemm_reduce_kernel, which then applies the
// epilogue.  Epilogues: STORE y = acc, ADD y += acc (residual), SWIGLU (rows
// interleave gate/up, h = silu(gate)*up written as bf16 for the next GEMM).
// A second, exact-weight kernel (gemm_q4_0_x2_kernel, below) serves the
// forward pass of multi-token spans.
#include "device_common.h"
#include "kernels.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int Q4_0_UNIT_DW = 9;  // two Q4_0 blocks = 64 weights = 36 bytes

// W rows of the virtual row `vr`: single matrix, three concatenated (q|k|v)
// or two interleaved (gate even, up odd).
__device__ __forceinline__ const uint32_t* gemm_row_ptr(const GemmArgs& a, int vr, int row_dw) {
  if (vr >= a.M) return nullptr;
  int seg = 0, r = vr;
  if (a.seg_mode == GEMM_SEG_INTERLEAVE) {
    seg = vr & 1;
    r = vr >> 1;
  } else if (a.seg_mode == GEMM_SEG_CONCAT) {
    if (r >= a.seg_rows[0]) {
      r -= a.seg_rows[0];
      seg = 1;
      if (r >= a.seg_rows[1]) {
        r -= a.seg_rows[1];
        seg = 2;
      }
    }
  }
  return reinterpret_cast<const uint32_t*>(a.w[seg]) + (size_t)r * row_dw;
}

// The 7 dwords of a 36-byte unit that lane group g needs: d of both blocks
// and 8 bytes of qs per block (qs[0..7] for even g, qs[8..15] for odd g).
struct UnitRegs {
  uint32_t a0, a1, a2, a3, b0, b1, b2;
};

__device__ __forceinline__ void load_unit(const uint32_t* p, int h, UnitRegs& u) {
  if (p) {
    u.a0 = p[0];
    u.a1 = p[2 * h];
    u.a2 = p[2 * h + 1];
    u.a3 = p[2 * h + 2];
    u.b0 = p[4];
    u.b1 = p[5 + 2 * h];
    u.b2 = p[6 + 2 * h];
  } else {
    u.a0 = u.a1 = u.a2 = u.a3 = u.b0 = u.b1 = u.b2 = 0u;
  }
}

// 8 weights d*(q-8) as bf16 from 8 nibbles held in bytes of q0 (k 0..3), q1 (k 4..7).
__device__ __forceinline__ bf16x8 dequant8(uint32_t q0, uint32_t q1, float d) {
  const float nd = -8.0f * d;
  bf16x8 r;
  r[0] = (__bf16)fmaf(cn_ubyte<0>(q0), d, nd);
  r[1] = (__bf16)fmaf(cn_ubyte<1>(q0), d, nd);
  r[2] = (__bf16)fmaf(cn_ubyte<2>(q0), d, nd);
  r[3] = (__bf16)fmaf(cn_ubyte<3>(q0), d, nd);
  r[4] = (__bf16)fmaf(cn_ubyte<0>(q1), d, nd);
  r[5] = (__bf16)fmaf(cn_ubyte<1>(q1), d, nd);
  r[6] = (__bf16)fmaf(cn_ubyte<2>(q1), d, nd);
  r[7] = (__bf16)fmaf(cn_ubyte<3>(q1), d, nd);
  return r;
}

// A operands of block A (first 32 weights) and block B of a unit for lane group g.
__device__ __forceinline__ void dequant_unit(const UnitRegs& u, int nshift, bf16x8& fa, bf16x8& fb) {
  const uint32_t qa0 = (__builtin_amdgcn_alignbyte(u.a2, u.a1, 2) >> nshift) & 0x0F0F0F0Fu;
  const uint32_t qa1 = (__builtin_amdgcn_alignbyte(u.a3, u.a2, 2) >> nshift) & 0x0F0F0F0Fu;
  const uint32_t qb0 = (u.b1 >> nshift) & 0x0F0F0F0Fu;
  const uint32_t qb1 = (u.b2 >> nshift) & 0x0F0F0F0Fu;
  fa = dequant8(qa0, qa1, cn_h2f(u.a0));
  fb = dequant8(qb0, qb1, cn_h2f(u.b0 >> 16));
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  const __bf16 a = (__bf16)lo, b = (__bf16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// v as bf16 hi + bf16 lo (hi + lo carries ~16 significant bits of v).
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  const __bf16 h = (__bf16)v;
  const __bf16 l = (__bf16)(v - (float)h);
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, l);
}

// h[n][j] = silu(gate) * up, as bf16 (and its low part when hb_lo is set).
__device__ __forceinline__ void write_h(const GemmArgs& a, int n, int j, float v) {
  const size_t i = (size_t)n * a.ldh + j;
  if (a.hb_lo) {
    uint16_t hi, lo;
    split_bf16(v, hi, lo);
    a.hb[i] = hi;
    a.hb_lo[i] = lo;
  } else {
    a.hb[i] = __builtin_bit_cast(uint16_t, (__bf16)v);
  }
}

// Final write of 4 consecutive rows m..m+3 of column n.
__device__ __forceinline__ void write_out4(const GemmArgs& a, int epi, int n, int m, f32x4 v) {
  if (n >= a.N || m >= a.M) return;
  const bool full = (m + 3 < a.M) && ((a.ldy & 3) == 0);
  if (epi == GEMV_EPI_SWIGLU) {
    // rows (m, m+1) and (m+2, m+3) are (gate, up) pairs of h[m/2], h[m/2+1]
    if (m + 3 < a.M && !a.hb_lo) {
      uint16_t* h = a.hb + (size_t)n * a.ldh + (m >> 1);
      *reinterpret_cast<uint32_t*>(h) = pack2_bf16(silu_mul(v[0], v[1]), silu_mul(v[2], v[3]));
    } else {
      write_h(a, n, m >> 1, silu_mul(v[0], v[1]));
      if (m + 3 < a.M) write_h(a, n, (m >> 1) + 1, silu_mul(v[2], v[3]));
    }
    return;
  }
  float* y = a.y + (size_t)n * a.ldy + m;
  if (full) {
    f32x4* p = reinterpret_cast<f32x4*>(y);
    if (epi == GEMV_EPI_ADD) *p = *p + v;
    else *p = v;
  } else {
    for (int i = 0; i < 4 && m + i < a.M; i++) y[i] = (epi == GEMV_EPI_ADD) ? y[i] + v[i] : v[i];
  }
}

template <int MT, int NT, int KC>
__global__ __launch_bounds__(CN_BLOCK) void gemm_q4_0_kernel(GemmArgs a) {
  constexpr int BN = 16 * NT;
  constexpr int XS = KC + 8;             // LDS row stride (bf16): 16 B pad -> conflict-free b128 reads
  constexpr int XV = BN * KC / 8;        // 16-byte x vectors per chunk
  constexpr int XR = (XV + CN_BLOCK - 1) / CN_BLOCK;
  constexpr int UPC = KC / 64;           // units per chunk
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][BN * XS];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int h = g & 1, nshift = (g >> 1) * 4;

  // Workgroup -> (m tile, n tile, K split); the n tiles of one m tile are
  // adjacent so their W reads meet in L2.
  const int n_nt = (a.N + BN - 1) / BN;
  int bid = blockIdx.x;
  const int ks = bid % a.splits;
  bid /= a.splits;
  const int nt = bid % n_nt;
  const int mt = bid / n_nt;
  const int m_wave = mt * 64 * MT + wave * 16 * MT;
  const int n0 = nt * BN;

  const int nchunks = a.K / KC;
  const int cps = (nchunks + a.splits - 1) / a.splits;
  const int c_begin = ks * cps;
  const int c_end = min(nchunks, c_begin + cps);

  const int row_dw = a.K / 64 * Q4_0_UNIT_DW;
  const uint32_t* wrow[MT];
#pragma unroll
  for (int r = 0; r < MT; r++) wrow[r] = gemm_row_ptr(a, m_wave + 16 * r + li, row_dw);

  f32x4 acc[MT][NT];
#pragma unroll
  for (int r = 0; r < MT; r++)
#pragma unroll
    for (int c = 0; c < NT; c++) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (c_begin >= c_end) {
    // empty split: contributes zeros
  } else {
    uint4 xr[XR];
    UnitRegs wr[MT][UPC];

    auto load_x = [&](int c) {
      const int k0 = c * KC;
#pragma unroll
      for (int j = 0; j < XR; j++) {
        const int i = threadIdx.x + CN_BLOCK * j;
        const int n = i / (KC / 8), k8 = i % (KC / 8);
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (i < XV && n0 + n < a.N)
          v = *reinterpret_cast<const uint4*>(a.xb + (size_t)(n0 + n) * a.K + k0 + 8 * k8);
        xr[j] = v;
      }
    };
    auto store_x = [&](int buf) {
#pragma unroll
      for (int j = 0; j < XR; j++) {
        const int i = threadIdx.x + CN_BLOCK * j;
        if (i < XV) {
          const int n = i / (KC / 8), k8 = i % (KC / 8);
          *reinterpret_cast<uint4*>(&xs[buf][n * XS + 8 * k8]) = xr[j];
        }
      }
    };
    auto load_w = [&](int c) {
#pragma unroll
      for (int r = 0; r < MT; r++)
#pragma unroll
        for (int u = 0; u < UPC; u++)
          load_unit(wrow[r] ? wrow[r] + (size_t)(c * UPC + u) * Q4_0_UNIT_DW : nullptr, h, wr[r][u]);
    };

    load_x(c_begin);
    load_w(c_begin);
    store_x(0);
    __syncthreads();

    for (int c = c_begin; c < c_end; c++) {
      const int buf = (c - c_begin) & 1;
      UnitRegs cur[MT][UPC];
#pragma unroll
      for (int r = 0; r < MT; r++)
#pragma unroll
        for (int u = 0; u < UPC; u++) cur[r][u] = wr[r][u];
      const bool more = c + 1 < c_end;
      if (more) {
        load_x(c + 1);  // x first: vector-memory counters retire in order
        load_w(c + 1);
      }
      const uint16_t* xt = xs[buf];
#pragma unroll
      for (int u = 0; u < UPC; u++) {
        bf16x8 fa[MT], fb[MT];
#pragma unroll
        for (int r = 0; r < MT; r++) dequant_unit(cur[r][u], nshift, fa[r], fb[r]);
#pragma unroll
        for (int half = 0; half < 2; half++) {
          const int kofs = u * 64 + half * 32 + 8 * g;
#pragma unroll
          for (int cc = 0; cc < NT; cc++) {
            const uint4 bv = *reinterpret_cast<const uint4*>(&xt[(16 * cc + li) * XS + kofs]);
            const bf16x8 bfr = __builtin_bit_cast(bf16x8, bv);
#pragma unroll
            for (int r = 0; r < MT; r++)
              acc[r][cc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(half ? fb[r] : fa[r], bfr, acc[r][cc], 0, 0, 0);
          }
        }
      }
      if (more) store_x(buf ^ 1);
      __syncthreads();
    }
  }

  // D layout: lane holds rows 4g..4g+3 of column li of each 16x16 tile.
#pragma unroll
  for (int r = 0; r < MT; r++) {
    const int m = m_wave + 16 * r + 4 * g;
#pragma unroll
    for (int cc = 0; cc < NT; cc++) {
      const int n = n0 + 16 * cc + li;
      if (a.splits > 1) {
        if (n < a.N && m < a.M) {
          float* p = a.part + ((size_t)ks * a.N + n) * a.M + m;
          if (m + 3 < a.M && (a.M & 3) == 0) *reinterpret_cast<f32x4*>(p) = acc[r][cc];
          else
            for (int i = 0; i < 4 && m + i < a.M; i++) p[i] = acc[r][cc][i];
        }
      } else {
        write_out4(a, a.epi, n, m, acc[r][cc]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Exact-weight variant for multi-token LlamaModel.Forward spans.
//
// The single-pass kernel rounds both operands to bf16 (2^-9 each), which
// leaves ~3e-3 relative noise per projection; over a 22-layer stack that moves
// logits by ~1e-2 and can flip greedy near-ties.  Here the weights enter the
// MFMA exactly — (q - 8) is a small integer — and x as two bf16 planes
// hi + lo (~2^-17 relative): per Q4_0 block and output
//   p = sum_k x_hi[k] (q_k - 8) + sum_k x_lo[k] (q_k - 8)    (two MFMAs, fp32)
//   acc += d * p
// The operands are swapped relative to the single-pass kernel (x is A, W is
// B) so that a lane's four outputs (columns 4g..4g+3 of the x rows, one W row
// m = li) all need the block scale d of the row that lane itself loaded.
// ---------------------------------------------------------------------------

// Exact (q - 8) of 8 nibbles as bf16.
__device__ __forceinline__ bf16x8 qm8(uint32_t q0, uint32_t q1) {
  bf16x8 r;
  r[0] = (__bf16)(cn_ubyte<0>(q0) - 8.0f);
  r[1] = (__bf16)(cn_ubyte<1>(q0) - 8.0f);
  r[2] = (__bf16)(cn_ubyte<2>(q0) - 8.0f);
  r[3] = (__bf16)(cn_ubyte<3>(q0) - 8.0f);
  r[4] = (__bf16)(cn_ubyte<0>(q1) - 8.0f);
  r[5] = (__bf16)(cn_ubyte<1>(q1) - 8.0f);
  r[6] = (__bf16)(cn_ubyte<2>(q1) - 8.0f);
  r[7] = (__bf16)(cn_ubyte<3>(q1) - 8.0f);
  return r;
}

__device__ __forceinline__ void exact_unit(const UnitRegs& u, int nshift, bf16x8& fa, bf16x8& fb, float& da,
                                           float& db) {
  const uint32_t qa0 = (__builtin_amdgcn_alignbyte(u.a2, u.a1, 2) >> nshift) & 0x0F0F0F0Fu;
  const uint32_t qa1 = (__builtin_amdgcn_alignbyte(u.a3, u.a2, 2) >> nshift) & 0x0F0F0F0Fu;
  const uint32_t qb0 = (u.b1 >> nshift) & 0x0F0F0F0Fu;
  const uint32_t qb1 = (u.b2 >> nshift) & 0x0F0F0F0Fu;
  fa = qm8(qa0, qa1);
  fb = qm8(qb0, qb1);
  da = cn_h2f(u.a0);
  db = cn_h2f(u.b0 >> 16);
}

template <int MT, int NT, int KC>
__global__ __launch_bounds__(CN_BLOCK) void gemm_q4_0_x2_kernel(GemmArgs a) {
  constexpr int BN = 16 * NT;
  constexpr int XS = KC + 8;
  constexpr int XV = BN * KC / 8;
  constexpr int XR = (XV + CN_BLOCK - 1) / CN_BLOCK;
  constexpr int UPC = KC / 64;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][2][BN * XS];  // [buffer][hi, lo]

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int h = g & 1, nshift = (g >> 1) * 4;

  const int n_nt = (a.N + BN - 1) / BN;
  int bid = blockIdx.x;
  const int ks = bid % a.splits;
  bid /= a.splits;
  const int nt = bid % n_nt;
  const int mt = bid / n_nt;
  const int m_wave = mt * 64 * MT + wave * 16 * MT;
  const int n0 = nt * BN;

  const int nchunks = a.K / KC;
  const int cps = (nchunks + a.splits - 1) / a.splits;
  const int c_begin = ks * cps;
  const int c_end = min(nchunks, c_begin + cps);

  const int row_dw = a.K / 64 * Q4_0_UNIT_DW;
  const uint32_t* wrow[MT];
#pragma unroll
  for (int r = 0; r < MT; r++) wrow[r] = gemm_row_ptr(a, m_wave + 16 * r + li, row_dw);

  f32x4 acc[MT][NT];
#pragma unroll
  for (int r = 0; r < MT; r++)
#pragma unroll
    for (int c = 0; c < NT; c++) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (c_begin < c_end) {
    uint4 xr[2][XR];
    UnitRegs wr[MT][UPC];

    auto load_x = [&](int c) {
      const int k0 = c * KC;
#pragma unroll
      for (int j = 0; j < XR; j++) {
        const int i = threadIdx.x + CN_BLOCK * j;
        const int n = i / (KC / 8), k8 = i % (KC / 8);
        uint4 vh = make_uint4(0u, 0u, 0u, 0u), vl = vh;
        if (i < XV && n0 + n < a.N) {
          const size_t off = (size_t)(n0 + n) * a.K + k0 + 8 * k8;
          vh = *reinterpret_cast<const uint4*>(a.xb + off);
          vl = *reinterpret_cast<const uint4*>(a.xb_lo + off);
        }
        xr[0][j] = vh;
        xr[1][j] = vl;
      }
    };
    auto store_x = [&](int buf) {
#pragma unroll
      for (int j = 0; j < XR; j++) {
        const int i = threadIdx.x + CN_BLOCK * j;
        if (i < XV) {
          const int n = i / (KC / 8), k8 = i % (KC / 8);
          *reinterpret_cast<uint4*>(&xs[buf][0][n * XS + 8 * k8]) = xr[0][j];
          *reinterpret_cast<uint4*>(&xs[buf][1][n * XS + 8 * k8]) = xr[1][j];
        }
      }
    };
    auto load_w = [&](int c) {
#pragma unroll
      for (int r = 0; r < MT; r++)
#pragma unroll
        for (int u = 0; u < UPC; u++)
          load_unit(wrow[r] ? wrow[r] + (size_t)(c * UPC + u) * Q4_0_UNIT_DW : nullptr, h, wr[r][u]);
    };

    load_x(c_begin);
    load_w(c_begin);
    store_x(0);
    __syncthreads();

    for (int c = c_begin; c < c_end; c++) {
      const int buf = (c - c_begin) & 1;
      UnitRegs cur[MT][UPC];
#pragma unroll
      for (int r = 0; r < MT; r++)
#pragma unroll
        for (int u = 0; u < UPC; u++) cur[r][u] = wr[r][u];
      const bool more = c + 1 < c_end;
      if (more) {
        load_x(c + 1);
        load_w(c + 1);
      }
#pragma unroll
      for (int u = 0; u < UPC; u++) {
        bf16x8 fa[MT], fb[MT];
        float da[MT], db[MT];
#pragma unroll
        for (int r = 0; r < MT; r++) exact_unit(cur[r][u], nshift, fa[r], fb[r], da[r], db[r]);
#pragma unroll
        for (int half = 0; half < 2; half++) {
          const int kofs = u * 64 + half * 32 + 8 * g;
#pragma unroll
          for (int cc = 0; cc < NT; cc++) {
            const int xo = (16 * cc + li) * XS + kofs;
            const bf16x8 xh = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&xs[buf][0][xo]));
            const bf16x8 xl = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&xs[buf][1][xo]));
#pragma unroll
            for (int r = 0; r < MT; r++) {
              const bf16x8 wf = half ? fb[r] : fa[r];
              f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wf, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
              p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wf, p, 0, 0, 0);
              const float d = half ? db[r] : da[r];
              acc[r][cc] += d * p;
            }
          }
        }
      }
      if (more) store_x(buf ^ 1);
      __syncthreads();
    }
  }

  // D layout: lane holds x rows 4g..4g+3 of tile column li = W row m.
#pragma unroll
  for (int r = 0; r < MT; r++) {
    const int m = m_wave + 16 * r + li;
#pragma unroll
    for (int cc = 0; cc < NT; cc++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int n = n0 + 16 * cc + 4 * g + i;
        const float v = acc[r][cc][i];
        if (a.splits > 1) {
          if (n < a.N && m < a.M) a.part[((size_t)ks * a.N + n) * a.M + m] = v;
        } else if (a.epi == GEMV_EPI_SWIGLU) {
          const float up = __shfl_xor(v, 1, CN_WAVE);  // row m+1 sits in lane li+1
          if ((m & 1) == 0 && m + 1 < a.M && n < a.N) write_h(a, n, m >> 1, silu_mul(v, up));
        } else if (n < a.N && m < a.M) {
          float* y = a.y + (size_t)n * a.ldy + m;
          *y = (a.epi == GEMV_EPI_ADD) ? *y + v : v;
        }
      }
    }
  }
}

// Sums the K-split partials [splits][N][M] and applies the epilogue; one
// thread per 4 consecutive rows of one column.
__global__ __launch_bounds__(CN_BLOCK) void gemm_reduce_kernel(GemmArgs a) {
  const int m4 = (a.M + 3) / 4;
  const long long t = (long long)blockIdx.x * CN_BLOCK + threadIdx.x;
  if (t >= (long long)m4 * a.N) return;
  const int n = (int)(t / m4), m = (int)(t % m4) * 4;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < a.splits; k++) {
    const float* p = a.part + ((size_t)k * a.N + n) * a.M + m;
    if (m + 3 < a.M && (a.M & 3) == 0) {
      s += *reinterpret_cast<const f32x4*>(p);
    } else {
      for (int i = 0; i < 4 && m + i < a.M; i++) s[i] += p[i];
    }
  }
  write_out4(a, a.epi, n, m, s);
}

// fp32 -> bf16 (round to nearest even), 4 elements per thread.
__global__ __launch_bounds__(CN_BLOCK) void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ xb,
                                                          size_t n) {
  const size_t i = ((size_t)blockIdx.x * CN_BLOCK + threadIdx.x) * 4;
  if (i + 3 < n) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    uint2 o;
    o.x = pack2_bf16(v.x, v.y);
    o.y = pack2_bf16(v.z, v.w);
    *reinterpret_cast<uint2*>(xb + i) = o;
  } else {
    for (size_t j = i; j < n; j++) xb[j] = __builtin_bit_cast(uint16_t, (__bf16)x[j]);
  }
}

// RMSNorm of each row (TensorMath.RmsNorm, TensorMath.cs:97-165) written as
// bf16 for the next GEMM: xb[r] = bf16((x[r] * rms_r) * g).  One workgroup per row.
__global__ __launch_bounds__(CN_BLOCK) void rmsnorm_bf16_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ g, float eps,
                                                               uint16_t* __restrict__ xb,
                                                               uint16_t* __restrict__ xb_lo, int dim) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * dim;
  uint16_t* o = xb + (size_t)blockIdx.x * dim;
  float ss = 0.f;
  for (int i = threadIdx.x * 4; i < dim; i += CN_BLOCK * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = cn_block_sum(ss, red);
  const float rms = 1.0f / sqrtf(ss / (float)dim + eps);
  for (int i = threadIdx.x * 4; i < dim; i += CN_BLOCK * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + i);
    const float4 w = *reinterpret_cast<const float4*>(g + i);
    const float y0 = v.x * rms * w.x, y1 = v.y * rms * w.y, y2 = v.z * rms * w.z, y3 = v.w * rms * w.w;
    if (xb_lo) {
      uint16_t h[4], l[4];
      split_bf16(y0, h[0], l[0]);
      split_bf16(y1, h[1], l[1]);
      split_bf16(y2, h[2], l[2]);
      split_bf16(y3, h[3], l[3]);
      *reinterpret_cast<uint2*>(o + i) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
      *reinterpret_cast<uint2*>(xb_lo + (size_t)blockIdx.x * dim + i) =
          make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    } else {
      *reinterpret_cast<uint2*>(o + i) = make_uint2(pack2_bf16(y0, y1), pack2_bf16(y2, y3));
    }
  }
}

struct GemmShape {
  int mt, nt, kc, splits;
};

GemmShape pick_gemm(int M, int N, int K, int num_cus, bool precise) {
  GemmShape s;
  // Column tile: up to 128 columns so each dequantized W operand feeds NT MFMAs.
  s.nt = N <= 16 ? 1 : (N <= 32 ? 2 : (N <= 64 ? 4 : 8));
  s.mt = (N >= 256 && M >= 128 * num_cus / 2) ? 2 : 1;
  // K chunk staged in LDS per step; the two-plane variant halves it at 128
  // columns to stay within 80 KB of LDS.
  s.kc = (K % 128 == 0 && !(precise && s.nt == 8)) ? 128 : 64;
  const int bm = 64 * s.mt, bn = 16 * s.nt;
  const long long tiles = (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  const int nchunks = K / s.kc;
  s.splits = 1;
  // Split K until the grid covers the chip twice, keeping >= 4 chunks per split.
  while (tiles * s.splits < 2LL * num_cus && nchunks / (s.splits * 2) >= 4 && s.splits < 16) s.splits *= 2;
  return s;
}

template <bool PRECISE, int MT, int NT, int KC>
hipError_t launch_gemm_t(const GemmArgs& a, int grid, hipStream_t st) {
  if constexpr (PRECISE)
    hipLaunchKernelGGL((gemm_q4_0_x2_kernel<MT, NT, KC>), dim3(grid), dim3(CN_BLOCK), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_q4_0_kernel<MT, NT, KC>), dim3(grid), dim3(CN_BLOCK), 0, st, a);
  return hipGetLastError();
}

template <bool PRECISE, int MT, int NT>
hipError_t launch_gemm_kc(const GemmArgs& a, int kc, int grid, hipStream_t st) {
  if constexpr (PRECISE && NT == 8) {
    return launch_gemm_t<PRECISE, MT, NT, 64>(a, grid, st);
  } else {
    if (kc == 128) return launch_gemm_t<PRECISE, MT, NT, 128>(a, grid, st);
    return launch_gemm_t<PRECISE, MT, NT, 64>(a, grid, st);
  }
}

template <bool PRECISE, int MT>
hipError_t launch_gemm_nt(const GemmArgs& a, int nt, int kc, int grid, hipStream_t st) {
  switch (nt) {
    case 1: return launch_gemm_kc<PRECISE, MT, 1>(a, kc, grid, st);
    case 2: return launch_gemm_kc<PRECISE, MT, 2>(a, kc, grid, st);
    case 4: return launch_gemm_kc<PRECISE, MT, 4>(a, kc, grid, st);
    default: return launch_gemm_kc<PRECISE, MT, 8>(a, kc, grid, st);
  }
}

template <bool PRECISE>
hipError_t launch_gemm(const GemmArgs& a, const GemmShape& s, int grid, hipStream_t st) {
  return s.mt == 2 ? launch_gemm_nt<PRECISE, 2>(a, s.nt, s.kc, grid, st)
                   : launch_gemm_nt<PRECISE, 1>(a, s.nt, s.kc, grid, st);
}

}  // namespace

bool gemm_supports(int qtype, int K) { return qtype == 2 && K > 0 && K % 64 == 0; }

size_t gemm_workspace_bytes(int M, int N, int K, int num_cus, bool precise) {
  const GemmShape s = pick_gemm(M, N, K, num_cus, precise);
  return s.splits > 1 ? (size_t)s.splits * N * M * sizeof(float) : 0;
}

hipError_t gemm_launch(const GemmArgs& a_in, int num_cus, hipStream_t st) {
  if (!gemm_supports(a_in.qtype, a_in.K) || a_in.M <= 0 || a_in.N <= 0) return hipErrorInvalidValue;
  const bool precise = a_in.precise != 0;
  if (precise && !a_in.xb_lo) return hipErrorInvalidValue;
  const GemmShape s = pick_gemm(a_in.M, a_in.N, a_in.K, num_cus, precise);
  GemmArgs a = a_in;
  a.splits = s.splits;
  if (s.splits > 1 && !a.part) return hipErrorInvalidValue;
  const int bm = 64 * s.mt, bn = 16 * s.nt;
  const long long grid = (long long)((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn) * s.splits;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipError_t e = precise ? launch_gemm<true>(a, s, (int)grid, st) : launch_gemm<false>(a, s, (int)grid, st);
  if (e != hipSuccess || s.splits == 1) return e;
  const long long work = (long long)((a.M + 3) / 4) * a.N;
  hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((work + CN_BLOCK - 1) / CN_BLOCK)), dim3(CN_BLOCK), 0, st, a);
  return hipGetLastError();
}

hipError_t to_bf16_launch(const float* x, uint16_t* xb, size_t n, hipStream_t st) {
  const size_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((threads + CN_BLOCK - 1) / CN_BLOCK)), dim3(CN_BLOCK), 0, st,
                     x, xb, n);
  return hipGetLastError();
}

hipError_t rmsnorm_bf16_launch(const float* x, const float* g, float eps, uint16_t* xb, uint16_t* xb_lo, int rows,
                               int dim, hipStream_t st) {
  if (dim % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3(rows), dim3(CN_BLOCK), 0, st, x, g, eps, xb, xb_lo, dim);
  return hipGetLastError();
}
