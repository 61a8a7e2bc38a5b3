// gemm.hip — quantized-weight GEMM on the matrix cores of gfx950 (N >= 8).
//
// y[n][m] = sum_k W[m][k] * x[n][k] for a batch of N inputs: the batched form
// of TensorMath.MatVecMulQ4_0 (src/ChatNet.Core/Tensors/TensorMath.cs:548-578)
// that chatnet_matmul with N >= 8 and a multi-token LlamaModel.Forward span
// (LlamaModel.cs:93-238) need.
//
// W is read either as raw Q4_0 blocks or as packed units (gemm_pack_kernel:
// the other block types re-encoded as u8 codes with an fp32 scale and offset
// per 16 weights); x arrives from the producer kernel in the cn_span_pos
// order, either as one fp16 plane scaled per column by a power of two
// (to_f16_scaled_kernel, chatnet_matmul) or, for the exact-weight variant the
// spans run, as fp16 hi + lo planes (conversion, RMSNorm, attention or the
// SwiGLU epilogue).  W bytes and x tiles stream through an LDS ring by direct
// global->LDS loads; each wave dequantizes its W rows into
// v_mfma_f32_32x32x16_f16 operands in registers (one rounded plane, or two
// exact planes) and accumulates in fp32.  When the tile grid leaves the chip
// under-filled the K range is split and gemm_reduce_kernel sums the partial
// tiles and applies the epilogue.  Epilogues: STORE y = acc, ADD y += acc
// (residual), SWIGLU (rows interleave gate/up; h = silu(gate)*up is written
// in the next GEMM's input format).
#include <algorithm>

#include "device_common.h"
#include "kernels.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

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
  // a select, not a[seg]: indexing the argument array would copy it to scratch
  const uint8_t* w = seg == 0 ? a.w[0] : (seg == 1 ? a.w[1] : a.w[2]);
  return reinterpret_cast<const uint32_t*>(w) + (size_t)r * row_dw;
}

// silu(g) * u = g * u / (1 + e^-g) (TensorMath.SiluElementwiseMul,
// TensorMath.cs:253-286) with the hardware exp2 and reciprocal: about 1e-7
// relative, below the resolution of the fp16 hi + lo planes h is stored in
// (the span epilogue runs it for every h element of the tile).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * u * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// h[n][j] = silu(gate) * up as the next span GEMM's input: fp16 hi + lo
// planes in the span order (cn_span_pos).
__device__ __forceinline__ void write_h(const GemmArgs& a, int n, int j, float v) {
  const size_t i = (size_t)n * a.ldh + cn_span_pos(j);
  uint32_t hi, lo;
  cn_split_f16x2(v, 0.f, hi, lo);
  a.hb[i] = (uint16_t)hi;
  a.hb_lo[i] = (uint16_t)lo;
}

// Final write of 4 consecutive rows m..m+3 of column n.
__device__ __forceinline__ void write_out4(const GemmArgs& a, int epi, int n, int m, f32x4 v) {
  if (n >= a.N || m >= a.M) return;
  const bool full = (m + 3 < a.M) && ((a.ldy & 3) == 0);
  if (epi == GEMV_EPI_SWIGLU) {
    // rows (m, m+1) and (m+2, m+3) are (gate, up) pairs of h[m/2], h[m/2+1]
    // (m/2 even: the two stay adjacent in the span order too)
    if (m + 3 < a.M) {
      const float h0 = silu_mul(v[0], v[1]), h1 = silu_mul(v[2], v[3]);
      const size_t i = (size_t)n * a.ldh + cn_span_pos(m >> 1);
      uint32_t hi, lo;
      cn_split_f16x2(h0, h1, hi, lo);
      *reinterpret_cast<uint32_t*>(a.hb + i) = hi;
      *reinterpret_cast<uint32_t*>(a.hb_lo + i) = lo;
    } else {
      write_h(a, n, m >> 1, silu_mul(v[0], v[1]));
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

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Exact-weight (span) kernel, raw Q4_0, fp16 operands.  One MFMA step of a
// lane takes one qs dword of its block; wp holds its bytes in the order
// b0 b2 b1 b3, so that the elements (4s, 4s+1) sit in the low nibbles at bits
// 0-3 / 16-19, (4s+2, 4s+3) at bits 8-11 / 24-27, (16+4s, 16+4s+1) in the
// high nibbles at bits 4-7 / 20-23 and (16+4s+2, 16+4s+3) at 12-15 / 28-31:
// the element order cn_span_pos stores x in.  A pair (q_a, q_b) becomes two
// fp16 halves 0x6400 | q = 1024 + q (or 0x6400 | q << 4 = 1024 + 16q), and a
// packed fp16 add (fma) turns each into q - 8 exactly.  The weight d*(q-8)
// then splits exactly as Wa = (q-8)*dh + Wb = (q-8)*dl, dh = d with its three
// low mantissa bits cleared, dl = d - dh: (q-8) has at most 3 significant
// bits, dh at most 8 and dl at most 3, so both products are fp16 values for
// |d| < 4096 (fp16 subnormals included) and need no rounding.  `magic` holds
// 0x64006400 in a register (v_and_or_b32 takes no two literals).
__device__ __forceinline__ void dequant_q4_f16(uint32_t wp, uint32_t magic, cn_half2 dh, cn_half2 dl, f16x8& wa,
                                               f16x8& wb) {
  const uint32_t u = wp >> 8;
  const cn_half2 t0 = __builtin_bit_cast(cn_half2, (wp & 0x000F000Fu) | magic);
  const cn_half2 t1 = __builtin_bit_cast(cn_half2, (u & 0x000F000Fu) | magic);
  const cn_half2 t2 = __builtin_bit_cast(cn_half2, (wp & 0x00F000F0u) | magic);
  const cn_half2 t3 = __builtin_bit_cast(cn_half2, (u & 0x00F000F0u) | magic);
  const cn_half2 m1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const cn_half2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const cn_half2 m72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const cn_half2 p0 = t0 + m1032, p1 = t1 + m1032;
  const cn_half2 p2 = t2 * s16 + m72, p3 = t3 * s16 + m72;
  const cn_half2 a0 = p0 * dh, a1 = p1 * dh, a2 = p2 * dh, a3 = p3 * dh;
  const cn_half2 b0 = p0 * dl, b1 = p1 * dl, b2 = p2 * dl, b3 = p3 * dl;
  wa = (f16x8){a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  wb = (f16x8){b0[0], b0[1], b1[0], b1[1], b2[0], b2[1], b3[0], b3[1]};
}

// Exact-weight kernel, packed units: the 8 weights of one MFMA step, codes of
// ca with (sc0, of0) then codes of cb with (sc1, of1), as fp16 hi + lo
// (w = fmaf(code, sc, of) carries up to 24 bits; hi + lo keep ~22).
__device__ __forceinline__ void dequant_u8_f16(uint32_t ca, uint32_t cb, float sc0, float of0, float sc1, float of1,
                                               f16x8& wa, f16x8& wb) {
  float w[8];
  w[0] = fmaf(cn_ubyte<0>(ca), sc0, of0);
  w[1] = fmaf(cn_ubyte<1>(ca), sc0, of0);
  w[2] = fmaf(cn_ubyte<2>(ca), sc0, of0);
  w[3] = fmaf(cn_ubyte<3>(ca), sc0, of0);
  w[4] = fmaf(cn_ubyte<0>(cb), sc1, of1);
  w[5] = fmaf(cn_ubyte<1>(cb), sc1, of1);
  w[6] = fmaf(cn_ubyte<2>(cb), sc1, of1);
  w[7] = fmaf(cn_ubyte<3>(cb), sc1, of1);
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int t = 0; t < 4; t++) cn_split_f16x2(w[2 * t], w[2 * t + 1], hi[t], lo[t]);
  wa = __builtin_bit_cast(f16x8, make_uint4(hi[0], hi[1], hi[2], hi[3]));
  wb = __builtin_bit_cast(f16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
}

// One-plane kernel (chatnet_matmul), raw Q4_0: the 8 weights of one MFMA step
// as fp16(d * (q - 8)), one rounding each.  The nibble pairs of wp (bytes b0 b2
// b1 b3 of a qs dword, as dequant_q4_f16 takes them) become q - 8 exactly as
// there, and one packed fp16 multiply by d rounds each product once (|d| <
// 8188 keeps every product finite).
__device__ __forceinline__ f16x8 dequant_q4_h(uint32_t wp, uint32_t magic, cn_half2 d2) {
  const uint32_t u = wp >> 8;
  const cn_half2 t0 = __builtin_bit_cast(cn_half2, (wp & 0x000F000Fu) | magic);
  const cn_half2 t1 = __builtin_bit_cast(cn_half2, (u & 0x000F000Fu) | magic);
  const cn_half2 t2 = __builtin_bit_cast(cn_half2, (wp & 0x00F000F0u) | magic);
  const cn_half2 t3 = __builtin_bit_cast(cn_half2, (u & 0x00F000F0u) | magic);
  const cn_half2 m1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const cn_half2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const cn_half2 m72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const cn_half2 a0 = (t0 + m1032) * d2, a1 = (t1 + m1032) * d2;
  const cn_half2 a2 = (t2 * s16 + m72) * d2, a3 = (t3 * s16 + m72) * d2;
  return (f16x8){a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
}

// One-plane kernel, packed units: the 8 weights of one MFMA step, codes of ca
// with (sc0, of0) then codes of cb with (sc1, of1), each fmaf(code, sc, of) in
// fp32 (the type's value) rounded once to fp16.
__device__ __forceinline__ f16x8 dequant_u8_h(uint32_t ca, uint32_t cb, float sc0, float of0, float sc1, float of1) {
  const cn_float2 w0 = {fmaf(cn_ubyte<0>(ca), sc0, of0), fmaf(cn_ubyte<1>(ca), sc0, of0)};
  const cn_float2 w1 = {fmaf(cn_ubyte<2>(ca), sc0, of0), fmaf(cn_ubyte<3>(ca), sc0, of0)};
  const cn_float2 w2 = {fmaf(cn_ubyte<0>(cb), sc1, of1), fmaf(cn_ubyte<1>(cb), sc1, of1)};
  const cn_float2 w3 = {fmaf(cn_ubyte<2>(cb), sc1, of1), fmaf(cn_ubyte<3>(cb), sc1, of1)};
  const cn_half2 h0 = __builtin_convertvector(w0, cn_half2), h1 = __builtin_convertvector(w1, cn_half2);
  const cn_half2 h2 = __builtin_convertvector(w2, cn_half2), h3 = __builtin_convertvector(w3, cn_half2);
  return (f16x8){h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// ---------------------------------------------------------------------------
// Pipelined 32x32 tile kernels (gemm_p_kernel, gemm_s_kernel): raw W bytes
// and the x tile stream into an LDS ring through direct global->LDS loads
// (global_load_lds_dwordx4, no registers held), so later chunks of 64 K are in
// flight while one is computed; a workgroup waits only for the chunk it needs
// (s_waitcnt vmcnt(n) + a bare s_barrier), not for the whole queue.
//
// Per chunk (one 36-byte Q4_0 unit per W row) lane half h of row li takes
// block h of the unit, and the x fragment of the same lane reads the same 8 k
// of every MFMA step, so the K order inside a chunk is permuted consistently
// for both operands (each kernel's comment gives its order).
// LDS layout per stage: x planes [BN rows][8 x 16 B] with the 16-byte chunk
// of logical index c of row r stored at c ^ ((r >> 1) & 7) (reads of 32 rows
// stay 2-way per bank), then W [128 rows][48 B] holding unit bytes [0,16),
// [16,32) and [20,36) (packed units: [128 rows][96 B]).
// A wave owns 32 W rows x 32*TN columns; the 4 waves stack along M and share
// the x tile.  Output layout of a 32x32 tile: lane l, accumulator v holds row
// 8*(v/4) + 4*(l/32) + v%4, column l%32.
// ---------------------------------------------------------------------------
// 16 bytes from global memory straight into LDS: lane i of the wave writes
// lds_wave_base + 16*i (lds_wave_base must be the same for the whole wave).
// Issued as inline assembly: the compiler treats its own LDS-DMA builtin as
// a write to all of LDS and waits for every load in flight (vmcnt(0)) before
// the next LDS read, which would drain the ring at every chunk; the kernels
// instead wait for the chunk they read with vm_wait and a barrier.  The
// compiler's own waits stay correct with these loads in flight (vector-memory
// counters retire in order, so a wait for one of its loads can only wait
// longer).
__device__ __forceinline__ void lds_dma16(const void* g, void* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t m = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds_wave_base);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m) : "memory");
#endif
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until only the `later` chunks issued after the needed one (at most
// K, VPS vector-memory instructions each) may still be in flight.
template <int VPS, int K>
__device__ __forceinline__ void vm_wait_later(int later) {
  if constexpr (K == 0 || K * VPS > 63) {
    if constexpr (K == 0) vm_wait<0>();
    else vm_wait_later<VPS, K - 1>(later);
  } else {
    if (later >= K) vm_wait<K * VPS>();
    else vm_wait_later<VPS, K - 1>(later);
  }
}

__device__ __forceinline__ void wg_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS reads issued as inline assembly, so that the compiler neither sinks them
// next to their first use nor waits for them itself: a chunk's reads are all
// issued at its start and each step waits (lds_wait) only for the reads it
// consumes.  LDS reads of one wave retire in order.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
// OFF: a constant byte offset carried in the instruction's offset field (no
// address arithmetic for it).
template <int OFF = 0>
__device__ __forceinline__ cn_u32x4 lds_read128(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  cn_u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint2 lds_read64(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  uint2 v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint32_t lds_read32(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
// The x fragments of one MFMA step for column tiles CC .. TN-1: tile cc lies
// 32 x-rows (4096 bytes) after tile cc-1, at the same swizzled chunk.
template <int CC, int TN>
__device__ __forceinline__ void lds_read_xtiles(uint32_t base, cn_u32x4 (&xr)[TN]) {
  if constexpr (CC < TN) {
    xr[CC] = lds_read128<CC * 4096>(base);
    lds_read_xtiles<CC + 1, TN>(base, xr);
  }
}
// Waits until at most N of this wave's LDS reads are outstanding.  A value
// read by lds_read* must pass through reg_fence after the wait that covers it,
// so that its uses stay behind that wait.
template <int N>
__device__ __forceinline__ void lds_wait() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}
template <class T>
__device__ __forceinline__ void reg_fence(T& r) {
  asm volatile("" : "+v"(r));
}

// MT: 32-row tiles per wave, TN: 32-column tiles per wave; each x fragment
// read from LDS feeds MT MFMAs, each dequantized W fragment TN.  WNC: waves
// along N (1: the four waves stack along M, BM = 128 * MT; 2: a 2 x 2 grid of
// waves, BM = 64 * MT, BN = 64 * TN, each wave reading half the x tile).
// WF: how W is stored (GemmArgs::packed): GEMM_W_Q4_0 raw blocks,
// GEMM_W_PACKED units, GEMM_W_F16 / GEMM_W_F32 rows of the float type (their
// 16-byte pieces XOR-swizzled in LDS as the x rows are), GEMM_W_Q4_K raw
// super-blocks (per chunk of 64: the 16-byte header, then the 32 qs bytes of
// the chunk's two sub-blocks).
template <bool PRECISE, int TN, int S, int WF, int MT = 1, int WNC = 1>
struct PipeCfg {
  static constexpr int PL = PRECISE ? 2 : 1;
  static constexpr int MTILES = MT;
  static constexpr int WN = WNC, WM = 4 / WNC;  // waves along N and M
  static constexpr int BM = 32 * WM * MT, BN = 32 * TN * WN;
  static constexpr bool PK = WF == GEMM_W_PACKED;
  static constexpr bool FLT = WF == GEMM_W_F16 || WF == GEMM_W_F32;
  static constexpr bool Q4K = WF == GEMM_W_Q4_K;
  // global bytes per row and chunk of 64
  static constexpr int UNIT = WF == GEMM_W_F32 ? 256 : (WF == GEMM_W_F16 ? 128 : (PK ? kGemmPackUnit : 36));
  static constexpr int WP = FLT ? UNIT / 16 : (PK ? 6 : 3);  // 16-byte pieces per row and chunk
  static constexpr int WROW = 16 * WP;         // LDS bytes per row and chunk
  static constexpr int XB = BN * 128;          // bytes per x plane per stage
  static constexpr int WB = BM * WROW;         // bytes of W per stage
  static constexpr int STAGE = PL * XB + WB;
  static constexpr int LDS = S * STAGE;        // the ring
  static constexpr int XPW = BN * 8 / 4;       // x pieces (16 B) per wave per plane
  static constexpr int XI = XPW / 64;
  static constexpr int WPW = BM * WP / 4;      // W pieces per wave
  static constexpr int WI = (WPW + 63) / 64;
  static constexpr int VPS = PL * XI + WI;     // vector-memory instructions per stage per wave
  static constexpr int WD = FLT ? UNIT / 8 : (PK ? 12 : (Q4K ? 8 : 5));  // W dwords a lane reads per chunk
  static constexpr bool PACKED = PK;
  static constexpr int TNW = TN;                // column tiles per wave
  static_assert(XPW % 64 == 0, "x pieces per wave must fill whole instructions");
};

// Tile coordinates, K range and stage loads of one workgroup (both kernels).
template <class C>
struct TileIO {
  int lane, wave, wm, wn, h, li, ks, m0, n0, c_begin, c_end;
  const uint16_t* xsrc[C::PL][C::XI];
  const char* wsrc[C::WI];
  int wstep[C::WI];  // Q4_K: bytes the piece moves per chunk within a super-block
  bool wact[C::WI];

  // The tile and K range of blockIdx.x (tile-major, K split innermost); a
  // stream-K launch (a.sk_wgs > 0) sets each of its segments with set_tile.
  __device__ __forceinline__ explicit TileIO(const GemmArgs& a) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave % C::WM;
    wn = wave / C::WM;
    h = lane >> 5;
    li = lane & 31;
    ks = 0;
    if (a.sk_wgs > 0) return;  // stream-K launches do not split K (a.splits == 1)
    int bid = blockIdx.x;
    ks = bid % a.splits;
    bid /= a.splits;
    const int nchunks = a.K / 64;
    const int cps = (nchunks + a.splits - 1) / a.splits;
    set_tile(a, bid, ks * cps, min(nchunks, ks * cps + cps));
  }

  // Tile `tile` (row tile tile / n_nt, column tile tile % n_nt), chunks [cb, ce).
  __device__ __forceinline__ void set_tile(const GemmArgs& a, int tile, int cb, int ce) {
    const int n_nt = (a.N + C::BN - 1) / C::BN;
    m0 = (tile / n_nt) * C::BM;
    n0 = (tile % n_nt) * C::BN;
    c_begin = cb;
    c_end = ce;
    const int row_dw = a.K / 64 * (C::UNIT / 4);
#pragma unroll
    for (int p = 0; p < C::PL; p++)
#pragma unroll
      for (int j = 0; j < C::XI; j++) {
        const int piece = wave * C::XPW + 64 * j + lane;
        const int row = piece >> 3, ch = piece & 7;
        const int n = min(n0 + row, a.N - 1);
        const int logical = ch ^ ((row >> 1) & 7);
        xsrc[p][j] = (p ? a.xb_lo : a.xb) + (size_t)n * a.K + 8 * logical;
      }
#pragma unroll
    for (int j = 0; j < C::WI; j++) {
      const int q = 64 * j + lane;
      wact[j] = q < C::WPW;
      const int piece = wave * C::WPW + (wact[j] ? q : 0);
      const int row = piece / C::WP, part = piece % C::WP;
      const int vr = min(m0 + row, a.M - 1);
      // Q4_0: pieces at unit bytes 0, 16 and 20, exactly the 36 bytes, no read
      // past the unit; packed: the 6 pieces of the 96-byte unit; float rows:
      // LDS slot `part` holds the row's piece part ^ ((row >> 1) & 7)
      const int off = C::FLT ? 16 * (part ^ ((row >> 1) & 7)) : (!C::PACKED && !C::Q4K && part == 2 ? 20 : 16 * part);
      wsrc[j] = reinterpret_cast<const char*>(gemm_row_ptr(a, vr, row_dw)) + off;
      wstep[j] = part ? 32 : 0;  // Q4_K: the header stays, the qs window moves
    }
  }

  // Chunk c's x planes and W rows into stage `st` (C::VPS vector-memory
  // instructions per wave).
  __device__ __forceinline__ void issue(int c, char* st) const {
#pragma unroll
    for (int p = 0; p < C::PL; p++)
#pragma unroll
      for (int j = 0; j < C::XI; j++)
        lds_dma16(xsrc[p][j] + c * 64, st + p * C::XB + (wave * C::XPW + 64 * j) * 16);
#pragma unroll
    for (int j = 0; j < C::WI; j++) {
      // Q4_K: super-block c / 4 (144 bytes), qs of its sub-blocks 2(c%4), 2(c%4)+1
      const char* src = C::Q4K ? wsrc[j] + (size_t)(c >> 2) * 144 + (c & 3) * wstep[j] : wsrc[j] + c * C::UNIT;
      if (wact[j]) lds_dma16(src, st + C::PL * C::XB + (wave * C::WPW + 64 * j) * 16);
    }
    asm volatile("" ::: "memory");
  }

  // The dwords of the lane's W slice in stage `st`.  Q4_0 (5 dwords): the
  // stage holds unit bytes [0,16) [16,32) [20,36): block A's d + qs at dwords
  // 0..4, block B's d in the high half of dword 4 and its qs at dwords
  // 8..11.  Packed (12 dwords): codes 32h..32h+31 (dwords 8h..8h+7), then
  // scales 2h, 2h+1 (unit bytes 64 + 8h) and offsets 2h, 2h+1 (80 + 8h).
  __device__ __forceinline__ void wraw(const char* st, uint32_t (&w)[C::WD], int mt = 0) const {
    const uint32_t* wb =
        reinterpret_cast<const uint32_t*>(st + C::PL * C::XB + (wm * 32 * C::MTILES + 32 * mt + li) * C::WROW);
    if constexpr (C::Q4K) {
      // the header (d | dmin, 12 scale bytes), then the qs of sub-block h of the chunk
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = wb[i];
#pragma unroll
      for (int i = 0; i < 4; i++) w[4 + i] = wb[4 + 4 * h + i];
    } else if constexpr (C::FLT) {
      // the lane's block h: logical pieces P*h .. P*h+P-1 of the row (P = 4
      // for F16, 8 for F32), each in its swizzled slot
      constexpr int P = C::WP / 2;
      const int sw = (li >> 1) & 7;
#pragma unroll
      for (int q = 0; q < P; q++) {
        const uint32_t* pc = wb + 4 * ((P * h + q) ^ sw);
#pragma unroll
        for (int i = 0; i < 4; i++) w[4 * q + i] = pc[i];
      }
    } else if constexpr (C::PACKED) {
#pragma unroll
      for (int i = 0; i < 8; i++) w[i] = wb[8 * h + i];
      w[8] = wb[16 + 2 * h];
      w[9] = wb[17 + 2 * h];
      w[10] = wb[20 + 2 * h];
      w[11] = wb[21 + 2 * h];
    } else {
      w[0] = wb[8 * h];
      w[1] = wb[8 * h + 1];
      w[2] = wb[8 * h + 2];
      w[3] = wb[8 * h + 3];
      w[4] = wb[4];
    }
  }

  // Where the 16-byte x fragment of MFMA step s, column tile cc, plane p lies.
  __device__ __forceinline__ const char* xfrag_ptr(const char* st, int p, int s, int cc) const {
    const int xrow = wn * 32 * C::TNW + 32 * cc + li;
    const int phys = (4 * h + s) ^ ((xrow >> 1) & 7);
    return st + p * C::XB + xrow * 128 + phys * 16;
  }

  // The 16-byte x fragment of MFMA step s, column tile cc, plane p.
  __device__ __forceinline__ uint4 xfrag(const char* st, int p, int s, int cc) const {
    const int xrow = wn * 32 * C::TNW + 32 * cc + li;
    const int phys = (4 * h + s) ^ ((xrow >> 1) & 7);
    return *reinterpret_cast<const uint4*>(st + p * C::XB + xrow * 128 + phys * 16);
  }

  // The output scale of each of the lane's columns: the one-plane kernel's x
  // of column n was scaled by 1 / xinv[n] (a power of two); 1 otherwise.
  // Loaded at the kernel's start, so the epilogue does not wait for it.
  template <int TN>
  __device__ __forceinline__ void load_scales(const GemmArgs& a, float (&sc)[TN]) const {
#pragma unroll
    for (int cc = 0; cc < TN; cc++) {
      const int n = n0 + wn * 32 * C::TNW + 32 * cc + li;
      sc[cc] = a.xinv ? a.xinv[n < a.N ? n : a.N - 1] : 1.0f;
    }
  }

  // Final tiles: K-split partials [splits][N][M] or the epilogue.
  template <int TN>
  __device__ __forceinline__ void store(const GemmArgs& a, const f32x16 (&acc)[TN], const float (&scl)[TN],
                                        int mt = 0) const {
#pragma unroll
    for (int cc = 0; cc < TN; cc++) {
      const int n = n0 + wn * 32 * C::TNW + 32 * cc + li;
      const float sc = scl[cc];
#pragma unroll
      for (int v4 = 0; v4 < 4; v4++) {
        const int m = m0 + wm * 32 * C::MTILES + 32 * mt + 8 * v4 + 4 * h;
        const f32x4 v = f32x4{acc[cc][4 * v4], acc[cc][4 * v4 + 1], acc[cc][4 * v4 + 2], acc[cc][4 * v4 + 3]} * sc;
        if (a.splits > 1) {
          if (n < a.N && m < a.M) {
            float* p = a.part + ((size_t)ks * a.N + n) * a.M + m;
            if (m + 3 < a.M && (a.M & 3) == 0) *reinterpret_cast<f32x4*>(p) = v;
            else
              for (int i = 0; i < 4 && m + i < a.M; i++) p[i] = v[i];
          }
        } else {
          write_out4(a, a.epi, n, m, v);
        }
      }
    }
  }
};

// One-plane kernel (chatnet_matmul): x as one fp16 plane in the cn_span_pos
// order, each column scaled by a power of two (to_f16_scaled_launch) that
// store() undoes.  The ring and the step order are the span kernel's (below):
// at the start of chunk c every wave has landed its part of the chunk and
// finished chunk c-1, chunk c+S-1 is issued into the freed stage, and each
// step's 8 weights are dequantized into one fp16 operand just ahead of its
// TN MFMAs (one v_mfma_f32_32x32x16_f16 per column tile).  Step s of lane
// half h: Q4_0 qs dword s of block h; packed codes 32h + 4s .. +3 and
// 32h + 16 + 4s .. +3 with the scale/offset pairs 2h and 2h+1.
template <int TN, int S, bool PK, int MT, int WNC, bool SK>
__global__ __launch_bounds__(CN_BLOCK) __attribute__((amdgpu_waves_per_eu(SK ? 2 : 1, 2))) void gemm_p_kernel(GemmArgs a) {
  using C = PipeCfg<false, TN, S, PK, MT, WNC>;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ int sk_last;
  TileIO<C> io(a);
  const int h = io.h;
  const uint32_t psel = h ? 0x03010200u : 0x05030402u;
  uint32_t magic = 0x64006400u;
  asm volatile("" : "+v"(magic));

  // Stream-K (SK): the launch's tiles x chunks of 64 as one sequence
  // (tile-major).  Workgroups 0 .. D-1 take tiles 0 .. D-1 whole; the other
  // G2 share the remaining tiles' chunks in equal ranges, each covering the
  // end of one tile and the start of the next at most.  Otherwise one
  // segment: the tile and K range of blockIdx.x.
  const int nc = a.K / 64;
  const long long units = (long long)a.sk_tiles * nc;
  constexpr bool sk = SK;
  const int D = a.sk_dp, G2 = a.sk_wgs - a.sk_dp;
  const long long u0 = (long long)D * nc, units2 = units - u0;
  auto lo_of = [&](int g) -> long long { return g < D ? (long long)g * nc : u0 + units2 * (g - D) / G2; };
  long long u = sk ? lo_of(blockIdx.x) : 0;
  const long long u_end = sk ? lo_of(blockIdx.x + 1) : 1;
  for (bool first = true; u < u_end; first = false) {
    int tile = 0;
    if constexpr (sk) {
      tile = (int)(u / nc);
      const int cb = (int)(u % nc);
      const int ce = (int)min((long long)nc, cb + (u_end - u));
      io.set_tile(a, tile, cb, ce);
      u += ce - cb;
      if (!first) __syncthreads();  // every wave is done with the previous segment's ring
    } else {
      u = u_end;
    }
    float xsc[TN];
    io.template load_scales<TN>(a, xsc);

    f32x16 acc[MT][TN];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int cc = 0; cc < TN; cc++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[mt][cc][v] = 0.f;

    const int c_begin = io.c_begin, c_end = io.c_end;
    if (c_begin < c_end) {
      auto slot_of = [&](int c) { return lds + ((c - c_begin) % S) * C::STAGE; };
#pragma unroll
      for (int i = 0; i < S - 1; i++)
        if (c_begin + i < c_end) io.issue(c_begin + i, lds + i * C::STAGE);
      for (int c = c_begin; c < c_end; c++) {
        char* st = slot_of(c);
        // chunks c+1 .. c+S-2 may stay in flight
        vm_wait_later<C::VPS, S - 2>(min(S - 2, c_end - 1 - c));
        wg_barrier();
        if (c + S - 1 < c_end) io.issue(c + S - 1, slot_of(c + S - 1));
        // the lane's W dwords (as wraw), then every x fragment of the chunk, all
        // issued at once; step s waits for its own fragments only
        uint32_t w[MT][C::WD];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          // the W rows follow the x planes in the stage (offset WO)
          constexpr int WO = C::PL * C::XB;
          const uint32_t wb = lds_addr(st + (io.wm * 32 * MT + 32 * mt + io.li) * C::WROW);
          if constexpr (PK) {
            const uint32_t wc = wb + 32 * h, ws = wb + 8 * h;
            const cn_u32x4 c0 = lds_read128<WO>(wc), c1 = lds_read128<WO + 16>(wc);
            const uint2 sc = lds_read64<WO + 64>(ws), of = lds_read64<WO + 80>(ws);
            w[mt][0] = c0[0], w[mt][1] = c0[1], w[mt][2] = c0[2], w[mt][3] = c0[3];
            w[mt][4] = c1[0], w[mt][5] = c1[1], w[mt][6] = c1[2], w[mt][7] = c1[3];
            w[mt][8] = sc.x, w[mt][9] = sc.y, w[mt][10] = of.x, w[mt][11] = of.y;
          } else {
            const cn_u32x4 q = lds_read128<WO>(wb + 32 * h);
            const uint32_t t = lds_read32<WO + 16>(wb);
            w[mt][0] = q[0], w[mt][1] = q[1], w[mt][2] = q[2], w[mt][3] = q[3], w[mt][4] = t;
          }
        }
        cn_u32x4 xr[4][TN];
#pragma unroll
        for (int s = 0; s < 4; s++) lds_read_xtiles<0, TN>(lds_addr(io.xfrag_ptr(st, 0, s, 0)), xr[s]);
        // Step s's W operands are dequantized during step s-1 (step 0's before
        // the first MFMA) and interleaved with its MFMAs: one wave issues in
        // order, so VALU work placed after a run of MFMAs waits behind them
        // while the matrix pipe drains; between them it runs in their shadow.
        auto dequant = [&](int s, int mt) -> f16x8 {
          if constexpr (PK) {
            return dequant_u8_h(w[mt][s], w[mt][4 + s], __uint_as_float(w[mt][8]), __uint_as_float(w[mt][10]),
                                __uint_as_float(w[mt][9]), __uint_as_float(w[mt][11]));
          } else {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(h ? (w[mt][4] >> 16) : (w[mt][0] & 0xFFFFu)));
            return dequant_q4_h(__builtin_amdgcn_perm(w[mt][s + 1], w[mt][s], psel), magic, (cn_half2){d, d});
          }
        };
        // the W dwords and step 0's fragments: reads issued after them are
        // those of steps 1 .. 3
        lds_wait<(3 * TN > 15 ? 15 : 3 * TN)>();
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int i = 0; i < C::WD; i++) reg_fence(w[mt][i]);
        f16x8 wa[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) wa[mt] = dequant(0, mt);
#pragma unroll
        for (int s = 0; s < 4; s++) {
          if (s == 1) lds_wait<2 * TN>();
          else if (s == 2) lds_wait<TN>();
          else if (s == 3) lds_wait<0>();
#pragma unroll
          for (int cc = 0; cc < TN; cc++) reg_fence(xr[s][cc]);
          f16x8 xh[TN];
#pragma unroll
          for (int cc = 0; cc < TN; cc++) xh[cc] = __builtin_bit_cast(f16x8, xr[s][cc]);
          f16x8 wn[MT];
#pragma unroll
          for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int cc = 0; cc < TN; cc++) acc[mt][cc] = mma32(wa[mt], xh[cc], acc[mt][cc]);
          }
          if (s < 3) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) wn[mt] = dequant(s + 1, mt);
            // one MFMA, then a share of the next step's dequantization, ...
            constexpr int kDequantValu = PK ? 24 : 14;  // VALU instructions per dequantized operand
            constexpr int kPer = (kDequantValu * MT + MT * TN - 1) / (MT * TN);
#pragma unroll
            for (int i = 0; i < MT * TN; i++) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, kPer, 0);
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) wa[mt] = wn[mt];
          }
          __builtin_amdgcn_sched_barrier(0);  // the next step's wait stays behind these MFMAs
        }
      }
    }
    if (!sk || (io.c_begin == 0 && io.c_end == nc)) {
#pragma unroll
      for (int mt = 0; mt < MT; mt++) io.template store<TN>(a, acc[mt], xsc, mt);
      continue;
    }
    // A tile shared by the workgroups gf .. gl (K order).  Each writes its
    // scaled part to a slot of its own (2g for its range's first segment,
    // 2g + 1 for its last; float j of thread t at j * CN_BLOCK + t) with
    // device-scope stores, waits for them, then arrives on the tile's counter.
    // The last to arrive reads the parts back with device-scope loads (its
    // own too, so that no accumulator stays live), sums them in K order as
    // the K-split reduce does (((0 + p_gf) + ...) + p_gl, whatever the
    // arrival order), applies the epilogue and sets the counter back to zero
    // for the next launch.  Device-scope accesses go past the XCD's L2 copy
    // without the L2-wide writeback and invalidation of a device fence (which
    // would empty the L2 under every other workgroup of the XCD).  No
    // workgroup waits for another.
    if constexpr (SK) {
      constexpr int NF = MT * TN * 16;  // floats per thread
      auto wg_of = [&](long long unit) {  // the workgroup whose range holds chunk `unit`
        return unit < u0 ? (int)(unit / nc) : D + (int)(((unit - u0 + 1) * G2 - 1) / units2);
      };
      auto slot = [&](int g) {
        const bool first_seg = lo_of(g) >= (long long)tile * nc;
        return a.part + (size_t)(2 * g + (first_seg ? 0 : 1)) * NF * CN_BLOCK + threadIdx.x;
      };
      const int gf = wg_of((long long)tile * nc), gl = wg_of((long long)tile * nc + nc - 1);
      float* mine = slot(blockIdx.x);
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int cc = 0; cc < TN; cc++)
#pragma unroll
          for (int v = 0; v < 16; v++)
            __hip_atomic_store(mine + ((mt * TN + cc) * 16 + v) * CN_BLOCK, acc[mt][cc][v] * xsc[cc], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the part has reached device scope
      __syncthreads();
      if (threadIdx.x == 0) {
        const unsigned arrived = __hip_atomic_fetch_add(a.tile_cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sk_last = arrived == (unsigned)(gl - gf);
        if (sk_last) __hip_atomic_store(a.tile_cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (sk_last) {
        // B contributors' parts per batch, every load of a batch in flight
        // together (one device-scope round trip per batch), added in K order
        constexpr int B = NF >= 64 ? 1 : 64 / NF;
        float sum[NF];
#pragma unroll
        for (int j = 0; j < NF; j++) sum[j] = 0.f;
        for (int g0 = gf; g0 <= gl; g0 += B) {
          float v[B][NF];
#pragma unroll
          for (int b = 0; b < B; b++) {
            const float* p = slot(min(g0 + b, gl));
#pragma unroll
            for (int j = 0; j < NF; j++) v[b][j] = __hip_atomic_load(p + j * CN_BLOCK, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
#pragma unroll
          for (int b = 0; b < B; b++)
            if (g0 + b <= gl)
#pragma unroll
              for (int j = 0; j < NF; j++) sum[j] += v[b][j];
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int cc = 0; cc < TN; cc++)
#pragma unroll
            for (int v4 = 0; v4 < 4; v4++) {
              const int j = (mt * TN + cc) * 16 + 4 * v4;
              write_out4(a, a.epi, io.n0 + io.wn * 32 * TN + 32 * cc + io.li,
                         io.m0 + io.wm * 32 * MT + 32 * mt + 8 * v4 + 4 * h,
                         f32x4{sum[j], sum[j + 1], sum[j + 2], sum[j + 3]});
            }
      }
    }
  }
}

// Span kernel (the exact-weight product of the forward pass's spans: fp16 x
// hi + lo planes in the cn_span_pos order).  An S-stage ring (S = 2 or 3): at
// the start of chunk c every wave has landed its part of the chunk and finished
// chunk c-1, chunk c+S-1 is issued into the freed stage, and chunk c's W is
// dequantized step by step just ahead of its MFMAs.  Two stages take 44 KB of
// LDS (raw Q4_0, 64 columns), so three workgroups share a CU and one's VALU
// work and waits overlap the others' MFMAs; three stages keep two chunks in
// flight for grids of at most two workgroups per CU.  Step s of lane half h:
// Q4_0 qs dword s of block h (dequant_q4_f16), packed codes 32h + 4s .. +3
// and 32h + 16 + 4s .. +3 with the scale/offset pairs 2h and 2h+1.  Three
// fp16 MFMAs per step: Wa*xh + Wa*xl + Wb*xh, W = Wa + Wb exact for Q4_0 (~22
// bits for packed units), x = xh + xl to ~2^-22; the dropped Wb*xl term is
// below 2^-19 relative.
template <int TN, int S, int WF>
__global__ __launch_bounds__(CN_BLOCK) void gemm_s_kernel(GemmArgs a) {
  using C = PipeCfg<true, TN, S, WF>;
  constexpr bool PK = C::PK;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const TileIO<C> io(a);
  const int h = io.h;

  f32x16 acc[TN];
#pragma unroll
  for (int cc = 0; cc < TN; cc++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[cc][v] = 0.f;

  // v_perm_b32 selectors: qs dword s of the lane's block (2 bytes into the
  // unit for block A) as bytes b0 b2 b1 b3; 0x64006400 kept in a register
  // so each nibble pair takes one v_and_or_b32
  const uint32_t psel = h ? 0x03010200u : 0x05030402u;
  uint32_t magic = 0x64006400u;
  asm volatile("" : "+v"(magic));

  const int c_begin = io.c_begin, c_end = io.c_end;
  if (c_begin < c_end) {
    auto slot_of = [&](int c) { return lds + ((c - c_begin) % S) * C::STAGE; };
#pragma unroll
    for (int i = 0; i < S - 1; i++)
      if (c_begin + i < c_end) io.issue(c_begin + i, lds + i * C::STAGE);
    for (int c = c_begin; c < c_end; c++) {
      char* st = slot_of(c);
      // this wave's part of chunk c (chunk c+1 may stay in flight with three stages)
      if (S >= 3 && c + 1 < c_end) vm_wait<C::VPS>();
      else vm_wait<0>();
      wg_barrier();  // every wave's part landed, every wave done with chunk c-1
      if (c + S - 1 < c_end) io.issue(c + S - 1, slot_of(c + S - 1));
      uint32_t w[C::WD];
      io.wraw(st, w);
      cn_half2 dh2 = {}, dl2 = {};
      float ksc = 0.f, kof = 0.f;
      if constexpr (C::Q4K) {
        // sub-block sb of the super-block (DequantQ4K.DecodeScales,
        // DequantQ4K.cs:218-264): its weights are d*sc*q - dmin*m, and both
        // products are exact in fp32 (11 x 6 bits)
        const int sb = 2 * (c & 3) + h;
        auto qb = [&](int i) { return (w[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFFu; };
        uint32_t sc, mm;
        if (sb < 4) {
          sc = qb(sb) & 63u;
          mm = qb(sb + 4) & 63u;
        } else {
          sc = (qb(sb + 4) & 0xFu) | ((qb(sb - 4) >> 6) << 4);
          mm = (qb(sb + 4) >> 4) | ((qb(sb) >> 6) << 4);
        }
        ksc = cn_h2f(w[0]) * (float)sc;
        kof = -(cn_h2f(w[0] >> 16) * (float)mm);
      }
      if constexpr (WF == GEMM_W_Q4_0) {
        // d = dh + dl: dh keeps the top 8 significant bits of the fp16 scale
        const uint32_t d16 = h ? (w[4] >> 16) : (w[0] & 0xFFFFu);
        const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)d16);
        const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(d16 & 0xFFF8u));
        const _Float16 dl = d - dh;
        dh2 = (cn_half2){dh, dh};
        dl2 = (cn_half2){dl, dl};
      }
      f16x8 xh[2][TN], xl[2][TN];
      auto load_x = [&](int s, int b) {
#pragma unroll
        for (int cc = 0; cc < TN; cc++) {
          xh[b][cc] = __builtin_bit_cast(f16x8, io.xfrag(st, 0, s, cc));
          xl[b][cc] = __builtin_bit_cast(f16x8, io.xfrag(st, 1, s, cc));
        }
      };
      load_x(0, 0);
#pragma unroll
      for (int s = 0; s < 4; s++) {
        if (s < 3) load_x(s + 1, (s + 1) & 1);
        f16x8 wa, wb;
        if constexpr (WF == GEMM_W_F16) {
          // elements 4s..4s+3 and 16+4s..16+4s+3 of the lane's block, already
          // fp16: W * (xh + xl), exact products
          wa = __builtin_bit_cast(f16x8, (cn_u32x4){w[2 * s], w[2 * s + 1], w[8 + 2 * s], w[9 + 2 * s]});
        } else if constexpr (WF == GEMM_W_F32) {
          // the same elements as fp32, split as W = Wa + Wb in fp16 (one
          // rounding each, ~22 bits together)
          uint32_t hi[4], lo[4];
#pragma unroll
          for (int k = 0; k < 2; k++) {
            cn_split_f16x2(__uint_as_float(w[4 * s + 2 * k]), __uint_as_float(w[4 * s + 2 * k + 1]), hi[k], lo[k]);
            cn_split_f16x2(__uint_as_float(w[16 + 4 * s + 2 * k]), __uint_as_float(w[16 + 4 * s + 2 * k + 1]),
                           hi[2 + k], lo[2 + k]);
          }
          wa = __builtin_bit_cast(f16x8, (cn_u32x4){hi[0], hi[1], hi[2], hi[3]});
          wb = __builtin_bit_cast(f16x8, (cn_u32x4){lo[0], lo[1], lo[2], lo[3]});
        } else if constexpr (C::Q4K) {
          // qs dword s of the sub-block: low nibbles are elements 4s..4s+3,
          // high nibbles 16+4s..16+4s+3 (DequantQ4K.cs:59-72), the order x is stored in
          const uint32_t q = w[4 + s];
          dequant_u8_f16(q & 0x0F0F0F0Fu, (q >> 4) & 0x0F0F0F0Fu, ksc, kof, ksc, kof, wa, wb);
        } else if constexpr (PK) {
          dequant_u8_f16(w[s], w[4 + s], __uint_as_float(w[8]), __uint_as_float(w[10]), __uint_as_float(w[9]),
                         __uint_as_float(w[11]), wa, wb);
        } else {
          dequant_q4_f16(__builtin_amdgcn_perm(w[s + 1], w[s], psel), magic, dh2, dl2, wa, wb);
        }
#pragma unroll
        for (int cc = 0; cc < TN; cc++) acc[cc] = mma32(wa, xh[s & 1][cc], acc[cc]);
#pragma unroll
        for (int cc = 0; cc < TN; cc++) acc[cc] = mma32(wa, xl[s & 1][cc], acc[cc]);
        if constexpr (WF != GEMM_W_F16) {
#pragma unroll
          for (int cc = 0; cc < TN; cc++) acc[cc] = mma32(wb, xh[s & 1][cc], acc[cc]);
        }
      }
    }
  }
  float sc[TN];
  io.template load_scales<TN>(a, sc);
  io.template store<TN>(a, acc, sc);
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

// x [N][K] fp32 -> the one-plane kernel's input: per column n a power of two
// 2^e_n that brings max|x[n]| into [2^14, 2^15) (so every element stays
// inside fp16's range and as far above its subnormals as the column allows;
// e_n in [-125, 125]; 0 for a column that is all zero or holds an infinity),
// xh[n][cn_span_pos(k)] = fp16(x[n][k] * 2^e_n) (the scaling is exact, one
// rounding to nearest even) and xinv[n] = 2^-e_n.  One workgroup per column,
// the column held in registers between the max and the conversion.
template <int V>
__global__ __launch_bounds__(CN_BLOCK) void to_f16_scaled_kernel(const float* __restrict__ x,
                                                                uint16_t* __restrict__ xh,
                                                                float* __restrict__ xinv, int K) {
  __shared__ float red[4];
  const size_t n = blockIdx.x;
  const float* xr = x + n * K;
  f32x4 v[V];
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int i = (threadIdx.x + CN_BLOCK * j) * 4;
    v[j] = i < K ? *reinterpret_cast<const f32x4*>(xr + i) : f32x4{0.f, 0.f, 0.f, 0.f};
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j][0]), fabsf(v[j][1])), fmaxf(fabsf(v[j][2]), fabsf(v[j][3]))));
  }
  mx = cn_block_max(mx, red);
  int e = 0;
  if (mx > 0.f && mx <= 3.402823466e38f) {
    int E;
    (void)frexpf(mx, &E);  // mx = f * 2^E, f in [0.5, 1)
    e = min(125, max(-125, 15 - E));
  }
  if (threadIdx.x == 0) xinv[n] = ldexpf(1.0f, -e);
  const float sc = ldexpf(1.0f, e);
  uint16_t* o = xh + n * K;
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int i = (threadIdx.x + CN_BLOCK * j) * 4;
    if (i >= K) continue;
    const f32x4 y = v[j] * sc;  // 2^e is a normal float for e in [-125, 125]
    const cn_half2 a = __builtin_convertvector((cn_float2){y[0], y[1]}, cn_half2);
    const cn_half2 b = __builtin_convertvector((cn_float2){y[2], y[3]}, cn_half2);
    *reinterpret_cast<uint2*>(o + cn_span_pos(i)) =
        make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
  }
}

// RMSNorm of each row (TensorMath.RmsNorm, TensorMath.cs:97-165) written as
// the next span GEMM's input: (x[r] * rms_r) * g as fp16 hi + lo planes
// (xb, xb_lo) in the cn_span_pos order.  One workgroup per row, the row held in registers between the sum of
// squares and the scaling (one pass over memory).  With `part` (splits > 0)
// the row is first completed as a residual add of the preceding GEMM's K-split
// partials [splits][rows][dim], summed in split order exactly as
// gemm_reduce_kernel does (x += ((0 + p0) + p1) + ...), and written back to x.
template <int V, int SPL>
__global__ __launch_bounds__(CN_BLOCK) void add_rmsnorm_span_kernel(float* __restrict__ x,
                                                                   const float* __restrict__ part, int splits,
                                                                   const float* __restrict__ g, float eps,
                                                                   uint16_t* __restrict__ xb,
                                                                   uint16_t* __restrict__ xb_lo, int rows, int dim) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  float* xr = x + row * dim;
  f32x4 v[V];
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int i = (threadIdx.x + CN_BLOCK * j) * 4;
    v[j] = i < dim ? *reinterpret_cast<const f32x4*>(xr + i) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (SPL > 0) {
    // every partial's loads issued before the first add (SPL >= splits;
    // slots past splits are not read)
    f32x4 pv[SPL][V];
#pragma unroll
    for (int k = 0; k < SPL; k++) {
      const float* pr = part + ((size_t)(k < splits ? k : 0) * rows + row) * dim;
#pragma unroll
      for (int j = 0; j < V; j++) {
        const int i = (threadIdx.x + CN_BLOCK * j) * 4;
        pv[k][j] = (i < dim && k < splits) ? *reinterpret_cast<const f32x4*>(pr + i) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    f32x4 sum[V];
#pragma unroll
    for (int j = 0; j < V; j++) sum[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < SPL; k++)
#pragma unroll
      for (int j = 0; j < V; j++)
        if (k < splits) sum[j] += pv[k][j];
#pragma unroll
    for (int j = 0; j < V; j++) {
      const int i = (threadIdx.x + CN_BLOCK * j) * 4;
      v[j] = v[j] + sum[j];
      if (i < dim) *reinterpret_cast<f32x4*>(xr + i) = v[j];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < V; j++) ss += v[j][0] * v[j][0] + v[j][1] * v[j][1] + v[j][2] * v[j][2] + v[j][3] * v[j][3];
  ss = cn_block_sum(ss, red);
  const float rms = 1.0f / sqrtf(ss / (float)dim + eps);
  uint16_t* o = xb + row * dim;
#pragma unroll
  for (int j = 0; j < V; j++) {
    const int i = (threadIdx.x + CN_BLOCK * j) * 4;
    if (i >= dim) continue;
    const float4 w = *reinterpret_cast<const float4*>(g + i);
    const float y0 = v[j][0] * rms * w.x, y1 = v[j][1] * rms * w.y, y2 = v[j][2] * rms * w.z, y3 = v[j][3] * rms * w.w;
    // the four elements stay adjacent in the span order
    const int pos = cn_span_pos(i);
    uint2 hh, ll;
    cn_split_f16x2(y0, y1, hh.x, ll.x);
    cn_split_f16x2(y2, y3, hh.y, ll.y);
    *reinterpret_cast<uint2*>(o + pos) = hh;
    *reinterpret_cast<uint2*>(xb_lo + row * dim + pos) = ll;
  }
}

// ---------------------------------------------------------------------------
// Packing: one thread re-encodes the 64 weights of chunk c of row r as a
// 96-byte unit: 64 u8 codes in K order, then scale[4] and offset[4] (fp32,
// one pair per 16 weights).  Each block type's dequantized value is
// fmaf(code, scale, offset) with one rounding, as the reference rounds it:
//   Q4_0 (DequantQ4_0.cs)  code q,      scale d,        offset -8d
//   Q4_1 (DequantQ4_1.cs)  code q,      scale d,        offset m
//   Q5_0 (DequantQ5_0.cs)  code q5,     scale d,        offset -16d
//   Q5_1 (DequantQ5_1.cs)  code q5,     scale d,        offset m
//   Q8_0 (DequantQ8_0.cs)  code q+128,  scale d,        offset -128d
//   Q2_K (DequantQ2K.cs)   code q,      scale d*sc,     offset -(dmin*m)
//   Q3_K (DequantQ3K.cs)   code q3,     scale d*sc,     offset -4*d*sc
//   Q4_K (DequantQ4K.cs)   code q,      scale d*sc[s],  offset -(dmin*m[s])
//   Q5_K (DequantQ5K.cs)   code q5,     scale d*sc[s],  offset -(dmin*m[s])
//   Q6_K (DequantQ6K.cs)   code q+32,   scale d*sc[i],  offset -32*d*sc[i]
//   Q8_K (DequantQ8K.cs)   code q+128,  scale d (fp32), offset -128d
//   IQ4_NL, IQ4_XS (DequantIQ.cs)  code table[q]+128, scale d or d*sc, offset -128*scale
//   IQ3_S    code +-(sc*q3)+128, scale d, offset -128d (sc folded into the code)
//   IQ3_XXS  code q3, scale d, offset -4d
//   IQ2_XXS, IQ2_XS  code q, scale d or d*sc, offset -scale
//   IQ2_S    code +-q+128, scale d*sc, offset -128*scale
//   IQ1_S, IQ1_M  code 128+t (t in -1..1; IQ1_M 128+t*2 at full scale), scale d
//            (IQ1_M d/2), offset -128*scale
// (d*sc, dmin*m and the power-of-two multiples are exact in fp32, and so is
// code*scale for the fp16-scaled types, so their one rounding is the
// reference's final add (or none); Q6_K's (d*sc)*q and Q8_K's q*d are rounded
// once either way).  Q2_K and Q3_K elements follow the reference's layouts
// (DequantQ2K.cs:55-82: element 128g + 32t + 16h + l is bits 2t.. of qs[32g +
// 16h + l] with scale byte 8g + 2t + h; DequantQ3K.cs:52-63, :122-150).  Sub-block layouts: Q4_K / Q5_K sub-block s of a super-block
// holds its 32 weights in the reference's order (elements 0..15 are the
// low nibbles of qs[16s..16s+15], 16..31 the high ones), Q6_K as
// DequantQ6K.Dequantize (DequantQ6K.cs:37-88).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f_at(const uint8_t* p) { return cn_h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

// Q4_K / Q5_K 6-bit scale and min of sub-block j (DequantQ4K.cs:218-264).
__device__ __forceinline__ void k4_scale_min(const uint8_t* q, int j, int& sc, int& mn) {
  if (j < 4) {
    sc = q[j] & 63;
    mn = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// IQ4_NL's table (DequantIQ.IQ4NL_Table, DequantIQ.cs:29-33) plus 128: the
// packed code of each index.
__constant__ uint8_t cn_iq4nl_code[16] = {1, 24, 45, 63, 79, 93, 106, 118, 129, 141, 153, 166, 181, 197, 217, 241};

__global__ __launch_bounds__(CN_BLOCK) void gemm_pack_kernel(int qtype, const uint8_t* __restrict__ w,
                                                            size_t row_bytes, size_t w_bytes, int M, int nchunks,
                                                            uint8_t* __restrict__ dst) {
  const long long t = (long long)blockIdx.x * CN_BLOCK + threadIdx.x;
  if (t >= (long long)M * nchunks) return;
  const int r = (int)(t / nchunks), c = (int)(t % nchunks);
  const uint8_t* row = w + (size_t)r * row_bytes;
  uint32_t code[16];
  float sc[4], of[4];
  auto put = [&](int k, uint32_t v) {
    if ((k & 3) == 0) code[k >> 2] = 0;
    code[k >> 2] |= (v & 0xFFu) << (8 * (k & 3));
  };
  if (qtype == 2 || qtype == 8) {  // Q4_0 / Q8_0: blocks 2c and 2c+1 of 32
    const int bb = qtype == 2 ? 18 : 34;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const uint8_t* blk = row + (size_t)(2 * c + b) * bb;
      const float d = h2f_at(blk);
#pragma unroll
      for (int j = 0; j < 32; j++) {
        uint32_t v;
        if (qtype == 2) v = j < 16 ? (blk[2 + j] & 15u) : (uint32_t)(blk[2 + j - 16] >> 4);
        else v = (uint32_t)blk[2 + j] ^ 0x80u;
        put(32 * b + j, v);
      }
      sc[2 * b] = sc[2 * b + 1] = d;
      of[2 * b] = of[2 * b + 1] = (qtype == 2 ? -8.0f : -128.0f) * d;
    }
  } else if (qtype == 12 || qtype == 13) {  // Q4_K / Q5_K: sub-blocks 2(c%4), 2(c%4)+1
    const int sbb = qtype == 12 ? 144 : 176;
    const uint8_t* blk = row + (size_t)(c >> 2) * sbb;
    const float d = h2f_at(blk), dmin = h2f_at(blk + 2);
    const uint8_t* qs0 = blk + (qtype == 12 ? 16 : 48);
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int s = 2 * (c & 3) + b;
      int sv, mv;
      k4_scale_min(blk + 4, s, sv, mv);
      const uint8_t* qs = qs0 + 16 * s;
#pragma unroll
      for (int j = 0; j < 32; j++) {
        uint32_t v = j < 16 ? (qs[j] & 15u) : (uint32_t)(qs[j - 16] >> 4);
        if (qtype == 13) {
          const int e = 32 * s + j;
          v |= (uint32_t)((blk[16 + e / 8] >> (e % 8)) & 1) << 4;
        }
        put(32 * b + j, v);
      }
      sc[2 * b] = sc[2 * b + 1] = d * (float)sv;
      of[2 * b] = of[2 * b + 1] = -(dmin * (float)mv);
    }
  } else if (qtype == 3 || qtype == 6 || qtype == 7) {  // Q4_1 / Q5_0 / Q5_1: blocks 2c and 2c+1 of 32
    const int bb = qtype == 3 ? 20 : (qtype == 6 ? 22 : 24);
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const uint8_t* blk = row + (size_t)(2 * c + b) * bb;
      const float d = h2f_at(blk);
      const uint8_t* qs = blk + bb - 16;
      uint32_t qh = 0;
      if (qtype != 3) {
        const uint8_t* h = blk + (qtype == 6 ? 2 : 4);
        qh = (uint32_t)h[0] | ((uint32_t)h[1] << 8) | ((uint32_t)h[2] << 16) | ((uint32_t)h[3] << 24);
      }
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const uint32_t nib = j < 16 ? (qs[j] & 15u) : (uint32_t)(qs[j - 16] >> 4);
        put(32 * b + j, nib | (((qh >> j) & 1u) << 4));
      }
      sc[2 * b] = sc[2 * b + 1] = d;
      of[2 * b] = of[2 * b + 1] = qtype == 6 ? -16.0f * d : (qtype == 3 || qtype == 7 ? h2f_at(blk + 2) : 0.f);
    }
  } else if (qtype == 10) {  // Q2_K: elements 64(c%4) .. +63 of the super-block
    const uint8_t* blk = row + (size_t)(c >> 2) * 84;
    const float d = h2f_at(blk + 80), dmin = h2f_at(blk + 82);
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const int e = 64 * (c & 3) + j, g = e >> 7, t = (e & 127) >> 5, h = (e & 31) >> 4, l = e & 15;
      put(j, (uint32_t)(blk[16 + 32 * g + 16 * h + l] >> (2 * t)) & 3u);
      if ((j & 15) == 0) {
        const uint8_t sb = blk[8 * g + 2 * t + h];
        sc[j >> 4] = d * (float)(sb & 15);
        of[j >> 4] = -(dmin * (float)(sb >> 4));
      }
    }
  } else if (qtype == 11) {  // Q3_K: elements 64(c%4) .. +63 of the super-block
    const uint8_t* blk = row + (size_t)(c >> 2) * 110;
    const float d = h2f_at(blk + 108);
    const uint8_t* s = blk + 96;
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const int e = 64 * (c & 3) + j;
      const uint32_t q2 = (blk[32 + e / 4] >> (2 * (e % 4))) & 3u, hb = (blk[e / 8] >> (e % 8)) & 1u;
      put(j, q2 | (hb << 2));
      if ((j & 15) == 0) {
        const int i = e >> 4;  // the sub-block's 6-bit scale, stored + 32
        const int lo = i < 8 ? (s[i] & 15) : (s[i - 8] >> 4);
        const int v = (lo | (((s[8 + (i & 3)] >> (2 * (i >> 2))) & 3) << 4)) - 32;
        sc[j >> 4] = d * (float)v;
        of[j >> 4] = -4.0f * sc[j >> 4];
      }
    }
  } else if (qtype == 15) {  // Q8_K: elements 64(c%4) .. +63 of the super-block
    const uint8_t* blk = row + (size_t)(c >> 2) * 292;
    float d;
    __builtin_memcpy(&d, blk, 4);
#pragma unroll
    for (int j = 0; j < 64; j++) put(j, (uint32_t)blk[4 + 64 * (c & 3) + j] ^ 0x80u);
#pragma unroll
    for (int g = 0; g < 4; g++) {
      sc[g] = d;
      of[g] = -128.0f * d;
    }
  } else if (qtype == 20) {  // IQ4_NL: blocks 2c and 2c+1 of 32 (DequantIQ.cs:46-76)
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const uint8_t* blk = row + (size_t)(2 * c + b) * 18;
      const float d = h2f_at(blk);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        put(32 * b + j, cn_iq4nl_code[blk[2 + j] & 15]);
        put(32 * b + 16 + j, cn_iq4nl_code[blk[2 + j] >> 4]);
      }
      sc[2 * b] = sc[2 * b + 1] = d;
      of[2 * b] = of[2 * b + 1] = -128.0f * d;
    }
  } else if (qtype == 23) {  // IQ4_XS: sub-blocks 2(c%4), 2(c%4)+1 (DequantIQ.cs:139-176)
    const uint8_t* blk = row + (size_t)(c >> 2) * 136;
    const float d = h2f_at(blk);
    const int sh = blk[2] | (blk[3] << 8);
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int s = 2 * (c & 3) + b;
      // low scale bits from byte 4+s (bytes 8..11 are sub-block 0's first quants)
      const int scv = ((blk[4 + s] & 0x3F) | (((sh >> (2 * s)) & 3) << 6)) - 32;
      const uint8_t* qs = blk + 8 + 16 * s;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        put(32 * b + j, cn_iq4nl_code[qs[j] & 15]);
        put(32 * b + 16 + j, cn_iq4nl_code[qs[j] >> 4]);
      }
      sc[2 * b] = sc[2 * b + 1] = d * (float)scv;
      of[2 * b] = of[2 * b + 1] = -128.0f * sc[2 * b];
    }
  } else if (qtype == 21) {  // IQ3_S: elements 64(c%4) .. +63 (DequantIQ.cs:244-290)
    // sign bytes 98..129 and scale bytes 130..137 reach up to 28 bytes into the
    // next block; past the end of w they read as zero (the tail a model's
    // upload pads with)
    const size_t base = (size_t)r * row_bytes + (size_t)(c >> 2) * 110;
    auto at = [&](int off) -> uint32_t { return base + off < w_bytes ? w[base + off] : 0u; };
    const float d = h2f_at(w + base);
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const int idx = 64 * (c & 3) + j, sub = idx >> 3;
      const int q3 = (int)(((at(2 + idx / 4) >> (2 * (idx % 4))) & 3u) | (((at(66 + idx / 8) >> (idx % 8)) & 1u) << 2));
      const int scv = (int)((at(130 + sub / 4) >> (2 * (sub % 4))) & 3u) + 1;
      const int v = ((at(98 + sub) >> (idx & 7)) & 1u) ? -scv * q3 : scv * q3;
      put(j, (uint32_t)(v + 128));
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
      sc[g] = d;
      of[g] = -128.0f * d;
    }
  } else if (qtype == 18) {  // IQ3_XXS: d * (q3 - 4) (DequantIQ.cs:364-399)
    const uint8_t* blk = row + (size_t)(c >> 2) * 98;
    const float d = h2f_at(blk);
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const int idx = 64 * (c & 3) + j;
      const uint8_t* p = blk + 2 + 3 * (idx >> 3);
      const uint32_t word = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16);
      put(j, (word >> (3 * (idx & 7))) & 7u);
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
      sc[g] = d;
      of[g] = -4.0f * d;
    }
  } else if (qtype == 16 || qtype == 17 || qtype == 22) {  // IQ2_XXS / IQ2_XS / IQ2_S: sub-blocks 4(c%4) ..
    const int bb = qtype == 16 ? 66 : (qtype == 17 ? 74 : 82);
    const uint8_t* blk = row + (size_t)(c >> 2) * bb;
    const float d = h2f_at(blk);
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int sub = 4 * (c & 3) + g;
      const uint8_t* qs = blk + 2 + 4 * sub;
      if (qtype == 22) {  // (d * (low nibble + 1)) * q, elements 0..3 signed (DequantIQ.cs:656-696)
        const uint32_t qh = blk[66 + sub];
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int q = (qs[e >> 2] >> (2 * (e & 3))) & 3;
          const bool neg = e < 4 && ((qh >> (4 + e)) & 1u);
          put(16 * g + e, (uint32_t)((neg ? -q : q) + 128));
        }
        sc[g] = d * (float)((qh & 15u) + 1);
        of[g] = -128.0f * sc[g];
      } else {  // d * (q - 1) or (d * sc) * (q - 1), sc a signed nibble - 8 (DequantIQ.cs:456-598)
#pragma unroll
        for (int e = 0; e < 16; e++) put(16 * g + e, (qs[e >> 2] >> (2 * (e & 3))) & 3u);
        float dsc = d;
        if (qtype == 17) {
          const int raw = (int8_t)blk[66 + sub / 2];
          dsc = d * (float)(((sub & 1) ? (raw >> 4) & 15 : raw & 15) - 8);
        }
        sc[g] = dsc;
        of[g] = -dsc;
      }
    }
  } else if (qtype == 19 || qtype == 29) {  // IQ1_S / IQ1_M: ternary (DequantIQ.cs:767-805, :869-914)
    const int bb = qtype == 19 ? 50 : 56;
    const uint8_t* blk = row + (size_t)(c >> 2) * bb;
    const float d = h2f_at(blk);
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const int idx = 64 * (c & 3) + j, sub = idx >> 3, e = idx & 7;
      const int tv = ((blk[2 + sub] >> e) & 1) ? 1 : (((blk[34 + sub / 2] >> ((sub & 1) * 4 + e / 2)) & 1) ? -1 : 0);
      // IQ1_M: d * sc with sc 1 or 0.5 (bit sub%8 of byte 50 + sub/8) as (d/2) * (2 or 1)
      const int m = qtype == 19 ? 1 : (((blk[50 + sub / 8] >> (sub & 7)) & 1) ? 2 : 1);
      put(j, (uint32_t)(128 + tv * m));
    }
    const float step = qtype == 19 ? d : 0.5f * d;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      sc[g] = step;
      of[g] = -128.0f * step;
    }
  } else {  // Q6_K: elements 64(c%4) .. +63 of the super-block
    const uint8_t* blk = row + (size_t)(c >> 2) * 210;
    const float d = h2f_at(blk + 208);
    const int8_t* scl = reinterpret_cast<const int8_t*>(blk + 192);
#pragma unroll
    for (int j = 0; j < 64; j++) {
      const int e = 64 * (c & 3) + j, hh = e >> 7, e2 = e & 127, qq = e2 >> 5, l = e2 & 31;
      const uint8_t qlb = blk[64 * hh + l + 32 * (qq & 1)];
      const uint32_t nib = qq >= 2 ? (uint32_t)(qlb >> 4) : (qlb & 15u);
      const uint32_t hb = (blk[128 + 32 * hh + l] >> (2 * qq)) & 3u;
      put(j, nib | (hb << 4));
      if ((j & 15) == 0) {
        const float s = d * (float)scl[8 * hh + l / 16 + 2 * qq];
        sc[j >> 4] = s;
        of[j >> 4] = -32.0f * s;
      }
    }
  }
  uint4* o = reinterpret_cast<uint4*>(dst + ((size_t)r * nchunks + c) * kGemmPackUnit);
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = make_uint4(code[4 * i], code[4 * i + 1], code[4 * i + 2], code[4 * i + 3]);
  o[4] = make_uint4(__float_as_uint(sc[0]), __float_as_uint(sc[1]), __float_as_uint(sc[2]), __float_as_uint(sc[3]));
  o[5] = make_uint4(__float_as_uint(of[0]), __float_as_uint(of[1]), __float_as_uint(of[2]), __float_as_uint(of[3]));
}

// Column tile by batch size and kernel.  One-plane kernel: see pick_gemm
// (at least 8 chunks of 64 per split).  Span kernel: 32 or 64 columns; a tile grid of more than two workgroups per CU
// takes the 2-stage ring (44 KB for raw Q4_0 at 64 columns, three workgroups
// per CU; 56 KB for packed units, two), a smaller one the 3-stage ring (two
// per CU) and a K split into the largest count that keeps the grid within one
// round of resident workgroups with at least 8 chunks per split (a grid just
// over a round would run a second round on a few CUs).
struct GemmShape {
  int tn, splits, stages, mt = 1;
  int sk_wgs = 0, sk_dp = 0;  // one-plane kernel: stream-K workgroups (0: none), of them whole-tile ones
  long long tiles = 0;
};

constexpr int kStages = 3;

template <bool PRECISE, int TN, int S, int WF>
constexpr int ring_bytes() {
  return PipeCfg<PRECISE, TN, S, WF>::LDS;
}

template <int WF>
int span_ring_bytes_t(int tn, int stages) {
  if (stages == 2) return tn == 1 ? ring_bytes<true, 1, 2, WF>() : ring_bytes<true, 2, 2, WF>();
  return tn == 1 ? ring_bytes<true, 1, 3, WF>() : ring_bytes<true, 2, 3, WF>();
}

int span_ring_bytes(int tn, int stages, int wf) {
  switch (wf) {
    case GEMM_W_PACKED: return span_ring_bytes_t<GEMM_W_PACKED>(tn, stages);
    case GEMM_W_F16: return span_ring_bytes_t<GEMM_W_F16>(tn, stages);
    case GEMM_W_F32: return span_ring_bytes_t<GEMM_W_F32>(tn, stages);
    case GEMM_W_Q4_K: return span_ring_bytes_t<GEMM_W_Q4_K>(tn, stages);
    default: return span_ring_bytes_t<GEMM_W_Q4_0>(tn, stages);
  }
}

GemmShape pick_gemm(int M, int N, int K, int num_cus, bool precise, int wf, bool stream_k = false) {
  GemmShape s;
  const int nchunks = K / 64;
  s.splits = 1;
  s.stages = kStages;
  if (precise) {
    s.tn = N <= 32 ? 1 : 2;
    const long long tiles = (long long)((M + 127) / 128) * ((N + 32 * s.tn - 1) / (32 * s.tn));
    s.stages = tiles > 2LL * num_cus ? 2 : 3;
    const int per_cu = std::max(1, std::min(3, 160 * 1024 / span_ring_bytes(s.tn, s.stages, wf)));
    const long long slots = (long long)per_cu * num_cus;
    while (s.splits < 16 && tiles * (s.splits + 1) <= slots && nchunks / (s.splits + 1) >= 8) s.splits++;
  } else {
    // 32, 64 or 128 columns per workgroup.  Tiles of 64 and 128 columns run
    // the 2-stage ring (44 KB of LDS for raw Q4_0 at 128 columns: three
    // workgroups per CU, which hide each other's waits better than a deeper
    // ring with fewer workgroups) and split K only while the tile grid is
    // smaller than the CU count (a split's partials cost a reduce pass over
    // N x M x splits floats); 32-column tiles (N <= 32, HBM-bound) run a
    // 4-stage ring (40 KB) under the same split rule.  Measured per call,
    // 11008 x 4096 at N = 512: 93.6 us with 3 stages and splits up to two
    // workgroups per CU, 81.4 us with this rule; at N = 8: 20.4 us with 3
    // stages and that wider split, 17.8 us with this rule (6 and 8 stages:
    // 18.4, 18.9).
    s.tn = N <= 32 ? 1 : (N <= 64 ? 2 : 4);
    s.stages = s.tn == 1 ? 4 : 2;
    // Two 32-row tiles per wave (256-row workgroups, each x fragment read
    // from LDS feeding two MFMAs) where that still leaves a tile per CU:
    // 32000 x 2048 at N = 512, 96.7 -> 85.3 us per call; 11008 x 4096 (172
    // such tiles) went 79.3 -> 88.3 us and keeps one.
    // Stream-K for a grid of 128-row tiles just over one per CU (a partial
    // second round: 11008 x 4096 at N = 512 has 344 tiles, and 88 CUs ran
    // two while the rest idled): one whole tile per CU, and a second
    // workgroup per CU takes an equal share (at least 8 chunks) of the
    // remaining tiles' chunks.  Measured per call (same box, alternating
    // builds): 11008 x 4096 N = 512 74.4 -> 71.2 us, N = 480 74.2 -> 70.6;
    // at 448 tiles (14336 x 4096) 82.1 -> 87.1, so only up to 1.4 tiles per
    // CU.  Sharing every tile of a smaller grid this way instead of splitting
    // K measured slower than the split and its reduce pass (4096 x 4096 N =
    // 512 41.5 -> 46.3 us, N = 8 11008 x 4096 18.7 -> 21.0): a shared tile's
    // parts cost device-scope round trips (store, arrival, reads).
    const long long tiles1 = (long long)((M + 127) / 128) * ((N + 32 * s.tn - 1) / (32 * s.tn));
    if (stream_k && tiles1 > num_cus && tiles1 <= kGemmTileCounters && tiles1 * 5 <= 7LL * num_cus &&
        (tiles1 - num_cus) * nchunks / num_cus >= 8) {
      s.tiles = tiles1;
      s.sk_dp = num_cus;
      s.sk_wgs = 2 * num_cus;
      return s;
    }
    if (s.tn == 4 && (long long)((M + 255) / 256) * ((N + 127) / 128) >= num_cus) s.mt = 2;
    const long long tiles = (long long)((M + 128 * s.mt - 1) / (128 * s.mt)) * ((N + 32 * s.tn - 1) / (32 * s.tn));
    s.tiles = tiles;
    const long long want = num_cus;
    while (tiles * s.splits < want && nchunks / (s.splits * 2) >= 8 && s.splits < 16) s.splits *= 2;
  }
  return s;
}

template <int TN, int S, bool PK, int MT, bool SK = false>
hipError_t launch_p(const GemmArgs& a, int grid, hipStream_t st) {
  constexpr int lds = PipeCfg<false, TN, S, PK, MT, 1>::LDS;
  static_assert(lds <= 160 * 1024, "LDS ring exceeds the CU's 160 KB");
  static std::atomic<uint64_t> lds_done{0};
  if (lds > 64 * 1024) {
    const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(&gemm_p_kernel<TN, S, PK, MT, 1, SK>), lds_done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemm_p_kernel<TN, S, PK, MT, 1, SK>), dim3(grid), dim3(CN_BLOCK), lds, st, a);
  return hipGetLastError();
}

// Stream-K launches run one-row-tile (MT = 1) instances.
template <int TN, bool PK>
hipError_t launch_p_ring(const GemmArgs& a, int mt, int grid, hipStream_t st) {
  constexpr int S = TN == 1 ? 4 : 2;
  if (a.sk_wgs > 0) return launch_p<TN, S, PK, 1, true>(a, grid, st);
  if constexpr (TN == 4) {
    if (mt == 2) return launch_p<TN, S, PK, 2>(a, grid, st);
  }
  return launch_p<TN, S, PK, 1>(a, grid, st);
}

template <int TN, int S, int WF>
hipError_t launch_s(const GemmArgs& a, int grid, hipStream_t st) {
  constexpr int lds = PipeCfg<true, TN, S, WF>::LDS;
  static_assert(lds <= 160 * 1024, "LDS ring exceeds the CU's 160 KB");
  static std::atomic<uint64_t> lds_done{0};
  if (lds > 64 * 1024) {
    const hipError_t e = allow_full_lds(reinterpret_cast<const void*>(&gemm_s_kernel<TN, S, WF>), lds_done);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((gemm_s_kernel<TN, S, WF>), dim3(grid), dim3(CN_BLOCK), lds, st, a);
  return hipGetLastError();
}

template <int TN, int WF>
hipError_t launch_s_ring(const GemmArgs& a, int stages, int grid, hipStream_t st) {
  return stages == 2 ? launch_s<TN, 2, WF>(a, grid, st) : launch_s<TN, 3, WF>(a, grid, st);
}

template <int TN>
hipError_t launch_s_fmt(const GemmArgs& a, int stages, int grid, hipStream_t st) {
  switch (a.packed) {
    case GEMM_W_PACKED: return launch_s_ring<TN, GEMM_W_PACKED>(a, stages, grid, st);
    case GEMM_W_F16: return launch_s_ring<TN, GEMM_W_F16>(a, stages, grid, st);
    case GEMM_W_F32: return launch_s_ring<TN, GEMM_W_F32>(a, stages, grid, st);
    case GEMM_W_Q4_K: return launch_s_ring<TN, GEMM_W_Q4_K>(a, stages, grid, st);
    default: return launch_s_ring<TN, GEMM_W_Q4_0>(a, stages, grid, st);
  }
}

hipError_t launch_kernel(const GemmArgs& a, const GemmShape& s, bool precise, int grid, hipStream_t st) {
  const bool pk = a.packed != 0;
  const int tn = s.tn;
  if (precise) return tn == 1 ? launch_s_fmt<1>(a, s.stages, grid, st) : launch_s_fmt<2>(a, s.stages, grid, st);
  if (tn == 1) return pk ? launch_p_ring<1, true>(a, 1, grid, st) : launch_p_ring<1, false>(a, 1, grid, st);
  if (tn == 2) return pk ? launch_p_ring<2, true>(a, 1, grid, st) : launch_p_ring<2, false>(a, 1, grid, st);
  return pk ? launch_p_ring<4, true>(a, s.mt, grid, st) : launch_p_ring<4, false>(a, s.mt, grid, st);
}

}  // namespace

bool gemm_supports(int qtype, int K) { return qtype == 2 && K > 0 && K % 64 == 0; }

bool gemm_pack_supports(int qtype, int K) {
  if (K <= 0) return false;
  if (qtype == 2 || qtype == 3 || qtype == 6 || qtype == 7 || qtype == 8 || qtype == 20) return K % 64 == 0;
  if ((qtype >= 10 && qtype <= 19) || (qtype >= 21 && qtype <= 23) || qtype == 29) return K % 256 == 0;
  return false;
}

size_t gemm_pack_bytes(int M, int K) { return (size_t)M * (size_t)(K / 64) * kGemmPackUnit; }

hipError_t gemm_pack_launch(int qtype, const void* w, int M, int K, void* dst, hipStream_t st) {
  if (!gemm_pack_supports(qtype, K) || M <= 0 || !w || !dst) return hipErrorInvalidValue;
  size_t row_bytes;
  switch (qtype) {
    case 2: row_bytes = (size_t)K / 32 * 18; break;
    case 3: row_bytes = (size_t)K / 32 * 20; break;
    case 6: row_bytes = (size_t)K / 32 * 22; break;
    case 7: row_bytes = (size_t)K / 32 * 24; break;
    case 8: row_bytes = (size_t)K / 32 * 34; break;
    case 10: row_bytes = (size_t)K / 256 * 84; break;
    case 11: row_bytes = (size_t)K / 256 * 110; break;
    case 12: row_bytes = (size_t)K / 256 * 144; break;
    case 13: row_bytes = (size_t)K / 256 * 176; break;
    case 15: row_bytes = (size_t)K / 256 * 292; break;
    case 16: row_bytes = (size_t)K / 256 * 66; break;
    case 17: row_bytes = (size_t)K / 256 * 74; break;
    case 18: row_bytes = (size_t)K / 256 * 98; break;
    case 19: row_bytes = (size_t)K / 256 * 50; break;
    case 20: row_bytes = (size_t)K / 32 * 18; break;
    case 21: row_bytes = (size_t)K / 256 * 110; break;
    case 22: row_bytes = (size_t)K / 256 * 82; break;
    case 23: row_bytes = (size_t)K / 256 * 136; break;
    case 29: row_bytes = (size_t)K / 256 * 56; break;
    default: row_bytes = (size_t)K / 256 * 210; break;
  }
  const long long n = (long long)M * (K / 64);
  const long long blocks = (n + CN_BLOCK - 1) / CN_BLOCK;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gemm_pack_kernel, dim3((unsigned)blocks), dim3(CN_BLOCK), 0, st, qtype,
                     static_cast<const uint8_t*>(w), row_bytes, (size_t)M * row_bytes, M, K / 64,
                     static_cast<uint8_t*>(dst));
  return hipGetLastError();
}

size_t gemm_workspace_bytes(int M, int N, int K, int num_cus, bool precise, int wfmt, bool stream_k) {
  const GemmShape s = pick_gemm(M, N, K, num_cus, precise, wfmt, stream_k && !precise);
  if (s.sk_wgs > 0) return (size_t)2 * s.sk_wgs * (128 * s.mt) * (32 * s.tn) * sizeof(float);
  return s.splits > 1 ? (size_t)s.splits * N * M * sizeof(float) : 0;
}

hipError_t gemm_launch(const GemmArgs& a_in, int num_cus, hipStream_t st, int* splits_left) {
  if (a_in.packed < GEMM_W_Q4_0 || a_in.packed > GEMM_W_Q4_K || (a_in.packed > GEMM_W_PACKED && !a_in.precise))
    return hipErrorInvalidValue;  // float rows and raw Q4_K only in the span kernel
  const bool k_ok = a_in.packed == GEMM_W_Q4_K ? (a_in.K > 0 && a_in.K % 256 == 0)
                    : a_in.packed                ? (a_in.K > 0 && a_in.K % 64 == 0)
                                                 : gemm_supports(a_in.qtype, a_in.K);
  if (!k_ok || a_in.M <= 0 || a_in.N <= 0) return hipErrorInvalidValue;
  const bool precise = a_in.precise != 0;
  if (precise && !a_in.xb_lo) return hipErrorInvalidValue;
  // partials can be left only for a store or a residual add (the folding
  // kernels apply no other epilogue)
  if (splits_left && a_in.epi != GEMV_EPI_STORE && a_in.epi != GEMV_EPI_ADD) return hipErrorInvalidValue;
  if (a_in.epi == GEMV_EPI_SWIGLU && (!a_in.hb || !a_in.hb_lo)) return hipErrorInvalidValue;
  const GemmShape s =
      pick_gemm(a_in.M, a_in.N, a_in.K, num_cus, precise, a_in.packed, a_in.tile_cnt != nullptr && !precise);
  GemmArgs a = a_in;
  a.splits = s.splits;
  a.sk_wgs = s.sk_wgs;
  a.sk_dp = s.sk_dp;
  a.sk_tiles = (int)s.tiles;
  if ((s.splits > 1 || s.sk_wgs > 0) && !a.part) return hipErrorInvalidValue;
  const long long grid = s.sk_wgs > 0 ? s.sk_wgs
                                      : (long long)((a.M + 128 * s.mt - 1) / (128 * s.mt)) *
                                            ((a.N + 32 * s.tn - 1) / (32 * s.tn)) * s.splits;
  if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipError_t e = launch_kernel(a, s, precise, (int)grid, st);
  if (splits_left) *splits_left = 0;
  if (e != hipSuccess || s.splits == 1) return e;
  if (splits_left) {  // the caller folds the partials into its next kernel
    *splits_left = s.splits;
    return hipSuccess;
  }
  const long long work = (long long)((a.M + 3) / 4) * a.N;
  hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((work + CN_BLOCK - 1) / CN_BLOCK)), dim3(CN_BLOCK), 0, st, a);
  return hipGetLastError();
}

hipError_t to_f16_scaled_launch(const float* x, uint16_t* xh, float* xinv, int N, int K, hipStream_t st) {
  if (N <= 0 || K <= 0 || K % 32 || K > 16384) return hipErrorInvalidValue;
  const int v = (K + 4 * CN_BLOCK - 1) / (4 * CN_BLOCK);  // float4 per thread
  const dim3 grid(N), block(CN_BLOCK);
  if (v <= 2) hipLaunchKernelGGL((to_f16_scaled_kernel<2>), grid, block, 0, st, x, xh, xinv, K);
  else if (v <= 4) hipLaunchKernelGGL((to_f16_scaled_kernel<4>), grid, block, 0, st, x, xh, xinv, K);
  else if (v <= 8) hipLaunchKernelGGL((to_f16_scaled_kernel<8>), grid, block, 0, st, x, xh, xinv, K);
  else hipLaunchKernelGGL((to_f16_scaled_kernel<16>), grid, block, 0, st, x, xh, xinv, K);
  return hipGetLastError();
}

template <int V>
void add_rmsnorm_v(float* x, const float* part, int splits, const float* g, float eps, uint16_t* xb, uint16_t* xb_lo,
                   int rows, int dim, hipStream_t st) {
  const dim3 grid(rows), block(CN_BLOCK);
  if (V > 4 || splits <= 0) {  // wide rows: the norm alone (no partials folded)
    hipLaunchKernelGGL((add_rmsnorm_span_kernel<V, 0>), grid, block, 0, st, x, part, 0, g, eps, xb, xb_lo, rows, dim);
    return;
  }
  if constexpr (V <= 4) {
  if (splits <= 0) hipLaunchKernelGGL((add_rmsnorm_span_kernel<V, 0>), grid, block, 0, st, x, part, 0, g, eps, xb, xb_lo, rows, dim);
  else if (splits <= 2) hipLaunchKernelGGL((add_rmsnorm_span_kernel<V, 2>), grid, block, 0, st, x, part, splits, g, eps, xb, xb_lo, rows, dim);
  else if (splits <= 4) hipLaunchKernelGGL((add_rmsnorm_span_kernel<V, 4>), grid, block, 0, st, x, part, splits, g, eps, xb, xb_lo, rows, dim);
  else if (splits <= 8) hipLaunchKernelGGL((add_rmsnorm_span_kernel<V, 8>), grid, block, 0, st, x, part, splits, g, eps, xb, xb_lo, rows, dim);
  else hipLaunchKernelGGL((add_rmsnorm_span_kernel<V, 16>), grid, block, 0, st, x, part, splits, g, eps, xb, xb_lo, rows, dim);
  }
}

hipError_t add_rmsnorm_span_launch(float* x, const float* part, int splits, const float* g, float eps, uint16_t* xb,
                                   uint16_t* xb_lo, int rows, int dim, hipStream_t st) {
  if (dim % 4 || dim <= 0 || rows <= 0 || splits > 16 || (splits > 0 && !part)) return hipErrorInvalidValue;
  if (!xb || !xb_lo || dim % 32) return hipErrorInvalidValue;  // the span order permutes blocks of 32
  const int v = (dim + 4 * CN_BLOCK - 1) / (4 * CN_BLOCK);  // float4 per thread
  // at most 4 float4 per thread when partials are folded (the register budget of
  // 16 splits x 4 float4), 16 for the norm alone
  if (splits > 0 && v > 4) return hipErrorInvalidValue;
  if (v > 16) return hipErrorInvalidValue;
  if (v <= 2) add_rmsnorm_v<2>(x, part, splits, g, eps, xb, xb_lo, rows, dim, st);
  else if (v <= 4) add_rmsnorm_v<4>(x, part, splits, g, eps, xb, xb_lo, rows, dim, st);
  else if (v <= 8) add_rmsnorm_v<8>(x, part, 0, g, eps, xb, xb_lo, rows, dim, st);
  else add_rmsnorm_v<16>(x, part, 0, g, eps, xb, xb_lo, rows, dim, st);
  return hipGetLastError();
}

