/*
 * chatnet_oracle.c — CPU oracle (TEST INFRASTRUCTURE ONLY; see the header).
 *
 * Plain-C restatement of ChatNet's quantized Llama forward pass.  Citations
 * are path:line into the ChatNet sources.  Build with -ffp-contract=off so
 * that every `a*b + c` rounds twice, as RyuJIT's Vector128/Vector<T> code does.
 */
#include "chatnet_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* TensorMath.cs:28 — rows below this run serially. */
#define PARALLEL_ROW_THRESHOLD 512
/* Vector<float>.Count on AVX2 hardware (256-bit Vector<T>). */
#define VLEN 8

static int g_threads = 1;

void oracle_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int oracle_get_threads(void) { return g_threads; }

/* ---------------------------------------------------------------------------
 * DequantQ4_0.HalfToFloat (DequantQ4_0.cs:190-194): exact IEEE binary16 ->
 * binary32, subnormals, infinities and NaN payloads included.
 * ------------------------------------------------------------------------- */
float oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F;
  uint32_t man = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24, exact in binary32 */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400) == 0);
      man &= 0x3FF;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline float h2f(const uint8_t* p) { return oracle_half_to_float((uint16_t)(p[0] | (p[1] << 8))); }

/* Vector128.Sum for float: ((v0 + v1) + (v2 + v3)).  The JIT's lane order is
 * not visible in the C# source: parity unpinned at the last ulp. */
static inline float vsum4(const float v[4]) { return (v[0] + v[1]) + (v[2] + v[3]); }

/* TensorMath.VectorSum (TensorMath.cs:750-758) / LlamaModel.VectorSumFast
 * (LlamaModel.cs:353-362): sequential lane sum starting from 0. */
static inline float vsum8(const float v[VLEN]) {
  float s = 0.0f;
  for (int i = 0; i < VLEN; i++) s += v[i];
  return s;
}

/* ---------------------------------------------------------------------------
 * Q4_0 (DequantQ4_0.cs)
 * ------------------------------------------------------------------------- */

/* DequantQ4_0.Dequantize (DequantQ4_0.cs:28-58), partial last block included. */
void oracle_dequant_q4_0(const uint8_t* src, float* out, int n) {
  int blocks = (n + 31) / 32;
  int so = 0, dst = 0;
  for (int b = 0; b < blocks; b++) {
    float scale = h2f(src + so);
    so += 2;
    int remaining = n - dst;
    int half = remaining < 16 ? remaining : 16;
    for (int j = 0; j < half; j++) out[dst + j] = (float)((src[so + j] & 0x0F) - 8) * scale;
    int second = remaining < 32 ? (remaining > 16 ? remaining - 16 : 0) : 16;
    for (int j = 0; j < second; j++) out[dst + 16 + j] = (float)(((src[so + j] >> 4) & 0x0F) - 8) * scale;
    so += 16;
    dst += half + second;
  }
}

/* DequantQ4_0.DotProductVec128 (DequantQ4_0.cs:80-149). */
float oracle_dot_q4_0(const uint8_t* row, const float* x, int n) {
  int blocks = n / 32;
  float acc0[4] = {0, 0, 0, 0}, acc1[4] = {0, 0, 0, 0};
  const uint8_t* src = row;
  const float* in = x;
  for (int b = 0; b < blocks; b++) {
    float scale = h2f(src);
    src += 2;
    float lo[16], hi[16];
    for (int j = 0; j < 16; j++) {
      lo[j] = (float)((int)(src[j] & 0x0F) - 8);
      hi[j] = (float)((int)((src[j] >> 4) & 0x0F) - 8);
    }
    float ba0[4] = {0, 0, 0, 0}, ba1[4] = {0, 0, 0, 0};
    /* :121-124 then :135-138 — the accumulator alternates every 4 lanes */
    for (int l = 0; l < 4; l++) ba0[l] = ba0[l] + lo[l] * in[l];
    for (int l = 0; l < 4; l++) ba1[l] = ba1[l] + lo[4 + l] * in[4 + l];
    for (int l = 0; l < 4; l++) ba0[l] = ba0[l] + lo[8 + l] * in[8 + l];
    for (int l = 0; l < 4; l++) ba1[l] = ba1[l] + lo[12 + l] * in[12 + l];
    for (int l = 0; l < 4; l++) ba0[l] = ba0[l] + hi[l] * in[16 + l];
    for (int l = 0; l < 4; l++) ba1[l] = ba1[l] + hi[4 + l] * in[20 + l];
    for (int l = 0; l < 4; l++) ba0[l] = ba0[l] + hi[8 + l] * in[24 + l];
    for (int l = 0; l < 4; l++) ba1[l] = ba1[l] + hi[12 + l] * in[28 + l];
    /* :141-142 */
    for (int l = 0; l < 4; l++) {
      acc0[l] = acc0[l] + ba0[l] * scale;
      acc1[l] = acc1[l] + ba1[l] * scale;
    }
    src += 16;
    in += 32;
  }
  float s[4];
  for (int l = 0; l < 4; l++) s[l] = acc0[l] + acc1[l];
  return vsum4(s); /* :148 */
}

/* ---------------------------------------------------------------------------
 * Q4_K (DequantQ4K.cs) — the reference's own nibble order: sub-block s uses
 * qs[16s..16s+15]; low nibbles are elements 32s+0..15, high nibbles 32s+16..31.
 * ------------------------------------------------------------------------- */

/* DequantQ4K.DecodeScales / DecodeScalesUnsafe (DequantQ4K.cs:218-264),
 * llama.cpp get_scale_min_k4. */
static void q4k_scales(const uint8_t* q, int sc[8], int m[8]) {
  for (int j = 0; j < 4; j++) {
    sc[j] = q[j] & 63;
    m[j] = q[j + 4] & 63;
  }
  for (int j = 4; j < 8; j++) {
    sc[j] = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m[j] = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* DequantQ4K.Dequantize (DequantQ4K.cs:37-77). */
void oracle_dequant_q4_k(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 144;
    float d = h2f(blk + 0), dmin = h2f(blk + 2);
    int sc[8], m[8];
    q4k_scales(blk + 4, sc, m);
    for (int s = 0; s < 8; s++) {
      float dsc = d * (float)sc[s];
      float dm = dmin * (float)m[s];
      const uint8_t* qs = blk + 16 + s * 16;
      float* o = out + (size_t)b * 256 + s * 32;
      for (int j = 0; j < 16; j++) {
        o[j] = dsc * (float)(qs[j] & 0x0F) - dm;
        o[j + 16] = dsc * (float)((qs[j] >> 4) & 0x0F) - dm;
      }
    }
  }
}

/* DequantQ4K.DotProductVec128 (DequantQ4K.cs:89-163). */
float oracle_dot_q4_k(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float acc[4] = {0, 0, 0, 0};
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 144;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk + 0), dmin = h2f(blk + 2);
    int sc[8], m[8];
    q4k_scales(blk + 4, sc, m);
    float ba[4] = {0, 0, 0, 0};
    for (int s = 0; s < 8; s++) {
      float dsc = d * (float)sc[s];
      float dm = dmin * (float)m[s];
      const uint8_t* qs = blk + 16 + s * 16;
      const float* xi = in + s * 32;
      /* :137-140 low nibbles, then :151-154 high nibbles, 4 lanes at a time */
      for (int c = 0; c < 4; c++)
        for (int l = 0; l < 4; l++)
          ba[l] = ba[l] + ((float)(qs[4 * c + l] & 0x0F) * dsc - dm) * xi[4 * c + l];
      for (int c = 0; c < 4; c++)
        for (int l = 0; l < 4; l++)
          ba[l] = ba[l] + ((float)((qs[4 * c + l] >> 4) & 0x0F) * dsc - dm) * xi[16 + 4 * c + l];
    }
    for (int l = 0; l < 4; l++) acc[l] = acc[l] + ba[l]; /* :157 */
  }
  return vsum4(acc); /* :162 */
}

/* ---------------------------------------------------------------------------
 * Q6_K (DequantQ6K.cs): ql[128] @0, qh[64] @128, int8 scales[16] @192, d @208.
 * ------------------------------------------------------------------------- */

/* DequantQ6K.Dequantize (DequantQ6K.cs:37-88). */
void oracle_dequant_q6_k(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 210;
    float d = h2f(blk + 208);
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int h = 0; h < 2; h++) {
      const uint8_t* ql = blk + h * 64;
      const uint8_t* qh = blk + 128 + h * 32;
      float* o = out + (size_t)b * 256 + h * 128;
      for (int l = 0; l < 32; l++) {
        int si = h * 8 + l / 16;
        int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
        int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
        int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        o[l] = d * (float)sc[si] * (float)q1;
        o[l + 32] = d * (float)sc[si + 2] * (float)q2;
        o[l + 64] = d * (float)sc[si + 4] * (float)q3;
        o[l + 96] = d * (float)sc[si + 6] * (float)q4;
      }
    }
  }
}

/* DequantQ6K.DotProductVec128 (DequantQ6K.cs:104-188). */
float oracle_dot_q6_k(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float acc[4] = {0, 0, 0, 0};
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 210;
    float d = h2f(blk + 208);
    const int8_t* sc = (const int8_t*)(blk + 192);
    float ba[4] = {0, 0, 0, 0};
    for (int h = 0; h < 2; h++) {
      const uint8_t* ql = blk + h * 64;
      const uint8_t* qh = blk + 128 + h * 32;
      const float* in = x + (size_t)b * 256 + h * 128;
      for (int lb = 0; lb < 2; lb++) {
        int si = h * 8 + lb;
        float s0 = (float)sc[si], s2 = (float)sc[si + 2], s4 = (float)sc[si + 4], s6 = (float)sc[si + 6];
        for (int l = lb * 16; l < lb * 16 + 16; l += 4) {
          for (int i = 0; i < 4; i++) {
            float q1 = (float)(((ql[l + i] & 0xF) | (((qh[l + i] >> 0) & 3) << 4)) - 32);
            ba[i] = ba[i] + q1 * s0 * in[l + i];
          }
          for (int i = 0; i < 4; i++) {
            float q2 = (float)(((ql[l + 32 + i] & 0xF) | (((qh[l + i] >> 2) & 3) << 4)) - 32);
            ba[i] = ba[i] + q2 * s2 * in[l + 32 + i];
          }
          for (int i = 0; i < 4; i++) {
            float q3 = (float)(((ql[l + i] >> 4) | (((qh[l + i] >> 4) & 3) << 4)) - 32);
            ba[i] = ba[i] + q3 * s4 * in[l + 64 + i];
          }
          for (int i = 0; i < 4; i++) {
            float q4 = (float)(((ql[l + 32 + i] >> 4) | (((qh[l + i] >> 6) & 3) << 4)) - 32);
            ba[i] = ba[i] + q4 * s6 * in[l + 96 + i];
          }
        }
      }
    }
    for (int i = 0; i < 4; i++) acc[i] = acc[i] + ba[i] * d; /* :182 */
  }
  return vsum4(acc);
}

/* ---------------------------------------------------------------------------
 * fp32 ops (TensorMath.cs)
 * ------------------------------------------------------------------------- */

/* TensorMath.DotProductSimd (TensorMath.cs:666-702). */
float oracle_dot_f32(const float* a, const float* b, int n) {
  float sum = 0.0f;
  int i = 0;
  float v0[VLEN] = {0}, v1[VLEN] = {0};
  int lim2 = n - 2 * VLEN + 1;
  for (; i < lim2; i += 2 * VLEN)
    for (int l = 0; l < VLEN; l++) {
      v0[l] = v0[l] + a[i + l] * b[i + l];
      v1[l] = v1[l] + a[i + VLEN + l] * b[i + VLEN + l];
    }
  int lim1 = n - VLEN + 1;
  for (; i < lim1; i += VLEN)
    for (int l = 0; l < VLEN; l++) v0[l] = v0[l] + a[i + l] * b[i + l];
  float s[VLEN];
  for (int l = 0; l < VLEN; l++) s[l] = v0[l] + v1[l];
  sum = vsum8(s);
  for (; i < n; i++) sum += a[i] * b[i];
  return sum;
}

/* LlamaModel.MatVecMulF16 (LlamaModel.cs:570-598): dequantize the row, then a
 * sequential scalar dot. */
static float dot_f16_row(const uint8_t* row, const float* x, int n, float* buf) {
  for (int i = 0; i < n; i++) buf[i] = h2f(row + 2 * i);
  float dot = 0.0f;
  for (int i = 0; i < n; i++) dot += buf[i] * x[i];
  return dot;
}

/* ---------------------------------------------------------------------------
 * Q8_0 (DequantQ8_0.cs): fp16 d + 32 int8; value = (sbyte)q * d.
 * ------------------------------------------------------------------------- */

/* DequantQ8_0.Dequantize (DequantQ8_0.cs:18-41), partial last block included. */
void oracle_dequant_q8_0(const uint8_t* src, float* out, int n) {
  int blocks = (n + 31) / 32;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 34;
    float scale = h2f(blk);
    int count = n - 32 * b < 32 ? n - 32 * b : 32;
    for (int i = 0; i < count; i++) out[32 * b + i] = (float)(int8_t)blk[2 + i] * scale;
  }
}

/* DequantQ8_0.DotProductVec128 (DequantQ8_0.cs:51-90): acc0 takes lanes
 * i..i+3, acc1 lanes i+4..i+7 of each group of 8, as (v * scale) * x. */
float oracle_dot_q8_0(const uint8_t* row, const float* x, int n) {
  int blocks = n / 32;
  float acc0[4] = {0, 0, 0, 0}, acc1[4] = {0, 0, 0, 0};
  for (int b = 0; b < blocks; b++) {
    const uint8_t* src = row + (size_t)b * 34;
    const float* in = x + (size_t)b * 32;
    float scale = h2f(src);
    for (int i = 0; i < 32; i += 8)
      for (int l = 0; l < 4; l++) {
        acc0[l] = acc0[l] + ((float)(int8_t)src[2 + i + l] * scale) * in[i + l];
        acc1[l] = acc1[l] + ((float)(int8_t)src[2 + i + 4 + l] * scale) * in[i + 4 + l];
      }
  }
  float s[4];
  for (int l = 0; l < 4; l++) s[l] = acc0[l] + acc1[l];
  return vsum4(s);
}

/* ---------------------------------------------------------------------------
 * Q5_K (DequantQ5K.cs): d, dmin, 12 B scales/mins (Q4_K packing), qh[32] @16,
 * qs[128] @48 in Q4_K's nibble order; q5 = nibble | (bit e%8 of qh[e/8]) << 4,
 * value = d*sc[s]*q5 - dmin*m[s].
 * ------------------------------------------------------------------------- */
static inline int q5k_q(const uint8_t* blk, int e) {
  int s = e / 32, j = e % 32;
  int nib = j < 16 ? (blk[48 + 16 * s + j] & 0x0F) : ((blk[48 + 16 * s + j - 16] >> 4) & 0x0F);
  int hb = (blk[16 + e / 8] >> (e % 8)) & 1;
  return nib | (hb << 4);
}

/* DequantQ5K.Dequantize (DequantQ5K.cs:37-88). */
void oracle_dequant_q5_k(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 176;
    float d = h2f(blk + 0), dmin = h2f(blk + 2);
    int sc[8], m[8];
    q4k_scales(blk + 4, sc, m);
    for (int e = 0; e < 256; e++) {
      float dsc = d * (float)sc[e / 32], dm = dmin * (float)m[e / 32];
      out[(size_t)b * 256 + e] = dsc * (float)q5k_q(blk, e) - dm;
    }
  }
}

/* DequantQ5K.DotProductScalar (DequantQ5K.cs:97-151): one sequential sum per
 * super-block, added to the row sum. */
float oracle_dot_q5_k(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 176;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk + 0), dmin = h2f(blk + 2);
    int sc[8], m[8];
    q4k_scales(blk + 4, sc, m);
    float blockSum = 0.0f;
    for (int s = 0; s < 8; s++) {
      float dsc = d * (float)sc[s], dm = dmin * (float)m[s];
      for (int j = 0; j < 32; j++) {
        int e = 32 * s + j;
        blockSum = blockSum + (dsc * (float)q5k_q(blk, e) - dm) * in[e];
      }
    }
    sum = sum + blockSum;
  }
  return sum;
}

/* ---------------------------------------------------------------------------
 * Q4_1 (DequantQ4_1.cs): fp16 d, fp16 m, qs[16]; value = q*d + m (q unsigned
 * nibble, elements 0..15 low nibbles, 16..31 high nibbles).
 * ------------------------------------------------------------------------- */
static inline int nib32(const uint8_t* qs, int j) { return j < 16 ? (qs[j] & 0x0F) : ((qs[j - 16] >> 4) & 0x0F); }

/* DequantQ4_1.Dequantize (DequantQ4_1.cs:24-55), partial last block included. */
void oracle_dequant_q4_1(const uint8_t* src, float* out, int n) {
  int blocks = (n + 31) / 32;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 20;
    float d = h2f(blk), m = h2f(blk + 2);
    int count = n - 32 * b < 32 ? n - 32 * b : 32;
    for (int j = 0; j < count; j++) out[32 * b + j] = (float)nib32(blk + 4, j) * d + m;
  }
}

/* DequantQ4_1.DotProductVec128 (DequantQ4_1.cs:66-127): per block two 4-lane
 * accumulators (lanes of elements 0..3 / 8..11 / 16..19 / 24..27 into the
 * first, 4..7 / 12..15 / 20..23 / 28..31 into the second), each term
 * (q*d + m) * x, added to the row accumulators after the block. */
float oracle_dot_q4_1(const uint8_t* row, const float* x, int n) {
  int blocks = n / 32;
  float acc0[4] = {0, 0, 0, 0}, acc1[4] = {0, 0, 0, 0};
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 20;
    const float* in = x + (size_t)b * 32;
    float d = h2f(blk), m = h2f(blk + 2);
    float b0[4] = {0, 0, 0, 0}, b1[4] = {0, 0, 0, 0};
    for (int g = 0; g < 32; g += 8)
      for (int l = 0; l < 4; l++) {
        b0[l] = b0[l] + ((float)nib32(blk + 4, g + l) * d + m) * in[g + l];
        b1[l] = b1[l] + ((float)nib32(blk + 4, g + 4 + l) * d + m) * in[g + 4 + l];
      }
    for (int l = 0; l < 4; l++) {
      acc0[l] = acc0[l] + b0[l];
      acc1[l] = acc1[l] + b1[l];
    }
  }
  float s[4];
  for (int l = 0; l < 4; l++) s[l] = acc0[l] + acc1[l];
  return vsum4(s);
}

/* ---------------------------------------------------------------------------
 * Q5_0 / Q5_1 (DequantQ5_0.cs, DequantQ5_1.cs): q5 = nibble | bit j of the
 * little-endian qh word << 4; Q5_0 value = (q5 - 16) * d, Q5_1 q5 * d + m.
 * ------------------------------------------------------------------------- */
static inline int q5_32(const uint8_t* qh, const uint8_t* qs, int j) {
  uint32_t h = (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) | ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
  return nib32(qs, j) | (int)(((h >> j) & 1u) << 4);
}

/* DequantQ5_0.Dequantize (DequantQ5_0.cs:28-70). */
void oracle_dequant_q5_0(const uint8_t* src, float* out, int n) {
  int blocks = (n + 31) / 32;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 22;
    float d = h2f(blk);
    int count = n - 32 * b < 32 ? n - 32 * b : 32;
    for (int j = 0; j < count; j++) out[32 * b + j] = (float)(q5_32(blk + 2, blk + 6, j) - 16) * d;
  }
}

/* DequantQ5_0.DotProductScalar (DequantQ5_0.cs:79-118): the block's integer
 * (q5 - 16) * x terms summed in order, then sum += blockSum * d. */
float oracle_dot_q5_0(const uint8_t* row, const float* x, int n) {
  int blocks = n / 32;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 22;
    const float* in = x + (size_t)b * 32;
    float d = h2f(blk), bs = 0.0f;
    for (int j = 0; j < 32; j++) bs = bs + (float)(q5_32(blk + 2, blk + 6, j) - 16) * in[j];
    sum = sum + bs * d;
  }
  return sum;
}

/* DequantQ5_1.Dequantize (DequantQ5_1.cs:30-70). */
void oracle_dequant_q5_1(const uint8_t* src, float* out, int n) {
  int blocks = (n + 31) / 32;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 24;
    float d = h2f(blk), m = h2f(blk + 2);
    int count = n - 32 * b < 32 ? n - 32 * b : 32;
    for (int j = 0; j < count; j++) out[32 * b + j] = (float)q5_32(blk + 4, blk + 8, j) * d + m;
  }
}

/* DequantQ5_1.DotProductScalar (DequantQ5_1.cs:78-118): sum += blockSum * d +
 * inputSum * m per block, blockSum = sum of q5 * x, inputSum = sum of x. */
float oracle_dot_q5_1(const uint8_t* row, const float* x, int n) {
  int blocks = n / 32;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 24;
    const float* in = x + (size_t)b * 32;
    float d = h2f(blk), m = h2f(blk + 2), bs = 0.0f, is = 0.0f;
    for (int j = 0; j < 32; j++) {
      bs = bs + (float)q5_32(blk + 4, blk + 8, j) * in[j];
      is = is + in[j];
    }
    sum = sum + (bs * d + is * m); /* the right side first: sum += a + b */
  }
  return sum;
}

/* ---------------------------------------------------------------------------
 * Q2_K (DequantQ2K.cs): scales[16] @0 (low nibble scale, high nibble min per
 * 16 elements), qs[64] @16, d @80, dmin @82.  Element 128g + 32t + 16h + l
 * (g, h in {0,1}, t in 0..3, l < 16) is bits 2t..2t+1 of qs[32g + 16h + l]
 * with scale byte 8g + 2t + h; value = (d*sc) * q - dmin*m.
 * ------------------------------------------------------------------------- */
static inline void q2k_elem(const uint8_t* blk, int e, int* q, int* sb) {
  int g = e / 128, t = (e % 128) / 32, h = (e % 32) / 16, l = e % 16;
  *q = (blk[16 + 32 * g + 16 * h + l] >> (2 * t)) & 3;
  *sb = 8 * g + 2 * t + h;
}

/* DequantQ2K.Dequantize (DequantQ2K.cs:33-86). */
void oracle_dequant_q2_k(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 84;
    float d = h2f(blk + 80), dmin = h2f(blk + 82);
    for (int e = 0; e < 256; e++) {
      int q, sb;
      q2k_elem(blk, e, &q, &sb);
      float dl = d * (float)(blk[sb] & 0x0F), ml = dmin * (float)((blk[sb] >> 4) & 0x0F);
      out[(size_t)b * 256 + e] = dl * (float)q - ml;
    }
  }
}

/* DequantQ2K.DotProductScalar (DequantQ2K.cs:95-155): one sequential sum of
 * (dl*q - ml) * x per super-block in element order, added to the row sum. */
float oracle_dot_q2_k(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 84;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk + 80), dmin = h2f(blk + 82), bs = 0.0f;
    for (int e = 0; e < 256; e++) {
      int q, sb;
      q2k_elem(blk, e, &q, &sb);
      float dl = d * (float)(blk[sb] & 0x0F), ml = dmin * (float)((blk[sb] >> 4) & 0x0F);
      bs = bs + (dl * (float)q - ml) * in[e];
    }
    sum = sum + bs;
  }
  return sum;
}

/* ---------------------------------------------------------------------------
 * Q3_K (DequantQ3K.cs): hmask[32] @0, qs[64] @32, scales[12] @96, d @108.
 * Element i: q3 = (bits 2(i%4).. of qs[i/4]) | (bit i%8 of hmask[i/8]) << 2;
 * value = d * sc[i/16] * (q3 - 4), sc the signed 6-bit scales (low nibbles
 * of bytes 0..7 for 0..7, high nibbles for 8..15, two more bits from bytes
 * 8..11, minus 32).
 * ------------------------------------------------------------------------- */
static void q3k_scales(const uint8_t* p, int* sc) {
  for (int i = 0; i < 8; i++) {
    sc[i] = p[i] & 0x0F;
    sc[i + 8] = (p[i] >> 4) & 0x0F;
  }
  for (int i = 0; i < 4; i++) {
    int hb = p[8 + i];
    sc[i] |= (hb & 3) << 4;
    sc[i + 4] |= ((hb >> 2) & 3) << 4;
    sc[i + 8] |= ((hb >> 4) & 3) << 4;
    sc[i + 12] |= ((hb >> 6) & 3) << 4;
  }
  for (int i = 0; i < 16; i++) sc[i] -= 32;
}

static inline int q3k_q(const uint8_t* blk, int i) {
  return ((blk[32 + i / 4] >> (2 * (i % 4))) & 3) | (((blk[i / 8] >> (i % 8)) & 1) << 2);
}

/* DequantQ3K.Dequantize (DequantQ3K.cs:35-70, DecodeScales :122-150). */
void oracle_dequant_q3_k(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 110;
    float d = h2f(blk + 108);
    int sc[16];
    q3k_scales(blk + 96, sc);
    for (int i = 0; i < 256; i++) out[(size_t)b * 256 + i] = d * (float)sc[i / 16] * (float)(q3k_q(blk, i) - 4);
  }
}

/* DequantQ3K.DotProductScalar (DequantQ3K.cs:79-117): blockSum of the integer
 * sc * (q3 - 4) times x in element order, then sum += d * blockSum. */
float oracle_dot_q3_k(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 110;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk + 108), bs = 0.0f;
    int sc[16];
    q3k_scales(blk + 96, sc);
    for (int i = 0; i < 256; i++) bs = bs + (float)(sc[i / 16] * (q3k_q(blk, i) - 4)) * in[i];
    sum = sum + d * bs;
  }
  return sum;
}

/* ---------------------------------------------------------------------------
 * Q8_K (DequantQ8K.cs): fp32 d @0, int8 qs[256] @4, int16 bsums[16] @260
 * (not read); value = (sbyte)q * d.
 * ------------------------------------------------------------------------- */
static inline float f32_at(const uint8_t* p) {
  float f;
  memcpy(&f, p, 4);
  return f;
}

/* DequantQ8K.Dequantize (DequantQ8K.cs:26-51). */
void oracle_dequant_q8_k(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 292;
    float d = f32_at(blk);
    for (int i = 0; i < 256; i++) out[(size_t)b * 256 + i] = (float)(int8_t)blk[4 + i] * d;
  }
}

/* DequantQ8K.DotProductVec128 (DequantQ8K.cs:62-101): lanes of elements
 * 8k..8k+3 into acc0, 8k+4..8k+7 into acc1, each term (q * d) * x. */
float oracle_dot_q8_k(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float acc0[4] = {0, 0, 0, 0}, acc1[4] = {0, 0, 0, 0};
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 292;
    const float* in = x + (size_t)b * 256;
    float d = f32_at(blk);
    for (int i = 0; i < 256; i += 8)
      for (int l = 0; l < 4; l++) {
        acc0[l] = acc0[l] + ((float)(int8_t)blk[4 + i + l] * d) * in[i + l];
        acc1[l] = acc1[l] + ((float)(int8_t)blk[4 + i + 4 + l] * d) * in[i + 4 + l];
      }
  }
  float s[4];
  for (int l = 0; l < 4; l++) s[l] = acc0[l] + acc1[l];
  return vsum4(s);
}

/* ---------------------------------------------------------------------------
 * IQ family (DequantIQ.cs).  The reference's own decoders: bit fields with
 * small scales and no codebook grids (they do not decode llama.cpp's IQ
 * files).  Restated as written, their quirks included:
 *   IQ4_XS takes the low scale of sub-block s from byte 4+s (s < 8: bytes 8..11
 *     are the first quants), masked to 6 bits, and 2 more bits from scales_h
 *     placed at bits 6..7 (DequantIQ.cs:155-159);
 *   IQ3_S reads its sign bytes at 98..129 and its scale bytes at 130..137 of a
 *     110-byte block (DequantIQ.cs:255-283): a row's last block reads the first
 *     28 bytes of the next row, and the tensor's last block 28 bytes past its
 *     end (the wrapper in oracle.py appends zeros there, as the device copy's
 *     tail padding holds); its Dequantize over one embedding row therefore
 *     indexes past the row's span, which the reference reports as an
 *     IndexOutOfRangeException (load_embedding returns -5);
 *   IQ2_S negates only elements 0..3 of a 16-element sub-block (:677-678).
 * ------------------------------------------------------------------------- */

/* DequantIQ.IQ4NL_Table (DequantIQ.cs:29-33). */
static const float kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* IQ4NL.Dequantize (DequantIQ.cs:46-76), partial last block included. */
void oracle_dequant_iq4_nl(const uint8_t* src, float* out, int n) {
  int blocks = (n + 31) / 32;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 18;
    float d = h2f(blk);
    int rem = n - 32 * b;
    for (int j = 0; j < 16 && j < rem; j++) out[32 * b + j] = d * kIQ4NL[blk[2 + j] & 0x0F];
    for (int j = 0; j < 16 && 16 + j < rem; j++) out[32 * b + 16 + j] = d * kIQ4NL[(blk[2 + j] >> 4) & 0x0F];
  }
}

/* IQ4NL.DotProductScalar (DequantIQ.cs:85-125): the low nibbles' terms, then
 * the high nibbles', into one block sum; sum += blockSum * scale. */
float oracle_dot_iq4_nl(const uint8_t* row, const float* x, int n) {
  int blocks = n / 32;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 18;
    const float* in = x + (size_t)b * 32;
    float d = h2f(blk), bs = 0.0f;
    for (int j = 0; j < 16; j++) bs = bs + kIQ4NL[blk[2 + j] & 0x0F] * in[j];
    for (int j = 0; j < 16; j++) bs = bs + kIQ4NL[(blk[2 + j] >> 4) & 0x0F] * in[16 + j];
    sum = sum + bs * d;
  }
  return sum;
}

static inline int iq4xs_scale(const uint8_t* blk, int sub) {
  int sh = blk[2] | (blk[3] << 8);
  return ((blk[4 + sub] & 0x3F) | (((sh >> (2 * sub)) & 3) << 6)) - 32;
}

/* IQ4XS.Dequantize (DequantIQ.cs:139-176). */
void oracle_dequant_iq4_xs(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 136;
    float d = h2f(blk);
    for (int sub = 0; sub < 8; sub++) {
      float dsc = d * (float)iq4xs_scale(blk, sub);
      for (int j = 0; j < 16; j++) {
        uint8_t q = blk[8 + 16 * sub + j];
        out[(size_t)b * 256 + 32 * sub + j] = dsc * kIQ4NL[q & 0x0F];
        out[(size_t)b * 256 + 32 * sub + j + 16] = dsc * kIQ4NL[(q >> 4) & 0x0F];
      }
    }
  }
}

/* IQ4XS.DotProductScalar (DequantIQ.cs:184-234): per sub-block the low and
 * high nibble terms alternate; blockSum += dsc * subSum; sum += blockSum. */
float oracle_dot_iq4_xs(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 136;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 8; sub++) {
      float dsc = d * (float)iq4xs_scale(blk, sub), ss = 0.0f;
      for (int j = 0; j < 16; j++) {
        uint8_t q = blk[8 + 16 * sub + j];
        ss = ss + kIQ4NL[q & 0x0F] * in[32 * sub + j];
        ss = ss + kIQ4NL[(q >> 4) & 0x0F] * in[32 * sub + j + 16];
      }
      bs = bs + dsc * ss;
    }
    sum = sum + bs;
  }
  return sum;
}

/* IQ3_S element idx of the block at blk: the unsigned 3-bit magnitude and the
 * sign bit (byte 98 + idx/8, bit idx%8), the scale (byte 130 + idx/32) . */
static inline int iq3s_q(const uint8_t* blk, int idx) {
  return ((blk[2 + idx / 4] >> (2 * (idx % 4))) & 3) | (((blk[66 + idx / 8] >> (idx % 8)) & 1) << 2);
}
static inline int iq3s_sc(const uint8_t* blk, int sub) { return ((blk[130 + sub / 4] >> (2 * (sub % 4))) & 3) + 1; }

/* IQ3S.Dequantize (DequantIQ.cs:244-290). */
void oracle_dequant_iq3_s(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 110;
    float d = h2f(blk);
    for (int sub = 0; sub < 32; sub++) {
      float dsc = d * (float)iq3s_sc(blk, sub);
      uint8_t sb = blk[98 + sub];
      for (int j = 0; j < 8; j++) {
        int idx = 8 * sub + j;
        float val = dsc * (float)iq3s_q(blk, idx);
        if ((sb >> j) & 1) val = -val;
        out[(size_t)b * 256 + idx] = val;
      }
    }
  }
}

/* IQ3S.DotProductScalar (DequantIQ.cs:299-349). */
float oracle_dot_iq3_s(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 110;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 32; sub++) {
      float dsc = d * (float)iq3s_sc(blk, sub), ss = 0.0f;
      uint8_t sb = blk[98 + sub];
      for (int j = 0; j < 8; j++) {
        float val = (float)iq3s_q(blk, 8 * sub + j);
        if ((sb >> j) & 1) val = -val;
        ss = ss + val * in[8 * sub + j];
      }
      bs = bs + dsc * ss;
    }
    sum = sum + bs;
  }
  return sum;
}

static inline int iq3xxs_q(const uint8_t* blk, int idx) {
  const uint8_t* p = blk + 2 + 3 * (idx / 8);
  uint32_t packed = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16);
  return (int)((packed >> (3 * (idx % 8))) & 7);
}

/* IQ3XXS.Dequantize (DequantIQ.cs:364-399): d * (q3 - 4). */
void oracle_dequant_iq3_xxs(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 98;
    float d = h2f(blk);
    for (int i = 0; i < 256; i++) out[(size_t)b * 256 + i] = d * (float)(iq3xxs_q(blk, i) - 4);
  }
}

/* IQ3XXS.DotProductScalar (DequantIQ.cs:408-447). */
float oracle_dot_iq3_xxs(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 98;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int i = 0; i < 256; i++) bs = bs + (float)(iq3xxs_q(blk, i) - 4) * in[i];
    sum = sum + d * bs;
  }
  return sum;
}

/* IQ2 element e of a 16-element sub-block sub: bits 2(e%4) of qs[4 sub + e/4]. */
static inline int iq2_q(const uint8_t* blk, int sub, int e) { return (blk[2 + 4 * sub + e / 4] >> (2 * (e % 4))) & 3; }
static inline int iq2xs_sc(const uint8_t* blk, int sub) {
  int raw = (int8_t)blk[66 + sub / 2];
  return (sub & 1) == 0 ? (raw & 0x0F) - 8 : ((raw >> 4) & 0x0F) - 8;
}

/* IQ2XS.Dequantize (DequantIQ.cs:456-496): dsc * (q - 1). */
void oracle_dequant_iq2_xs(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 74;
    float d = h2f(blk);
    for (int sub = 0; sub < 16; sub++) {
      float dsc = d * (float)iq2xs_sc(blk, sub);
      for (int e = 0; e < 16; e++) out[(size_t)b * 256 + 16 * sub + e] = dsc * (float)(iq2_q(blk, sub, e) - 1);
    }
  }
}

/* IQ2XS.DotProductScalar (DequantIQ.cs:505-559). */
float oracle_dot_iq2_xs(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 74;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 16; sub++) {
      float dsc = d * (float)iq2xs_sc(blk, sub), ss = 0.0f;
      for (int e = 0; e < 16; e++) ss = ss + (float)(iq2_q(blk, sub, e) - 1) * in[16 * sub + e];
      bs = bs + dsc * ss;
    }
    sum = sum + bs;
  }
  return sum;
}

/* IQ2XXS.Dequantize (DequantIQ.cs:568-598): d * (q - 1). */
void oracle_dequant_iq2_xxs(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 66;
    float d = h2f(blk);
    for (int sub = 0; sub < 16; sub++)
      for (int e = 0; e < 16; e++) out[(size_t)b * 256 + 16 * sub + e] = d * (float)(iq2_q(blk, sub, e) - 1);
  }
}

/* IQ2XXS.DotProductScalar (DequantIQ.cs:607-647). */
float oracle_dot_iq2_xxs(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 66;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 16; sub++)
      for (int e = 0; e < 16; e++) bs = bs + (float)(iq2_q(blk, sub, e) - 1) * in[16 * sub + e];
    sum = sum + d * bs;
  }
  return sum;
}

/* IQ2S.Dequantize (DequantIQ.cs:656-696): dsc * q, elements 0..3 of a
 * sub-block negated by the sign nibble of qh[sub]. */
void oracle_dequant_iq2_s(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 82;
    float d = h2f(blk);
    for (int sub = 0; sub < 16; sub++) {
      uint8_t qh = blk[66 + sub];
      float dsc = d * (float)((qh & 0x0F) + 1);
      int sign = (qh >> 4) & 0x0F;
      for (int e = 0; e < 16; e++) {
        float val = dsc * (float)iq2_q(blk, sub, e);
        if (e < 4 && ((sign >> e) & 1)) val = -val;
        out[(size_t)b * 256 + 16 * sub + e] = val;
      }
    }
  }
}

/* IQ2S.DotProductScalar (DequantIQ.cs:705-758). */
float oracle_dot_iq2_s(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 82;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 16; sub++) {
      uint8_t qh = blk[66 + sub];
      float dsc = d * (float)((qh & 0x0F) + 1), ss = 0.0f;
      int sign = (qh >> 4) & 0x0F;
      for (int e = 0; e < 16; e++) {
        float val = (float)iq2_q(blk, sub, e);
        if (e < 4 && ((sign >> e) & 1)) val = -val;
        ss = ss + val * in[16 * sub + e];
      }
      bs = bs + dsc * ss;
    }
    sum = sum + bs;
  }
  return sum;
}

/* IQ1 ternary element j of 8-element sub-block sub: +1 if bit j of qs[sub],
 * else -1 if bit (sub%2)*4 + j/2 of qh[sub/2], else 0. */
static inline int iq1_t(const uint8_t* blk, int sub, int j) {
  if ((blk[2 + sub] >> j) & 1) return 1;
  return ((blk[34 + sub / 2] >> ((sub % 2) * 4 + j / 2)) & 1) ? -1 : 0;
}

/* IQ1S.Dequantize (DequantIQ.cs:767-805): d, -d or 0. */
void oracle_dequant_iq1_s(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 50;
    float d = h2f(blk);
    for (int sub = 0; sub < 32; sub++)
      for (int j = 0; j < 8; j++) {
        int t = iq1_t(blk, sub, j);
        out[(size_t)b * 256 + 8 * sub + j] = t == 1 ? d : (t == -1 ? -d : 0.0f);
      }
  }
}

/* IQ1S.DotProductScalar (DequantIQ.cs:814-860). */
float oracle_dot_iq1_s(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 50;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 32; sub++)
      for (int j = 0; j < 8; j++) bs = bs + (float)iq1_t(blk, sub, j) * in[8 * sub + j];
    sum = sum + d * bs;
  }
  return sum;
}

/* IQ1_M sub-block scale: bit sub%8 of scales[sub/8] selects 1 or 0.5
 * (DequantIQ.cs:884-890; sub/8 < 4 < 6 always). */
static inline float iq1m_sc(const uint8_t* blk, int sub) {
  int idx = sub / 8;
  if (idx >= 6) return 1.0f;
  return ((blk[50 + idx] >> (sub % 8)) & 1) ? 1.0f : 0.5f;
}

/* IQ1M.Dequantize (DequantIQ.cs:869-914): d*sc, -d*sc or 0. */
void oracle_dequant_iq1_m(const uint8_t* src, float* out, int n) {
  int blocks = n / 256;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = src + (size_t)b * 56;
    float d = h2f(blk);
    for (int sub = 0; sub < 32; sub++) {
      float sc = iq1m_sc(blk, sub);
      for (int j = 0; j < 8; j++) {
        int t = iq1_t(blk, sub, j);
        out[(size_t)b * 256 + 8 * sub + j] = t == 1 ? d * sc : (t == -1 ? -d * sc : 0.0f);
      }
    }
  }
}

/* IQ1M.DotProductScalar (DequantIQ.cs:923-975). */
float oracle_dot_iq1_m(const uint8_t* row, const float* x, int n) {
  int blocks = n / 256;
  float sum = 0.0f;
  for (int b = 0; b < blocks; b++) {
    const uint8_t* blk = row + (size_t)b * 56;
    const float* in = x + (size_t)b * 256;
    float d = h2f(blk), bs = 0.0f;
    for (int sub = 0; sub < 32; sub++) {
      float sc = iq1m_sc(blk, sub);
      for (int j = 0; j < 8; j++) {
        int t = iq1_t(blk, sub, j);
        float w = t == 1 ? sc : (t == -1 ? -sc : 0.0f);
        bs = bs + w * in[8 * sub + j];
      }
    }
    sum = sum + d * bs;
  }
  return sum;
}

/* TensorMath.MatVecMulQ4_0 / MatVecMulQ6K / MatVecMulGeneric / MatVecMul
 * (TensorMath.cs:527-656) dispatched as LlamaModel.MatVecMulByType
 * (LlamaModel.cs:470-567).  Rows are independent (TensorMath.cs:47-51), so the
 * thread count never changes a result. */
int oracle_matvec(uint32_t type, const void* W, const float* x, float* y, int M, int K) {
  const uint8_t* w = (const uint8_t*)W;
  size_t bpr;
  float (*dot)(const uint8_t*, const float*, int) = NULL;
  switch (type) {
    case ORACLE_Q4_0: bpr = (size_t)(K / 32) * 18; dot = oracle_dot_q4_0; break;
    case ORACLE_Q4_K: bpr = (size_t)(K / 256) * 144; dot = oracle_dot_q4_k; break;
    case ORACLE_Q6_K: bpr = (size_t)(K / 256) * 210; dot = oracle_dot_q6_k; break;
    case ORACLE_Q8_0: bpr = (size_t)(K / 32) * 34; dot = oracle_dot_q8_0; break;
    case ORACLE_Q5_K: bpr = (size_t)(K / 256) * 176; dot = oracle_dot_q5_k; break;
    case ORACLE_Q4_1: bpr = (size_t)(K / 32) * 20; dot = oracle_dot_q4_1; break;
    case ORACLE_Q5_0: bpr = (size_t)(K / 32) * 22; dot = oracle_dot_q5_0; break;
    case ORACLE_Q5_1: bpr = (size_t)(K / 32) * 24; dot = oracle_dot_q5_1; break;
    case ORACLE_Q2_K: bpr = (size_t)(K / 256) * 84; dot = oracle_dot_q2_k; break;
    case ORACLE_Q3_K: bpr = (size_t)(K / 256) * 110; dot = oracle_dot_q3_k; break;
    case ORACLE_Q8_K: bpr = (size_t)(K / 256) * 292; dot = oracle_dot_q8_k; break;
    case ORACLE_IQ2_XXS: bpr = (size_t)(K / 256) * 66; dot = oracle_dot_iq2_xxs; break;
    case ORACLE_IQ2_XS: bpr = (size_t)(K / 256) * 74; dot = oracle_dot_iq2_xs; break;
    case ORACLE_IQ3_XXS: bpr = (size_t)(K / 256) * 98; dot = oracle_dot_iq3_xxs; break;
    case ORACLE_IQ1_S: bpr = (size_t)(K / 256) * 50; dot = oracle_dot_iq1_s; break;
    case ORACLE_IQ4_NL: bpr = (size_t)(K / 32) * 18; dot = oracle_dot_iq4_nl; break;
    case ORACLE_IQ3_S: bpr = (size_t)(K / 256) * 110; dot = oracle_dot_iq3_s; break;
    case ORACLE_IQ2_S: bpr = (size_t)(K / 256) * 82; dot = oracle_dot_iq2_s; break;
    case ORACLE_IQ4_XS: bpr = (size_t)(K / 256) * 136; dot = oracle_dot_iq4_xs; break;
    case ORACLE_IQ1_M: bpr = (size_t)(K / 256) * 56; dot = oracle_dot_iq1_m; break;
    case ORACLE_F32: {
      const float* wf = (const float*)W;
      for (int r = 0; r < M; r++) y[r] = oracle_dot_f32(wf + (size_t)r * K, x, K);
      return 0;
    }
    case ORACLE_F16: {
      float* buf = (float*)malloc(sizeof(float) * (size_t)K);
      for (int r = 0; r < M; r++) y[r] = dot_f16_row(w + (size_t)r * K * 2, x, K, buf);
      free(buf);
      return 0;
    }
    default: return -3;
  }
  if (M >= PARALLEL_ROW_THRESHOLD && g_threads > 1) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int r = 0; r < M; r++) y[r] = dot(w + (size_t)r * bpr, x, K);
  } else {
    for (int r = 0; r < M; r++) y[r] = dot(w + (size_t)r * bpr, x, K);
  }
  return 0;
}

/* TensorMath.RmsNorm (TensorMath.cs:97-165). */
void oracle_rmsnorm(const float* x, const float* w, float* out, int n, float eps) {
  float sumSq = 0.0f;
  int i = 0;
  if (n >= VLEN) {
    float a0[VLEN] = {0}, a1[VLEN] = {0};
    int lim2 = n - 2 * VLEN + 1;
    for (; i < lim2; i += 2 * VLEN)
      for (int l = 0; l < VLEN; l++) {
        a0[l] = a0[l] + x[i + l] * x[i + l];
        a1[l] = a1[l] + x[i + VLEN + l] * x[i + VLEN + l];
      }
    int lim1 = n - VLEN + 1;
    for (; i < lim1; i += VLEN)
      for (int l = 0; l < VLEN; l++) a0[l] = a0[l] + x[i + l] * x[i + l];
    float s[VLEN];
    for (int l = 0; l < VLEN; l++) s[l] = a0[l] + a1[l];
    sumSq = vsum8(s);
  }
  for (; i < n; i++) sumSq += x[i] * x[i];
  float rms = 1.0f / sqrtf(sumSq / (float)n + eps); /* :142 */
  for (i = 0; i < n; i++) out[i] = x[i] * rms * w[i]; /* :155, :162 */
}

/* TensorMath.Softmax (TensorMath.cs:177-241). */
void oracle_softmax(float* d, int n) {
  float mx = -INFINITY;
  for (int i = 0; i < n; i++)
    if (d[i] > mx) mx = d[i];
  float sum = 0.0f;
  for (int i = 0; i < n; i++) {
    float v = expf(d[i] - mx);
    d[i] = v;
    sum += v;
  }
  if (sum > 0.0f) {
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) d[i] = d[i] * inv;
  }
}

/* TensorMath.SiluElementwiseMul (TensorMath.cs:253-286). */
void oracle_silu_mul(float* gate, const float* up, int n) {
  for (int i = 0; i < n; i++) {
    float xv = gate[i];
    gate[i] = (xv / (1.0f + expf(-xv))) * up[i];
  }
}

/* TensorMath.Add (TensorMath.cs:712-733). */
void oracle_add(float* a, const float* b, int n) {
  for (int i = 0; i < n; i++) a[i] = a[i] + b[i];
}

/* TensorMath.ApplyRoPE (TensorMath.cs:408-458), rotaryDim = headDim. */
void oracle_rope(float* q, float* k, int position, int hd, int nh, int nkv, float base) {
  float negLogBase = -logf(base);
  float dimInv = 1.0f / (float)hd;
  for (int pass = 0; pass < 2; pass++) {
    float* v = pass == 0 ? q : k;
    int heads = pass == 0 ? nh : nkv;
    for (int h = 0; h < heads; h++) {
      float* vec = v + (size_t)h * hd;
      for (int i = 0; i < hd; i += 2) {
        float theta = (float)position * expf((float)i * dimInv * negLogBase);
        float c = cosf(theta), s = sinf(theta);
        float x0 = vec[i], x1 = vec[i + 1];
        vec[i] = x0 * c - x1 * s;
        vec[i + 1] = x0 * s + x1 * c;
      }
    }
  }
}

/* TensorMath.ApplyRoPENeox (TensorMath.cs:475-520), rotaryDim = headDim:
 * element i of a head is rotated with element i + hd/2 by
 * theta = pos * exp(i * (2/hd) * -ln base). */
void oracle_rope_neox(float* q, float* k, int position, int hd, int nh, int nkv, float base) {
  float negLogBase = -logf(base);
  float dimInv = 2.0f / (float)hd;
  int half = hd / 2;
  for (int pass = 0; pass < 2; pass++) {
    float* v = pass == 0 ? q : k;
    int heads = pass == 0 ? nh : nkv;
    for (int h = 0; h < heads; h++) {
      float* vec = v + (size_t)h * hd;
      for (int i = 0; i < half; i++) {
        float theta = (float)position * expf((float)i * dimInv * negLogBase);
        float c = cosf(theta), s = sinf(theta);
        float x0 = vec[i], x1 = vec[i + half];
        vec[i] = x0 * c - x1 * s;
        vec[i + half] = x1 * c + x0 * s;
      }
    }
  }
}

/* GreedySampler.Sample (GreedySampler.cs:13-26): first maximum wins. */
int oracle_argmax(const float* logits, int n) {
  int best = 0;
  float bv = logits[0];
  for (int i = 1; i < n; i++)
    if (logits[i] > bv) {
      bv = logits[i];
      best = i;
    }
  return best;
}

/* ---------------------------------------------------------------------------
 * System.Random(int seed) (TemperatureSampler.cs:29 constructs it; :97 draws
 * NextDouble once per Sample).  The generator lives in the .NET BCL (net10.0,
 * ChatNet.Core.csproj:3), which the reference does not vendor; a seeded
 * Random keeps the compat implementation: Knuth's subtractive method as in
 * Numerical Recipes in C (2nd ed.) "ran3", MBIG = int.MaxValue,
 * MSEED = 161803398, 55-entry table with lags 21/55, NextDouble =
 * InternalSample * (1.0 / MBIG).  Restated from that published algorithm.
 * ------------------------------------------------------------------------- */
#define NR_MBIG 2147483647
#define NR_MSEED 161803398

void oracle_net_random_init(oracle_net_random* r, int32_t seed) {
  int32_t subtraction = seed == INT32_MIN ? INT32_MAX : (seed < 0 ? -seed : seed);
  int32_t mj = NR_MSEED - subtraction;
  r->seed_array[0] = 0;
  r->seed_array[55] = mj;
  int32_t mk = 1;
  for (int i = 1; i < 55; i++) {
    int ii = (21 * i) % 55;
    r->seed_array[ii] = mk;
    mk = mj - mk;
    if (mk < 0) mk += NR_MBIG;
    mj = r->seed_array[ii];
  }
  for (int k = 1; k < 5; k++)
    for (int i = 1; i < 56; i++) {
      r->seed_array[i] -= r->seed_array[1 + (i + 30) % 55];
      if (r->seed_array[i] < 0) r->seed_array[i] += NR_MBIG;
    }
  r->inext = 0;
  r->inextp = 21;
}

int32_t oracle_net_random_sample(oracle_net_random* r) {
  int32_t a = r->inext, b = r->inextp;
  if (++a >= 56) a = 1;
  if (++b >= 56) b = 1;
  int32_t v = r->seed_array[a] - r->seed_array[b];
  if (v == NR_MBIG) v--;
  if (v < 0) v += NR_MBIG;
  r->seed_array[a] = v;
  r->inext = a;
  r->inextp = b;
  return v;
}

double oracle_net_random_next_double(oracle_net_random* r) {
  return oracle_net_random_sample(r) * (1.0 / NR_MBIG);
}

/* ---------------------------------------------------------------------------
 * TemperatureSampler (TemperatureSampler.cs:33-222)
 * ------------------------------------------------------------------------- */
static void ts_swap(float* p, int* idx, int a, int b) { /* :167-172 */
  float t = p[a];
  p[a] = p[b];
  p[b] = t;
  int u = idx[a];
  idx[a] = idx[b];
  idx[b] = u;
}

/* PartialSortDescending (:118-165): median-of-three quickselect. */
static void ts_partial_sort(float* p, int* idx, int left, int right, int k) {
  while (left < right) {
    int mid = left + (right - left) / 2;
    if (p[mid] > p[left]) ts_swap(p, idx, left, mid);
    if (p[right] > p[left]) ts_swap(p, idx, left, right);
    if (p[mid] > p[right]) ts_swap(p, idx, mid, right);
    float pivot = p[right];
    int store = left;
    for (int i = left; i < right; i++)
      if (p[i] > pivot) {
        ts_swap(p, idx, i, store);
        store++;
      }
    ts_swap(p, idx, store, right);
    if (store == k - 1) return;
    if (store < k - 1) left = store + 1;
    else right = store - 1;
  }
}

/* InsertionSortDescending (:177-194). */
static void ts_insertion_sort(float* p, int* idx, int count) {
  for (int i = 1; i < count; i++) {
    float kp = p[i];
    int ki = idx[i];
    int j = i - 1;
    while (j >= 0 && p[j] < kp) {
      p[j + 1] = p[j];
      idx[j + 1] = idx[j];
      j--;
    }
    p[j + 1] = kp;
    idx[j + 1] = ki;
  }
}

static float fminabs(float m, float d) {
  d = fabsf(d);
  return d < m ? d : m;
}

int oracle_temperature_sample(const float* logits, int n, float temperature, int top_k, float top_p, float r,
                              float* margin) {
  float mg = INFINITY;
  if (temperature <= 0.0f) { /* :37-41 */
    if (margin) *margin = mg;
    return oracle_argmax(logits, n);
  }
  if (top_k < 1) return -1;
  float* p = (float*)malloc(sizeof(float) * (size_t)n);
  int* idx = (int*)malloc(sizeof(int) * (size_t)n);
  float invTemp = 1.0f / temperature; /* :50-55 */
  for (int i = 0; i < n; i++) {
    p[i] = logits[i] * invTemp;
    idx[i] = i;
  }
  oracle_softmax(p, n); /* :58 */
  int k = top_k < n ? top_k : n; /* :62-63 */
  /* the k-th / (k+1)-th gap decides the set, relative to the k-th (a copy
   * keeps p's order intact) */
  if (k < n) {
    float* s = (float*)malloc(sizeof(float) * (size_t)n);
    int* si = (int*)malloc(sizeof(int) * (size_t)n);
    memcpy(s, p, sizeof(float) * (size_t)n);
    memcpy(si, idx, sizeof(int) * (size_t)n);
    ts_partial_sort(s, si, 0, n - 1, k + 1);
    ts_insertion_sort(s, si, k + 1);
    if (s[k - 1] > 0.0f) mg = fminabs(mg, (s[k - 1] - s[k]) / s[k - 1]);
    free(s);
    free(si);
  }
  ts_partial_sort(p, idx, 0, n - 1, k);
  ts_insertion_sort(p, idx, k); /* :67 */
  float cumulative = 0.0f; /* :70-80 */
  int cutoff = k;
  for (int i = 0; i < k; i++) {
    cumulative += p[i];
    mg = fminabs(mg, cumulative - top_p);
    if (cumulative >= top_p) {
      cutoff = i + 1;
      break;
    }
  }
  float sum = 0.0f; /* :83-92 */
  for (int i = 0; i < cutoff; i++) sum += p[i];
  float invSum = 1.0f / sum;
  for (int i = 0; i < cutoff; i++) p[i] *= invSum;
  float acc = 0.0f; /* :95-106 */
  int tok = idx[cutoff - 1];
  for (int i = 0; i < cutoff; i++) {
    acc += p[i];
    mg = fminabs(mg, r - acc);
    if (r < acc) {
      tok = idx[i];
      break;
    }
  }
  free(p);
  free(idx);
  if (margin) *margin = mg;
  return tok;
}

/* ---------------------------------------------------------------------------
 * Llama model (LlamaModel.cs, LlamaWeights.cs)
 * ------------------------------------------------------------------------- */

typedef struct tensor_ref {
  const void* data;
  uint32_t type;
} tensor_ref;

struct oracle_llama {
  oracle_config c;
  int kv_dim, kv_mul;
  tensor_ref emb, out, out_norm;
  tensor_ref *attn_norm, *ffn_norm, *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const float **bq, **bk, **bv; /* QwenWeights' optional biases (QwenWeights.cs:158-170) */
  float *kcache, *vcache;
  float *x, *xn, *q, *k, *v, *att, *gate, *up, *ffo, *scores, *rowbuf;
};

oracle_llama* oracle_llama_create(const oracle_config* cfg) {
  oracle_llama* m = (oracle_llama*)calloc(1, sizeof(oracle_llama));
  if (!m) return NULL;
  m->c = *cfg;
  int L = cfg->n_layers;
  m->kv_dim = cfg->n_kv_heads * cfg->head_dim; /* LlamaConfig.cs:34 */
  m->kv_mul = cfg->n_heads / cfg->n_kv_heads;  /* LlamaConfig.cs:37 */
  tensor_ref** arrs[] = {&m->attn_norm, &m->ffn_norm, &m->wq, &m->wk, &m->wv,
                         &m->wo,        &m->wg,       &m->wu, &m->wd};
  for (size_t i = 0; i < sizeof(arrs) / sizeof(arrs[0]); i++)
    *arrs[i] = (tensor_ref*)calloc((size_t)L, sizeof(tensor_ref));
  m->bq = (const float**)calloc((size_t)L, sizeof(float*));
  m->bk = (const float**)calloc((size_t)L, sizeof(float*));
  m->bv = (const float**)calloc((size_t)L, sizeof(float*));
  size_t kv = (size_t)L * cfg->context_length * m->kv_dim; /* LlamaModel.cs:60-61 */
  m->kcache = (float*)calloc(kv, sizeof(float));
  m->vcache = (float*)calloc(kv, sizeof(float));
  int dim = cfg->dim, hid = cfg->hidden_dim;
  m->x = (float*)calloc((size_t)dim, 4);
  m->xn = (float*)calloc((size_t)dim, 4);
  m->q = (float*)calloc((size_t)dim, 4);
  m->k = (float*)calloc((size_t)m->kv_dim, 4);
  m->v = (float*)calloc((size_t)m->kv_dim, 4);
  m->att = (float*)calloc((size_t)dim, 4);
  m->gate = (float*)calloc((size_t)hid, 4);
  m->up = (float*)calloc((size_t)hid, 4);
  m->ffo = (float*)calloc((size_t)dim, 4);
  m->scores = (float*)calloc((size_t)cfg->context_length, 4);
  m->rowbuf = (float*)calloc((size_t)(dim > hid ? dim : hid), 4);
  if (!m->kcache || !m->vcache) {
    oracle_llama_destroy(m);
    return NULL;
  }
  return m;
}

/* Name resolution of LlamaWeights.ResolveAll (LlamaWeights.cs:78-145), and for
 * ORACLE_ARCH_QWEN2 the F32 q/k/v biases of QwenWeights (QwenWeights.cs:158-170). */
int oracle_llama_set_tensor(oracle_llama* m, const char* name, uint32_t type, const void* data) {
  tensor_ref t = {data, type};
  if (!strcmp(name, "token_embd.weight")) { m->emb = t; return 0; }
  if (!strcmp(name, "output.weight")) { m->out = t; return 0; }
  if (!strcmp(name, "output_norm.weight")) { m->out_norm = t; return 0; }
  int l;
  char suffix[64];
  if (sscanf(name, "blk.%d.%63s", &l, suffix) != 2 || l < 0 || l >= m->c.n_layers) return -2;
  struct { const char* s; tensor_ref* a; } tab[] = {
      {"attn_norm.weight", m->attn_norm}, {"ffn_norm.weight", m->ffn_norm},
      {"attn_q.weight", m->wq},           {"attn_k.weight", m->wk},
      {"attn_v.weight", m->wv},           {"attn_output.weight", m->wo},
      {"ffn_gate.weight", m->wg},         {"ffn_up.weight", m->wu},
      {"ffn_down.weight", m->wd}};
  for (size_t i = 0; i < sizeof(tab) / sizeof(tab[0]); i++)
    if (!strcmp(suffix, tab[i].s)) {
      tab[i].a[l] = t;
      return 0;
    }
  if (m->c.arch == ORACLE_ARCH_QWEN2) {
    const float** b = !strcmp(suffix, "attn_q.bias")   ? m->bq
                      : !strcmp(suffix, "attn_k.bias") ? m->bk
                      : !strcmp(suffix, "attn_v.bias") ? m->bv
                                                       : NULL;
    if (b) {
      if (type != ORACLE_F32) return -3;
      b[l] = (const float*)data;
      return 0;
    }
  }
  return -2;
}

/* LlamaModel.LoadEmbedding (LlamaModel.cs:365-394): F32 copy, F16 per
 * element, any quantized type through its Dequantize (GetDequantInfo,
 * LlamaModel.cs:399-467) on the token's row. */
static int load_embedding(oracle_llama* m, int token, float* out) {
  int dim = m->c.dim;
  const uint8_t* e = (const uint8_t*)m->emb.data;
  switch (m->emb.type) {
    case ORACLE_F32: memcpy(out, e + (size_t)token * dim * 4, (size_t)dim * 4); return 0;
    case ORACLE_F16:
      for (int i = 0; i < dim; i++) out[i] = h2f(e + ((size_t)token * dim + i) * 2);
      return 0;
    case ORACLE_Q4_0: oracle_dequant_q4_0(e + (size_t)token * (dim / 32) * 18, out, dim); return 0;
    case ORACLE_Q8_0: oracle_dequant_q8_0(e + (size_t)token * (dim / 32) * 34, out, dim); return 0;
    case ORACLE_Q4_1: oracle_dequant_q4_1(e + (size_t)token * (dim / 32) * 20, out, dim); return 0;
    case ORACLE_Q5_0: oracle_dequant_q5_0(e + (size_t)token * (dim / 32) * 22, out, dim); return 0;
    case ORACLE_Q5_1: oracle_dequant_q5_1(e + (size_t)token * (dim / 32) * 24, out, dim); return 0;
    case ORACLE_Q2_K: oracle_dequant_q2_k(e + (size_t)token * (dim / 256) * 84, out, dim); return 0;
    case ORACLE_Q3_K: oracle_dequant_q3_k(e + (size_t)token * (dim / 256) * 110, out, dim); return 0;
    case ORACLE_Q4_K: oracle_dequant_q4_k(e + (size_t)token * (dim / 256) * 144, out, dim); return 0;
    case ORACLE_Q5_K: oracle_dequant_q5_k(e + (size_t)token * (dim / 256) * 176, out, dim); return 0;
    case ORACLE_Q6_K: oracle_dequant_q6_k(e + (size_t)token * (dim / 256) * 210, out, dim); return 0;
    case ORACLE_Q8_K: oracle_dequant_q8_k(e + (size_t)token * (dim / 256) * 292, out, dim); return 0;
    case ORACLE_IQ2_XXS: oracle_dequant_iq2_xxs(e + (size_t)token * (dim / 256) * 66, out, dim); return 0;
    case ORACLE_IQ2_XS: oracle_dequant_iq2_xs(e + (size_t)token * (dim / 256) * 74, out, dim); return 0;
    case ORACLE_IQ3_XXS: oracle_dequant_iq3_xxs(e + (size_t)token * (dim / 256) * 98, out, dim); return 0;
    case ORACLE_IQ1_S: oracle_dequant_iq1_s(e + (size_t)token * (dim / 256) * 50, out, dim); return 0;
    case ORACLE_IQ4_NL: oracle_dequant_iq4_nl(e + (size_t)token * (dim / 32) * 18, out, dim); return 0;
    case ORACLE_IQ2_S: oracle_dequant_iq2_s(e + (size_t)token * (dim / 256) * 82, out, dim); return 0;
    case ORACLE_IQ4_XS: oracle_dequant_iq4_xs(e + (size_t)token * (dim / 256) * 136, out, dim); return 0;
    case ORACLE_IQ1_M: oracle_dequant_iq1_m(e + (size_t)token * (dim / 256) * 56, out, dim); return 0;
    case ORACLE_IQ3_S: return -5; /* IQ3S.Dequantize indexes past the row's span (DequantIQ.cs:266, :280) */
    default: return -3;
  }
}

/* LlamaModel.ComputeAttention (LlamaModel.cs:241-346). */
static void attention(oracle_llama* m, int layer, int pos) {
  int hd = m->c.head_dim, kvd = m->kv_dim, ctx = m->c.context_length;
  size_t loff = (size_t)layer * ctx * kvd;
  int seq = pos + 1;
  float scale = 1.0f / sqrtf((float)hd);
  memset(m->att, 0, sizeof(float) * (size_t)m->c.dim);
  for (int h = 0; h < m->c.n_heads; h++) {
    const float* qp = m->q + (size_t)h * hd;
    int kvh = h / m->kv_mul;
    for (int p = 0; p < seq; p++) {
      const float* kp = m->kcache + loff + (size_t)p * kvd + (size_t)kvh * hd;
      float score = 0.0f;
      int d = 0;
      if (hd >= VLEN) {
        float a0[VLEN] = {0}, a1[VLEN] = {0};
        int lim = hd - 2 * VLEN + 1;
        for (; d < lim; d += 2 * VLEN)
          for (int l = 0; l < VLEN; l++) {
            a0[l] = a0[l] + qp[d + l] * kp[d + l];
            a1[l] = a1[l] + qp[d + VLEN + l] * kp[d + VLEN + l];
          }
        int lim1 = hd - VLEN + 1;
        for (; d < lim1; d += VLEN)
          for (int l = 0; l < VLEN; l++) a0[l] = a0[l] + qp[d + l] * kp[d + l];
        float s[VLEN];
        for (int l = 0; l < VLEN; l++) s[l] = a0[l] + a1[l];
        score = vsum8(s);
      }
      for (; d < hd; d++) score += qp[d] * kp[d];
      m->scores[p] = score * scale;
    }
    oracle_softmax(m->scores, seq);
    float* op = m->att + (size_t)h * hd;
    for (int p = 0; p < seq; p++) {
      float w = m->scores[p];
      if (w == 0.0f) continue; /* :322 */
      const float* vp = m->vcache + loff + (size_t)p * kvd + (size_t)kvh * hd;
      for (int d = 0; d < hd; d++) op[d] = op[d] + vp[d] * w;
    }
  }
}

/* LlamaModel.Forward (LlamaModel.cs:93-238); MistralModel.Forward
 * (MistralModel.cs:67-154) is the same computation.  ORACLE_ARCH_QWEN2 is
 * QwenModel.Forward (QwenModel.cs:69-178): biases added after the q/k/v
 * projections (:104-120), split-half RoPE (:124-126). */
int oracle_llama_forward(oracle_llama* m, const int32_t* tokens, int n, int position, float* logits) {
  const oracle_config* c = &m->c;
  int dim = c->dim, kvd = m->kv_dim, hid = c->hidden_dim;
  const tensor_ref* out = m->out.data ? &m->out : &m->emb; /* LlamaWeights.cs:89-98 */
  if (!m->emb.data || !m->out_norm.data) return -2;
  for (int t = 0; t < n; t++) {
    int pos = position + t;
    if (tokens[t] < 0 || tokens[t] >= c->vocab_size || pos < 0 || pos >= c->context_length) return -5;
    int rc = load_embedding(m, tokens[t], m->x);
    if (rc) return rc;
    for (int l = 0; l < c->n_layers; l++) {
      if (!m->wq[l].data || !m->wk[l].data || !m->wv[l].data || !m->wo[l].data || !m->wg[l].data ||
          !m->wu[l].data || !m->wd[l].data || !m->attn_norm[l].data || !m->ffn_norm[l].data)
        return -2;
      oracle_rmsnorm(m->x, (const float*)m->attn_norm[l].data, m->xn, dim, c->rms_norm_eps);
      if ((rc = oracle_matvec(m->wq[l].type, m->wq[l].data, m->xn, m->q, dim, dim))) return rc;
      if ((rc = oracle_matvec(m->wk[l].type, m->wk[l].data, m->xn, m->k, kvd, dim))) return rc;
      if ((rc = oracle_matvec(m->wv[l].type, m->wv[l].data, m->xn, m->v, kvd, dim))) return rc;
      if (c->arch == ORACLE_ARCH_QWEN2) {
        if (m->bq[l]) {
          if (!m->bk[l] || !m->bv[l]) return -2; /* GetTensorPointer throws for the missing one */
          for (int i = 0; i < dim; i++) m->q[i] += m->bq[l][i];
          for (int i = 0; i < kvd; i++) m->k[i] += m->bk[l][i];
          for (int i = 0; i < kvd; i++) m->v[i] += m->bv[l][i];
        }
        oracle_rope_neox(m->q, m->k, pos, c->head_dim, c->n_heads, c->n_kv_heads, c->rope_freq_base);
      } else {
        oracle_rope(m->q, m->k, pos, c->head_dim, c->n_heads, c->n_kv_heads, c->rope_freq_base);
      }
      size_t off = (size_t)l * c->context_length * kvd + (size_t)pos * kvd; /* :150-153 */
      memcpy(m->kcache + off, m->k, sizeof(float) * (size_t)kvd);
      memcpy(m->vcache + off, m->v, sizeof(float) * (size_t)kvd);
      attention(m, l, pos);
      if ((rc = oracle_matvec(m->wo[l].type, m->wo[l].data, m->att, m->ffo, dim, dim))) return rc;
      oracle_add(m->x, m->ffo, dim);
      oracle_rmsnorm(m->x, (const float*)m->ffn_norm[l].data, m->xn, dim, c->rms_norm_eps);
      if ((rc = oracle_matvec(m->wg[l].type, m->wg[l].data, m->xn, m->gate, hid, dim))) return rc;
      if ((rc = oracle_matvec(m->wu[l].type, m->wu[l].data, m->xn, m->up, hid, dim))) return rc;
      oracle_silu_mul(m->gate, m->up, hid);
      if ((rc = oracle_matvec(m->wd[l].type, m->wd[l].data, m->gate, m->ffo, dim, hid))) return rc;
      oracle_add(m->x, m->ffo, dim);
    }
    oracle_rmsnorm(m->x, (const float*)m->out_norm.data, m->xn, dim, c->rms_norm_eps);
    if (t == n - 1 && logits) { /* :207 — LM head only for the last token */
      if ((rc = oracle_matvec(out->type, out->data, m->xn, logits, c->vocab_size, dim))) return rc;
    }
  }
  return 0;
}

int oracle_llama_kv(oracle_llama* m, int layer, int position, int which, float* out) {
  if (layer < 0 || layer >= m->c.n_layers || position < 0 || position >= m->c.context_length) return -5;
  size_t off = (size_t)layer * m->c.context_length * m->kv_dim + (size_t)position * m->kv_dim;
  memcpy(out, (which ? m->vcache : m->kcache) + off, sizeof(float) * (size_t)m->kv_dim);
  return 0;
}

void oracle_llama_destroy(oracle_llama* m) {
  if (!m) return;
  free(m->attn_norm); free(m->ffn_norm); free(m->wq); free(m->wk); free(m->wv);
  free(m->wo); free(m->wg); free(m->wu); free(m->wd);
  free(m->bq); free(m->bk); free(m->bv);
  free(m->kcache); free(m->vcache);
  free(m->x); free(m->xn); free(m->q); free(m->k); free(m->v); free(m->att);
  free(m->gate); free(m->up); free(m->ffo); free(m->scores); free(m->rowbuf);
  free(m);
}
