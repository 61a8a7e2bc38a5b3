/*
 * synth.c — seeded synthetic weights and GGUF block quantizers
 * (libchatnet_synth.so, host only).
 *
 * Produces the raw bytes of a random-init Llama checkpoint in the block
 * layouts ChatNet decodes:
 *   Q4_0  DequantQ4_0.cs:9-22      fp16 d, 16 B nibbles; element j<16 = low
 *                                  nibble of qs[j], element 16+j = high nibble
 *   Q4_K  DequantQ4K.cs:11-34,59-72 fp16 d, fp16 dmin, 12 B 6-bit scales/mins
 *                                  (get_scale_min_k4 packing), 128 B qs where
 *                                  sub-block s owns qs[16s..16s+15] (low nibbles
 *                                  = elements 32s..32s+15, high = 32s+16..31)
 *   Q6_K  DequantQ6K.cs:11-32,53-83 ql[128], qh[64], int8 scales[16], fp16 d
 *   Q8_0  DequantQ8_0.cs:7-16      fp16 d, 32 int8
 *   Q5_K  DequantQ5K.cs:7-34,58-83 fp16 d, fp16 dmin, 12 B scales/mins, qh[32]
 *                                  (bit e%8 of qh[e/8] = bit 4 of element e),
 *                                  qs[128] in Q4_K's nibble order
 *   Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q8_K and the IQ family as the reference's
 *                                  dequantizers read them (DequantQ4_1.cs ..
 *                                  DequantQ8K.cs, DequantIQ.cs)
 * Every element is a pure function of (seed, stream, index): a splitmix64
 * counter hash feeds a Box-Muller transform, so any tensor can be regenerated
 * bit-identically, in any order, on any number of threads.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

static inline uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* FNV-1a of a tensor name: the per-tensor stream id. */
EXPORT uint64_t chatnet_synth_stream_id(const char* name) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (const unsigned char* p = (const unsigned char*)name; *p; p++) {
    h ^= *p;
    h *= 0x100000001B3ull;
  }
  return h;
}

/* Normal pair for pair index `pair` of stream (seed, stream). */
static inline void normal_pair(uint64_t key, uint64_t pair, double* z0, double* z1) {
  uint64_t a = splitmix64(key + 2 * pair), b = splitmix64(key + 2 * pair + 1);
  double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
  double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0, 1) */
  double r = sqrt(-2.0 * log(u1));
  double t = 6.283185307179586476925286766559 * u2;
  *z0 = r * cos(t);
  *z1 = r * sin(t);
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return splitmix64(seed * 0x9E3779B97F4A7C15ull ^ splitmix64(stream));
}

/* out[i] = sigma * N(0,1) for element index start+i of the stream. */
EXPORT void chatnet_synth_normal(uint64_t seed, uint64_t stream, uint64_t start, uint64_t n, float sigma,
                                 float* out) {
  uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < (int64_t)((n + 4095) / 4096); c++) {
    uint64_t i0 = (uint64_t)c * 4096, i1 = i0 + 4096 < n ? i0 + 4096 : n;
    for (uint64_t i = i0; i < i1;) {
      uint64_t e = start + i;
      double z0, z1;
      normal_pair(key, e >> 1, &z0, &z1);
      if (e & 1) {
        out[i++] = (float)(z1 * sigma);
      } else {
        out[i++] = (float)(z0 * sigma);
        if (i < i1) out[i++] = (float)(z1 * sigma);
      }
    }
  }
}

/* Uniform token ids in [0, vocab). */
EXPORT void chatnet_synth_tokens(uint64_t seed, uint64_t stream, int n, int vocab, int32_t* out) {
  uint64_t key = stream_key(seed, stream);
  for (int i = 0; i < n; i++) out[i] = (int32_t)(splitmix64(key + (uint64_t)i) % (uint64_t)vocab);
}

/* fp32 -> IEEE binary16, round to nearest even (subnormals, overflow to inf). */
EXPORT uint16_t chatnet_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal half */
    if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25 rounds to 0 */
    /* value = m * 2^(e-150); in units of 2^-24 that is m >> (126 - e), 14 <= shift <= 24 */
    uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    int shift = 126 - (int)e;
    uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (ax >> 23) - 127 + 15, m = ax & 0x7FFFFFu;
  uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
  return (uint16_t)(sign | q);
}

static float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
  if (exp == 0) {
    if (!man) bits = sign;
    else {
      int e = -1;
      do { man <<= 1; e++; } while (!(man & 0x400));
      bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FF) << 13);
    }
  } else if (exp == 31) bits = sign | 0x7F800000u | (man << 13);
  else bits = sign | ((exp + 112) << 23) | (man << 13);
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline int nearest_int(float f) { return (int)lrintf(f); }

/* Q4_0: d = amax / -8 (amax = the element of largest magnitude, sign kept),
 * q = min(15, (int)(w/d + 8.5)), w ~= (q - 8) * d. */
static void quant_block_q4_0(const float* w, uint8_t* out) {
  float amax = 0.f, mx = 0.f;
  for (int j = 0; j < 32; j++)
    if (fabsf(w[j]) > amax) { amax = fabsf(w[j]); mx = w[j]; }
  float d = mx / -8.0f, id = d != 0.f ? 1.0f / d : 0.f;
  put16(out, chatnet_float_to_half(d));
  for (int j = 0; j < 16; j++) {
    int q0 = (int)(w[j] * id + 8.5f), q1 = (int)(w[16 + j] * id + 8.5f);
    if (q0 > 15) q0 = 15;
    if (q1 > 15) q1 = 15;
    out[2 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

/* Q4_K: per 32-element sub-block, scale = (max - min) / 15 and offset
 * -min(0, min); both quantized to 6 bits against fp16 d / dmin; then
 * q = round((w + dmin*m) / (d*sc)) clamped to [0, 15]. */
static void quant_block_q4_k(const float* w, uint8_t* out) {
  float scale[8], mins[8], ms = 0.f, mm = 0.f;
  for (int s = 0; s < 8; s++) {
    float lo = 0.f, hi = w[32 * s];
    for (int j = 0; j < 32; j++) {
      float v = w[32 * s + j];
      if (v < lo) lo = v;
      if (v > hi) hi = v;
    }
    if (hi < lo) hi = lo;
    scale[s] = (hi - lo) / 15.0f;
    mins[s] = -lo;
    if (scale[s] > ms) ms = scale[s];
    if (mins[s] > mm) mm = mins[s];
  }
  uint16_t dh = chatnet_float_to_half(ms / 63.0f), mh = chatnet_float_to_half(mm / 63.0f);
  float d = half_to_float(dh), dmin = half_to_float(mh);
  int sc[8], m[8];
  for (int s = 0; s < 8; s++) {
    sc[s] = d > 0.f ? nearest_int(scale[s] / d) : 0;
    m[s] = dmin > 0.f ? nearest_int(mins[s] / dmin) : 0;
    if (sc[s] > 63) sc[s] = 63;
    if (sc[s] < 0) sc[s] = 0;
    if (m[s] > 63) m[s] = 63;
    if (m[s] < 0) m[s] = 0;
  }
  put16(out, dh);
  put16(out + 2, mh);
  uint8_t* q = out + 4;
  for (int j = 0; j < 4; j++) {
    q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    q[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  for (int s = 0; s < 8; s++) {
    float ds = d * (float)sc[s], dm = dmin * (float)m[s];
    for (int j = 0; j < 16; j++) {
      int q0 = 0, q1 = 0;
      if (ds > 0.f) {
        q0 = nearest_int((w[32 * s + j] + dm) / ds);
        q1 = nearest_int((w[32 * s + 16 + j] + dm) / ds);
      }
      q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
      q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
      out[16 + 16 * s + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

/* Q6_K: per 16-element group, scale = -(element of largest magnitude) / 32
 * (so signed int8 scales occur), quantized to int8 against fp16
 * d = max|scale| / 127; q = round(w / (d*sc)) clamped to [-32, 31], stored +32. */
static void quant_block_q6_k(const float* w, uint8_t* out) {
  float scale[16], amax_all = 0.f;
  for (int g = 0; g < 16; g++) {
    float amax = 0.f, mx = 0.f;
    for (int j = 0; j < 16; j++)
      if (fabsf(w[16 * g + j]) > amax) { amax = fabsf(w[16 * g + j]); mx = w[16 * g + j]; }
    scale[g] = -mx / 32.0f;
    if (fabsf(scale[g]) > amax_all) amax_all = fabsf(scale[g]);
  }
  uint16_t dh = chatnet_float_to_half(amax_all / 127.0f);
  float d = half_to_float(dh);
  int8_t sc[16];
  for (int g = 0; g < 16; g++) {
    int v = d > 0.f ? nearest_int(scale[g] / d) : 0;
    if (v > 127) v = 127;
    if (v < -128) v = -128;
    sc[g] = (int8_t)v;
  }
  uint8_t L[256];
  for (int e = 0; e < 256; e++) {
    float den = d * (float)sc[e / 16];
    int q = den != 0.f ? nearest_int(w[e] / den) : 0;
    if (q < -32) q = -32;
    if (q > 31) q = 31;
    L[e] = (uint8_t)(q + 32);
  }
  uint8_t* ql = out;
  uint8_t* qh = out + 128;
  memset(out, 0, 210);
  for (int h = 0; h < 2; h++)
    for (int l = 0; l < 32; l++) {
      const uint8_t* b = L + 128 * h;
      uint8_t q1 = b[l], q2 = b[l + 32], q3 = b[l + 64], q4 = b[l + 96];
      ql[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      ql[64 * h + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  memcpy(out + 192, sc, 16);
  put16(out + 208, dh);
}

/* Q8_0: d = max|w| / 127 as fp16, q = round(w / d) clamped to [-127, 127]. */
static void quant_block_q8_0(const float* w, uint8_t* out) {
  float amax = 0.f;
  for (int j = 0; j < 32; j++)
    if (fabsf(w[j]) > amax) amax = fabsf(w[j]);
  uint16_t dh = chatnet_float_to_half(amax / 127.0f);
  float d = half_to_float(dh), id = d != 0.f ? 1.0f / d : 0.f;
  put16(out, dh);
  for (int j = 0; j < 32; j++) {
    int q = nearest_int(w[j] * id);
    if (q > 127) q = 127;
    if (q < -127) q = -127;
    out[2 + j] = (uint8_t)(int8_t)q;
  }
}

/* Q5_K: as Q4_K with 5-bit quants (scale = (max - min) / 31), written in the
 * reference's layout (DequantQ5K.cs:30-34, :58-83): d, dmin, 12 scale bytes,
 * qh[32] with the high bit of element e at qh[e/8] bit e%8, qs[128] where
 * sub-block s keeps elements 32s+j / 32s+16+j in the low / high nibble of
 * qs[16s+j]. */
static void quant_block_q5_k(const float* w, uint8_t* out) {
  float scale[8], mins[8], ms = 0.f, mm = 0.f;
  for (int s = 0; s < 8; s++) {
    float lo = 0.f, hi = w[32 * s];
    for (int j = 0; j < 32; j++) {
      float v = w[32 * s + j];
      if (v < lo) lo = v;
      if (v > hi) hi = v;
    }
    if (hi < lo) hi = lo;
    scale[s] = (hi - lo) / 31.0f;
    mins[s] = -lo;
    if (scale[s] > ms) ms = scale[s];
    if (mins[s] > mm) mm = mins[s];
  }
  uint16_t dh = chatnet_float_to_half(ms / 63.0f), mh = chatnet_float_to_half(mm / 63.0f);
  float d = half_to_float(dh), dmin = half_to_float(mh);
  int sc[8], m[8];
  for (int s = 0; s < 8; s++) {
    sc[s] = d > 0.f ? nearest_int(scale[s] / d) : 0;
    m[s] = dmin > 0.f ? nearest_int(mins[s] / dmin) : 0;
    if (sc[s] > 63) sc[s] = 63;
    if (sc[s] < 0) sc[s] = 0;
    if (m[s] > 63) m[s] = 63;
    if (m[s] < 0) m[s] = 0;
  }
  memset(out, 0, 176);
  put16(out, dh);
  put16(out + 2, mh);
  uint8_t* q = out + 4;
  for (int j = 0; j < 4; j++) {
    q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    q[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  uint8_t* qh = out + 16;
  uint8_t* qs = out + 48;
  for (int s = 0; s < 8; s++) {
    float ds = d * (float)sc[s], dm = dmin * (float)m[s];
    for (int j = 0; j < 32; j++) {
      int e = 32 * s + j;
      int v = ds > 0.f ? nearest_int((w[e] + dm) / ds) : 0;
      v = v < 0 ? 0 : (v > 31 ? 31 : v);
      if (j < 16) qs[16 * s + j] |= (uint8_t)(v & 0xF);
      else qs[16 * s + j - 16] |= (uint8_t)((v & 0xF) << 4);
      if (v & 16) qh[e / 8] |= (uint8_t)(1u << (e % 8));
    }
  }
}

/* Q4_1: d = (max - min) / 15, m = min (both fp16), q = round((w - m) / d)
 * clamped to [0, 15]; element j < 16 in the low nibble of qs[j], 16 + j in the
 * high nibble. */
static void quant_block_q4_1(const float* w, uint8_t* out) {
  float lo = w[0], hi = w[0];
  for (int j = 1; j < 32; j++) {
    if (w[j] < lo) lo = w[j];
    if (w[j] > hi) hi = w[j];
  }
  uint16_t dh = chatnet_float_to_half((hi - lo) / 15.0f), mh = chatnet_float_to_half(lo);
  float d = half_to_float(dh), m = half_to_float(mh), id = d != 0.f ? 1.0f / d : 0.f;
  put16(out, dh);
  put16(out + 2, mh);
  for (int j = 0; j < 16; j++) {
    int q0 = nearest_int((w[j] - m) * id), q1 = nearest_int((w[16 + j] - m) * id);
    q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
    q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
    out[4 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

/* Q5_0 / Q5_1: 5-bit quants, the low nibble in qs (Q4_0's order) and bit 4
 * of element j in bit j of the little-endian qh word.  Q5_0: d = amax / -16
 * (sign of the largest-magnitude element kept), q = round(w/d) + 16 in
 * [0, 31]; Q5_1: d = (max - min) / 31, m = min, q = round((w - m) / d). */
static void put_q5(const int* q, uint8_t* qh, uint8_t* qs) {
  uint32_t h = 0;
  for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 0xF) | ((q[16 + j] & 0xF) << 4));
  for (int j = 0; j < 32; j++) h |= (uint32_t)((q[j] >> 4) & 1) << j;
  qh[0] = (uint8_t)h;
  qh[1] = (uint8_t)(h >> 8);
  qh[2] = (uint8_t)(h >> 16);
  qh[3] = (uint8_t)(h >> 24);
}

static void quant_block_q5_0(const float* w, uint8_t* out) {
  float amax = 0.f, mx = 0.f;
  for (int j = 0; j < 32; j++)
    if (fabsf(w[j]) > amax) { amax = fabsf(w[j]); mx = w[j]; }
  uint16_t dh = chatnet_float_to_half(mx / -16.0f);
  float d = half_to_float(dh), id = d != 0.f ? 1.0f / d : 0.f;
  int q[32];
  for (int j = 0; j < 32; j++) {
    int v = nearest_int(w[j] * id) + 16;
    q[j] = v < 0 ? 0 : (v > 31 ? 31 : v);
  }
  put16(out, dh);
  put_q5(q, out + 2, out + 6);
}

static void quant_block_q5_1(const float* w, uint8_t* out) {
  float lo = w[0], hi = w[0];
  for (int j = 1; j < 32; j++) {
    if (w[j] < lo) lo = w[j];
    if (w[j] > hi) hi = w[j];
  }
  uint16_t dh = chatnet_float_to_half((hi - lo) / 31.0f), mh = chatnet_float_to_half(lo);
  float d = half_to_float(dh), m = half_to_float(mh), id = d != 0.f ? 1.0f / d : 0.f;
  int q[32];
  for (int j = 0; j < 32; j++) {
    int v = nearest_int((w[j] - m) * id);
    q[j] = v < 0 ? 0 : (v > 31 ? 31 : v);
  }
  put16(out, dh);
  put16(out + 2, mh);
  put_q5(q, out + 4, out + 8);
}

/* Q2_K (the reference's layout, DequantQ2K.cs:15-20, :55-82): per 16-element
 * sub-block sb, scale (max - min) / 3 and offset -min(0, min), both 4-bit
 * against fp16 d / dmin; element 128g + 32t + 16h + l is bits 2t..2t+1 of
 * qs[32g + 16h + l] with scale byte sb = 8g + 2t + h (low nibble scale, high
 * nibble min). */
static void quant_block_q2_k(const float* w, uint8_t* out) {
  float scale[16], mins[16], ms = 0.f, mm = 0.f;
  for (int sb = 0; sb < 16; sb++) {
    int g = sb / 8, t = (sb % 8) / 2, h = sb % 2, e0 = 128 * g + 32 * t + 16 * h;
    float lo = 0.f, hi = w[e0];
    for (int l = 0; l < 16; l++) {
      if (w[e0 + l] < lo) lo = w[e0 + l];
      if (w[e0 + l] > hi) hi = w[e0 + l];
    }
    if (hi < lo) hi = lo;
    scale[sb] = (hi - lo) / 3.0f;
    mins[sb] = -lo;
    if (scale[sb] > ms) ms = scale[sb];
    if (mins[sb] > mm) mm = mins[sb];
  }
  uint16_t dh = chatnet_float_to_half(ms / 15.0f), mh = chatnet_float_to_half(mm / 15.0f);
  float d = half_to_float(dh), dmin = half_to_float(mh);
  memset(out, 0, 84);
  for (int sb = 0; sb < 16; sb++) {
    int sc = d > 0.f ? nearest_int(scale[sb] / d) : 0, m = dmin > 0.f ? nearest_int(mins[sb] / dmin) : 0;
    sc = sc < 0 ? 0 : (sc > 15 ? 15 : sc);
    m = m < 0 ? 0 : (m > 15 ? 15 : m);
    out[sb] = (uint8_t)(sc | (m << 4));
    int g = sb / 8, t = (sb % 8) / 2, h = sb % 2, e0 = 128 * g + 32 * t + 16 * h;
    float dl = d * (float)sc, ml = dmin * (float)m;
    for (int l = 0; l < 16; l++) {
      int q = dl > 0.f ? nearest_int((w[e0 + l] + ml) / dl) : 0;
      q = q < 0 ? 0 : (q > 3 ? 3 : q);
      out[16 + 32 * g + 16 * h + l] |= (uint8_t)(q << (2 * t));
    }
  }
  put16(out + 80, dh);
  put16(out + 82, mh);
}

/* Q3_K (the reference's layout, DequantQ3K.cs:9-21, :52-63): per 16-element
 * sub-block a signed 6-bit scale sc = round(-amax / 4 / d) (d = max|scale| /
 * 31 as fp16), q3 = round(w / (d*sc)) + 4 in [0, 7]; element i keeps bits 0-1
 * in qs[i/4] at 2(i%4) and bit 2 in hmask[i/8] bit i%8; scales stored + 32,
 * low nibbles in bytes 0..7 (sc 0..7 low, 8..15 high), two high bits per
 * scale in bytes 8..11. */
static void quant_block_q3_k(const float* w, uint8_t* out) {
  float scale[16], amax_all = 0.f;
  for (int sb = 0; sb < 16; sb++) {
    float amax = 0.f, mx = 0.f;
    for (int l = 0; l < 16; l++)
      if (fabsf(w[16 * sb + l]) > amax) { amax = fabsf(w[16 * sb + l]); mx = w[16 * sb + l]; }
    scale[sb] = -mx / 4.0f;
    if (fabsf(scale[sb]) > amax_all) amax_all = fabsf(scale[sb]);
  }
  uint16_t dh = chatnet_float_to_half(amax_all / 31.0f);
  float d = half_to_float(dh);
  memset(out, 0, 110);
  int sc[16];
  for (int sb = 0; sb < 16; sb++) {
    int v = d > 0.f ? nearest_int(scale[sb] / d) : 0;
    sc[sb] = v < -32 ? -32 : (v > 31 ? 31 : v);
  }
  for (int i = 0; i < 256; i++) {
    float den = d * (float)sc[i / 16];
    int q = den != 0.f ? nearest_int(w[i] / den) + 4 : 4;
    q = q < 0 ? 0 : (q > 7 ? 7 : q);
    out[32 + i / 4] |= (uint8_t)((q & 3) << (2 * (i % 4)));
    out[i / 8] |= (uint8_t)(((q >> 2) & 1) << (i % 8));
  }
  uint8_t* s = out + 96;
  for (int i = 0; i < 16; i++) {
    int u = sc[i] + 32;
    if (i < 8) s[i] |= (uint8_t)(u & 0xF);
    else s[i - 8] |= (uint8_t)((u & 0xF) << 4);
    s[8 + i % 4] |= (uint8_t)(((u >> 4) & 3) << (2 * (i / 4)));
  }
  put16(out + 108, dh);
}

/* Q8_K: fp32 d = max|w| / 127, q = round(w / d) in [-127, 127], then the 16
 * int16 block sums the format carries. */
static void quant_block_q8_k(const float* w, uint8_t* out) {
  float amax = 0.f;
  for (int i = 0; i < 256; i++)
    if (fabsf(w[i]) > amax) amax = fabsf(w[i]);
  float d = amax / 127.0f, id = d != 0.f ? 1.0f / d : 0.f;
  memcpy(out, &d, 4);
  for (int g = 0; g < 16; g++) {
    int sum = 0;
    for (int l = 0; l < 16; l++) {
      int q = nearest_int(w[16 * g + l] * id);
      q = q < -127 ? -127 : (q > 127 ? 127 : q);
      out[4 + 16 * g + l] = (uint8_t)(int8_t)q;
      sum += q;
    }
    out[260 + 2 * g] = (uint8_t)(sum & 0xFF);
    out[261 + 2 * g] = (uint8_t)((sum >> 8) & 0xFF);
  }
}

/* ---------------------------------------------------------------------------
 * The IQ family as the reference decodes it (DequantIQ.cs: bit fields, no
 * codebooks).  Each encoder picks, per weight, the nearest value the decoder
 * can produce under the fields it has already fixed.
 * ------------------------------------------------------------------------- */
static const float kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static int nearest_iq4(float v, float dsc) {
  int best = 0;
  float be = INFINITY;
  for (int q = 0; q < 16; q++) {
    float e = fabsf(dsc * kIQ4NL[q] - v);
    if (e < be) { be = e; best = q; }
  }
  return best;
}

static float signed_amax(const float* w, int n) {
  float a = 0.f;
  for (int i = 0; i < n; i++)
    if (fabsf(w[i]) > fabsf(a)) a = w[i];
  return a;
}

/* IQ4_NL (DequantIQ.cs:46-76): d = -amax/127, so the largest weight lands on
 * table[0]; elements j<16 low nibbles, 16+j high nibbles of qs[j]. */
static void quant_block_iq4_nl(const float* w, uint8_t* out) {
  uint16_t dh = chatnet_float_to_half(-signed_amax(w, 32) / 127.0f);
  float d = half_to_float(dh);
  put16(out, dh);
  for (int j = 0; j < 16; j++)
    out[2 + j] = (uint8_t)(nearest_iq4(w[j], d) | (nearest_iq4(w[16 + j], d) << 4));
}

/* IQ4_XS (DequantIQ.cs:139-176): sub-block s's scale is (byte 4+s & 63 |
 * 2 bits of scales_h << 6) - 32, and bytes 8..11 are also the first quants of
 * sub-block 0.  Sub-blocks 0..3 get their scale freely; sub-block 0 is
 * quantized next, which fixes the low 6 bits of the scales of 4..7, whose
 * high bits are then chosen nearest to the wanted scale. */
static void quant_block_iq4_xs(const float* w, uint8_t* out) {
  float amax = 0.f, want[8];
  for (int s = 0; s < 8; s++) {
    want[s] = fabsf(signed_amax(w + 32 * s, 32));
    if (want[s] > amax) amax = want[s];
  }
  uint16_t dh = chatnet_float_to_half(amax / (113.0f * 190.0f));
  float d = half_to_float(dh);
  memset(out, 0, 136);
  put16(out, dh);
  int sh = 0;
  for (int s = 0; s < 8; s++) {
    /* positive scales: the table's end on the largest weight's side (113 or -127) meets it */
    float sa = signed_amax(w + 32 * s, 32);
    int sc = d > 0.f ? nearest_int(fabsf(sa) / (sa > 0.f ? 113.0f : 127.0f) / d) : 0;
    if (s < 4) {
      int v = sc + 32;
      v = v < 0 ? 0 : (v > 255 ? 255 : v);
      out[4 + s] = (uint8_t)(v & 63);
      sh |= (v >> 6) << (2 * s);
    } else {
      int low = out[4 + s] & 63, best = 0, be = 1 << 30;
      for (int hi = 0; hi < 4; hi++) {
        int e = abs((low | (hi << 6)) - 32 - sc);
        if (e < be) { be = e; best = hi; }
      }
      sh |= best << (2 * s);
    }
    put16(out + 2, (uint16_t)sh);
    int scv = ((out[4 + s] & 63) | (((sh >> (2 * s)) & 3) << 6)) - 32;
    float dsc = d * (float)scv;
    for (int j = 0; j < 16; j++) {
      int lo = nearest_iq4(w[32 * s + j], dsc), hi = nearest_iq4(w[32 * s + 16 + j], dsc);
      out[8 + 16 * s + j] = (uint8_t)(lo | (hi << 4));
    }
  }
}

/* IQ3_S (DequantIQ.cs:244-290): value +-(d*sc)*q3; the signs of sub-blocks
 * 12..31 and all eight scale bytes are bytes 0..27 of the next block (`next`,
 * zeros past the tensor), fixed before this block is encoded; own sign bytes
 * (sub-blocks 0..11) follow the weights. */
static void quant_block_iq3_s(const float* w, uint8_t* out, const uint8_t* next) {
  int sc[32];
  float need = 0.f;
  for (int s = 0; s < 32; s++) {
    sc[s] = ((next[20 + s / 4] >> (2 * (s % 4))) & 3) + 1;
    float a = fabsf(signed_amax(w + 8 * s, 8)) / (7.0f * (float)sc[s]);
    if (a > need) need = a;
  }
  uint16_t dh = chatnet_float_to_half(need);
  float d = half_to_float(dh);
  memset(out, 0, 110);
  put16(out, dh);
  for (int s = 0; s < 32; s++) {
    uint8_t sb;
    if (s < 12) {
      sb = 0;
      for (int j = 0; j < 8; j++) sb |= (uint8_t)((w[8 * s + j] < 0.f) << j);
      out[98 + s] = sb;
    } else {
      sb = next[s - 12];
    }
    float dsc = d * (float)sc[s];
    for (int j = 0; j < 8; j++) {
      int idx = 8 * s + j, neg = (sb >> j) & 1;
      float v = w[idx];
      int q = 0;
      if (dsc > 0.f && ((v < 0.f) == (neg != 0))) {
        q = nearest_int(fabsf(v) / dsc);
        q = q > 7 ? 7 : q;
      }
      out[2 + idx / 4] |= (uint8_t)((q & 3) << (2 * (idx % 4)));
      out[66 + idx / 8] |= (uint8_t)(((q >> 2) & 1) << (idx % 8));
    }
  }
}

/* IQ3_XXS (DequantIQ.cs:364-399): d*(q3-4), 3-bit fields of a 24-bit word
 * per 8 elements. */
static void quant_block_iq3_xxs(const float* w, uint8_t* out) {
  uint16_t dh = chatnet_float_to_half(-signed_amax(w, 256) / 4.0f);
  float d = half_to_float(dh);
  memset(out, 0, 98);
  put16(out, dh);
  for (int s = 0; s < 32; s++) {
    uint32_t packed = 0;
    for (int j = 0; j < 8; j++) {
      int q = d != 0.f ? nearest_int(w[8 * s + j] / d) + 4 : 4;
      q = q < 0 ? 0 : (q > 7 ? 7 : q);
      packed |= (uint32_t)q << (3 * j);
    }
    out[2 + 3 * s] = (uint8_t)packed;
    out[3 + 3 * s] = (uint8_t)(packed >> 8);
    out[4 + 3 * s] = (uint8_t)(packed >> 16);
  }
}

/* The 2-bit fields of IQ2_XS / IQ2_XXS / IQ2_S: element e of sub-block s at
 * bits 2(e%4) of byte 2 + 4s + e/4. */
static inline void put_iq2(uint8_t* out, int s, int e, int q) { out[2 + 4 * s + e / 4] |= (uint8_t)((q & 3) << (2 * (e % 4))); }

/* IQ2_XS (DequantIQ.cs:456-496): (d*sc)*(q-1), sc a nibble - 8 per 16
 * elements; scales kept positive, q-1 spans -1..2. */
static void quant_block_iq2_xs(const float* w, uint8_t* out) {
  float amax = 0.f;
  for (int i = 0; i < 256; i++) amax = fabsf(w[i]) > amax ? fabsf(w[i]) : amax;
  uint16_t dh = chatnet_float_to_half(amax / 14.0f);
  float d = half_to_float(dh);
  memset(out, 0, 74);
  put16(out, dh);
  for (int s = 0; s < 16; s++) {
    float a = fabsf(signed_amax(w + 16 * s, 16));
    int sc = d > 0.f ? nearest_int(a / 2.0f / d) : 1;
    sc = sc < 1 ? 1 : (sc > 7 ? 7 : sc);
    out[66 + s / 2] |= (uint8_t)((sc + 8) << (4 * (s & 1)));
    float dsc = d * (float)sc;
    for (int e = 0; e < 16; e++) {
      int q = dsc > 0.f ? nearest_int(w[16 * s + e] / dsc) + 1 : 1;
      put_iq2(out, s, e, q < 0 ? 0 : (q > 3 ? 3 : q));
    }
  }
}

/* IQ2_XXS (DequantIQ.cs:568-598): d*(q-1). */
static void quant_block_iq2_xxs(const float* w, uint8_t* out) {
  float amax = 0.f;
  for (int i = 0; i < 256; i++) amax = fabsf(w[i]) > amax ? fabsf(w[i]) : amax;
  uint16_t dh = chatnet_float_to_half(amax / 2.0f);
  float d = half_to_float(dh);
  memset(out, 0, 66);
  put16(out, dh);
  for (int i = 0; i < 256; i++) {
    int q = d > 0.f ? nearest_int(w[i] / d) + 1 : 1;
    put_iq2(out, i / 16, i % 16, q < 0 ? 0 : (q > 3 ? 3 : q));
  }
}

/* IQ2_S (DequantIQ.cs:656-696): (d*sc)*q, q 0..3, sc = low nibble + 1; only
 * elements 0..3 of a sub-block can be negative (sign nibble). */
static void quant_block_iq2_s(const float* w, uint8_t* out) {
  float amax = 0.f;
  for (int i = 0; i < 256; i++) amax = fabsf(w[i]) > amax ? fabsf(w[i]) : amax;
  uint16_t dh = chatnet_float_to_half(amax / 48.0f);
  float d = half_to_float(dh);
  memset(out, 0, 82);
  put16(out, dh);
  for (int s = 0; s < 16; s++) {
    float a = fabsf(signed_amax(w + 16 * s, 16));
    int sc = d > 0.f ? nearest_int(a / 3.0f / d) : 1;
    sc = sc < 1 ? 1 : (sc > 16 ? 16 : sc);
    int sign = 0;
    float dsc = d * (float)sc;
    for (int e = 0; e < 16; e++) {
      float v = w[16 * s + e];
      if (e < 4 && v < 0.f) sign |= 1 << e;
      int q = (dsc > 0.f && (v >= 0.f || e < 4)) ? nearest_int(fabsf(v) / dsc) : 0;
      put_iq2(out, s, e, q > 3 ? 3 : q);
    }
    out[66 + s] = (uint8_t)((sc - 1) | (sign << 4));
  }
}

/* IQ1_S / IQ1_M (DequantIQ.cs:767-805, :869-914): element j of sub-block s is
 * +1 with bit j of qs[s], else -1 with bit (s%2)*4 + j/2 of qh[s/2] (shared by
 * two elements), else 0; times d (IQ1_S) or d*sc, sc = 1 or 0.5 (IQ1_M).  The
 * shared bit is set where it lowers the pair's error. */
static float iq1_encode_sub(const float* w, float step, uint8_t* qs, uint8_t* qh, int s, int write) {
  float err = 0.f;
  uint8_t bits = 0, hb = 0;
  for (int p = 0; p < 4; p++) {
    float e0 = 0.f, e1 = 0.f;  /* pair error without / with the shared -1 bit */
    uint8_t b0 = 0, b1 = 0;
    for (int k = 0; k < 2; k++) {
      int j = 2 * p + k;
      float v = w[j];
      float zero = fabsf(v), plus = fabsf(v - step), minus = fabsf(v + step);
      if (plus < zero) { e0 += plus; b0 |= (uint8_t)(1 << j); } else e0 += zero;
      if (plus < minus) { e1 += plus; b1 |= (uint8_t)(1 << j); } else e1 += minus;
    }
    if (e1 < e0) { err += e1; bits |= b1; hb |= (uint8_t)(1 << p); } else { err += e0; bits |= b0; }
  }
  if (write) {
    qs[s] = bits;
    qh[s / 2] |= (uint8_t)(hb << ((s % 2) * 4));
  }
  return err;
}

static void quant_block_iq1_s(const float* w, uint8_t* out) {
  float mean = 0.f;
  for (int i = 0; i < 256; i++) mean += fabsf(w[i]);
  uint16_t dh = chatnet_float_to_half(1.5f * mean / 256.0f);
  float d = half_to_float(dh);
  memset(out, 0, 50);
  put16(out, dh);
  for (int s = 0; s < 32; s++) iq1_encode_sub(w + 8 * s, d, out + 2, out + 34, s, 1);
}

static void quant_block_iq1_m(const float* w, uint8_t* out) {
  float mean = 0.f;
  for (int i = 0; i < 256; i++) mean += fabsf(w[i]);
  uint16_t dh = chatnet_float_to_half(2.0f * mean / 256.0f);
  float d = half_to_float(dh);
  memset(out, 0, 56);
  put16(out, dh);
  for (int s = 0; s < 32; s++) {
    int full = iq1_encode_sub(w + 8 * s, d, out + 2, out + 34, s, 0) <=
               iq1_encode_sub(w + 8 * s, 0.5f * d, out + 2, out + 34, s, 0);
    iq1_encode_sub(w + 8 * s, full ? d : 0.5f * d, out + 2, out + 34, s, 1);
    if (full) out[50 + s / 8] |= (uint8_t)(1 << (s % 8));
  }
}

static int block_info(uint32_t type, int* blk, int* bytes) {
  switch (type) {
    case 2: *blk = 32; *bytes = 18; return 0;
    case 8: *blk = 32; *bytes = 34; return 0;
    case 12: *blk = 256; *bytes = 144; return 0;
    case 13: *blk = 256; *bytes = 176; return 0;
    case 14: *blk = 256; *bytes = 210; return 0;
    case 3: *blk = 32; *bytes = 20; return 0;
    case 6: *blk = 32; *bytes = 22; return 0;
    case 7: *blk = 32; *bytes = 24; return 0;
    case 10: *blk = 256; *bytes = 84; return 0;
    case 11: *blk = 256; *bytes = 110; return 0;
    case 15: *blk = 256; *bytes = 292; return 0;
    case 16: *blk = 256; *bytes = 66; return 0;
    case 17: *blk = 256; *bytes = 74; return 0;
    case 18: *blk = 256; *bytes = 98; return 0;
    case 19: *blk = 256; *bytes = 50; return 0;
    case 20: *blk = 32; *bytes = 18; return 0;
    case 21: *blk = 256; *bytes = 110; return 0;
    case 22: *blk = 256; *bytes = 82; return 0;
    case 23: *blk = 256; *bytes = 136; return 0;
    case 29: *blk = 256; *bytes = 56; return 0;
    default: return -1;
  }
}

static void quant_block(uint32_t type, const float* src, uint8_t* dst) {
  switch (type) {
    case 2: quant_block_q4_0(src, dst); break;
    case 8: quant_block_q8_0(src, dst); break;
    case 12: quant_block_q4_k(src, dst); break;
    case 13: quant_block_q5_k(src, dst); break;
    case 3: quant_block_q4_1(src, dst); break;
    case 6: quant_block_q5_0(src, dst); break;
    case 7: quant_block_q5_1(src, dst); break;
    case 10: quant_block_q2_k(src, dst); break;
    case 11: quant_block_q3_k(src, dst); break;
    case 15: quant_block_q8_k(src, dst); break;
    case 16: quant_block_iq2_xxs(src, dst); break;
    case 17: quant_block_iq2_xs(src, dst); break;
    case 18: quant_block_iq3_xxs(src, dst); break;
    case 19: quant_block_iq1_s(src, dst); break;
    case 20: quant_block_iq4_nl(src, dst); break;
    case 22: quant_block_iq2_s(src, dst); break;
    case 23: quant_block_iq4_xs(src, dst); break;
    case 29: quant_block_iq1_m(src, dst); break;
    default: quant_block_q6_k(src, dst); break;
  }
}

/* Quantizes n floats (n a multiple of the block) into `out`. Returns bytes written or 0. */
EXPORT uint64_t chatnet_synth_quantize(uint32_t type, const float* w, uint64_t n, void* out) {
  int blk, bytes;
  if (block_info(type, &blk, &bytes) || n % (uint64_t)blk) return 0;
  uint64_t nb = n / (uint64_t)blk;
  uint8_t* o = (uint8_t*)out;
  if (type == 21) {  /* IQ3_S: each block reads 28 bytes of the next, so encode back to front */
    static const uint8_t zeros[28] = {0};
    for (int64_t b = (int64_t)nb - 1; b >= 0; b--)
      quant_block_iq3_s(w + (uint64_t)b * blk, o + (uint64_t)b * bytes,
                        b + 1 < (int64_t)nb ? o + (uint64_t)(b + 1) * bytes : zeros);
    return nb * (uint64_t)bytes;
  }
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < (int64_t)nb; b++) {
    const float* src = w + (uint64_t)b * blk;
    uint8_t* dst = o + (uint64_t)b * bytes;
    quant_block(type, src, dst);
  }
  return nb * (uint64_t)bytes;
}

/* Generates n = rows*cols N(0, sigma) weights of tensor `stream` and
 * quantizes them straight into `out` (no n-float intermediate). F32 (type 0)
 * writes the floats themselves. Returns bytes written or 0. */
EXPORT uint64_t chatnet_synth_tensor(uint32_t type, uint64_t seed, uint64_t stream, float sigma, uint64_t n,
                                     void* out) {
  if (type == 0) {
    chatnet_synth_normal(seed, stream, 0, n, sigma, (float*)out);
    return n * 4;
  }
  int blk, bytes;
  if (block_info(type, &blk, &bytes) || n % (uint64_t)blk) return 0;
  uint64_t nb = n / (uint64_t)blk;
  uint64_t key = stream_key(seed, stream);
  uint8_t* o = (uint8_t*)out;
  if (type == 21) {  /* IQ3_S: back to front, as chatnet_synth_quantize */
    static const uint8_t zeros[28] = {0};
    for (int64_t b = (int64_t)nb - 1; b >= 0; b--) {
      float w[256];
      uint64_t e0 = (uint64_t)b * blk;
      for (int j = 0; j < blk; j += 2) {
        double z0, z1;
        normal_pair(key, (e0 + j) >> 1, &z0, &z1);
        w[j] = (float)(z0 * sigma);
        w[j + 1] = (float)(z1 * sigma);
      }
      quant_block_iq3_s(w, o + (uint64_t)b * bytes, b + 1 < (int64_t)nb ? o + (uint64_t)(b + 1) * bytes : zeros);
    }
    return nb * (uint64_t)bytes;
  }
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < (int64_t)nb; b++) {
    float w[256];
    uint64_t e0 = (uint64_t)b * blk;
    for (int j = 0; j < blk; j += 2) {
      double z0, z1;
      normal_pair(key, (e0 + j) >> 1, &z0, &z1);
      w[j] = (float)(z0 * sigma);
      w[j + 1] = (float)(z1 * sigma);
    }
    uint8_t* dst = o + (uint64_t)b * bytes;
    quant_block(type, w, dst);
  }
  return nb * (uint64_t)bytes;
}
