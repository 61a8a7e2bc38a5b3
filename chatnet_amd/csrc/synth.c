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
 * Every element is a pure function of (seed, stream, index): a splitmix64
 * counter hash feeds a Box-Muller transform, so any tensor can be regenerated
 * bit-identically, in any order, on any number of threads.
 */
#include <math.h>
#include <stdint.h>
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
    default: quant_block_q6_k(src, dst); break;
  }
}

/* Quantizes n floats (n a multiple of the block) into `out`. Returns bytes written or 0. */
EXPORT uint64_t chatnet_synth_quantize(uint32_t type, const float* w, uint64_t n, void* out) {
  int blk, bytes;
  if (block_info(type, &blk, &bytes) || n % (uint64_t)blk) return 0;
  uint64_t nb = n / (uint64_t)blk;
  uint8_t* o = (uint8_t*)out;
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
