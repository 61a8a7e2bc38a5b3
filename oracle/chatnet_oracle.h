/*
 * chatnet_oracle.h — CPU oracle for the quantized Llama forward pass.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of ChatNet's CPU
 * algorithm (C#, not buildable here: no .NET toolchain in the image), used as
 * the parity checker for libchatnet_hip and as the CPU baseline timer.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path (chatnet_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates.  The restatement
 * keeps the reference's accumulation structure: Vector128<float> (4 lanes) in
 * the fused quant dots, Vector<float> (8 lanes, AVX2 width) in the other ops,
 * separate multiply and add (compiled with -ffp-contract=off), glibc
 * expf/sinf/cosf/logf/sqrtf for MathF.*.
 *
 * Pinning (how each function is checked; see tests/test_oracle_*.py):
 *   half_to_float     IEEE closed form, all 65536 inputs vs numpy float16.
 *   q4_0 dequant/dot  reference KATs QuantizationTests.cs:23-87,704-726 and a
 *                     float64 brute force on random blocks.
 *   q4_k dequant/dot  reference KATs QuantizationTests.cs:445-489,728-759,
 *                     a hand-derived single-sub-block nibble-order KAT, and
 *                     float64 brute force.
 *   q6_k dequant/dot  reference KATs QuantizationTests.cs:302-345, a
 *                     hand-derived element-position KAT, float64 brute force.
 *   q8_0 dequant/dot  reference KATs QuantizationTests.cs:235-295 and float64
 *                     brute force.
 *   q5_k dequant/dot  reference KAT QuantizationTests.cs:513-537 (dot 5184),
 *                     a hand-derived high-bit position KAT, float64 brute force.
 *   q4_1 q5_0 q5_1 q8_k  reference exact-value KATs QuantizationTests.cs:
 *                     93-110, 141-157, 189-205, 544-562, hand-derived position
 *                     KATs (high-bit words, nibble halves), float64 brute force.
 *   q2_k q3_k         hand-derived element/scale position KATs (each element's
 *                     bit field and scale byte set alone), closed forms
 *                     (uniform fields), float64 brute force.
 *   iq4_nl            reference KATs QuantizationTests.cs:594-635 (table
 *                     lookups, dot = dequantize-then-dot), float64 brute force.
 *   iq4_xs iq3_s iq3_xxs iq2_xs iq2_xxs iq2_s iq1_s iq1_m  hand-derived
 *                     position KATs for every bit field (one field set at a
 *                     time; the quirks above: IQ4_XS scale bytes 4..11, IQ3_S
 *                     signs/scales read from the next block, IQ2_S signs on
 *                     elements 0..3 only), closed forms, float64 brute force.
 *                     Sign of a zero weight (the reference's -0.0 for a negated
 *                     zero magnitude): parity unpinned (no test distinguishes).
 *   rope_neox         closed form at hd 4, identity at pos 0, pair norms, and
 *                     the exact identity neox = P^-1 . rope . P with P the
 *                     split-half -> interleaved permutation of each head.
 *   Qwen2 forward     the float64 numpy restatement of a tiny model with biases
 *                     and split-half RoPE (tests/npref.py).
 *   rmsnorm/rope/softmax/silu/add/attention/argmax: invariants (closed forms,
 *                     identity at pos 0, norm preservation, shift invariance,
 *                     tie rule) and a float64 numpy restatement of a tiny model.
 *   net_random        published outputs of .NET's Random (Random(0), Random(42))
 *                     and the |seed| / int.MinValue rules of its constructor.
 *   temperature_sample a float64 restatement of the sampling rule on random
 *                     logits, hand-derived special cases (greedy fallback,
 *                     top-1, nucleus of one, a top-2 split) and draw
 *                     frequencies.  The order the quickselect leaves equal
 *                     probabilities in: parity unpinned.
 *   Order of Vector128.Sum / MathF last-ulp results: parity unpinned (only
 *                     running .NET could pin them; covered by tolerance).
 */
#ifndef CHATNET_ORACLE_H
#define CHATNET_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_Q4_0 = 2, ORACLE_Q4_1 = 3, ORACLE_Q5_0 = 6, ORACLE_Q5_1 = 7,
       ORACLE_Q8_0 = 8, ORACLE_Q2_K = 10, ORACLE_Q3_K = 11, ORACLE_Q4_K = 12, ORACLE_Q5_K = 13, ORACLE_Q6_K = 14,
       ORACLE_Q8_K = 15, ORACLE_IQ2_XXS = 16, ORACLE_IQ2_XS = 17, ORACLE_IQ3_XXS = 18, ORACLE_IQ1_S = 19,
       ORACLE_IQ4_NL = 20, ORACLE_IQ3_S = 21, ORACLE_IQ2_S = 22, ORACLE_IQ4_XS = 23, ORACLE_IQ1_M = 29 };

void oracle_set_threads(int n);
int oracle_get_threads(void);

float oracle_half_to_float(uint16_t h);

void oracle_dequant_q4_0(const uint8_t* src, float* out, int n);
float oracle_dot_q4_0(const uint8_t* row, const float* x, int n);
void oracle_dequant_q4_k(const uint8_t* src, float* out, int n);
float oracle_dot_q4_k(const uint8_t* row, const float* x, int n);
void oracle_dequant_q6_k(const uint8_t* src, float* out, int n);
float oracle_dot_q6_k(const uint8_t* row, const float* x, int n);
void oracle_dequant_q8_0(const uint8_t* src, float* out, int n);
float oracle_dot_q8_0(const uint8_t* row, const float* x, int n);
void oracle_dequant_q5_k(const uint8_t* src, float* out, int n);
float oracle_dot_q5_k(const uint8_t* row, const float* x, int n);
void oracle_dequant_q4_1(const uint8_t* src, float* out, int n);
float oracle_dot_q4_1(const uint8_t* row, const float* x, int n);
void oracle_dequant_q5_0(const uint8_t* src, float* out, int n);
float oracle_dot_q5_0(const uint8_t* row, const float* x, int n);
void oracle_dequant_q5_1(const uint8_t* src, float* out, int n);
float oracle_dot_q5_1(const uint8_t* row, const float* x, int n);
void oracle_dequant_q2_k(const uint8_t* src, float* out, int n);
float oracle_dot_q2_k(const uint8_t* row, const float* x, int n);
void oracle_dequant_q3_k(const uint8_t* src, float* out, int n);
float oracle_dot_q3_k(const uint8_t* row, const float* x, int n);
void oracle_dequant_q8_k(const uint8_t* src, float* out, int n);
float oracle_dot_q8_k(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq4_nl(const uint8_t* src, float* out, int n);
float oracle_dot_iq4_nl(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq4_xs(const uint8_t* src, float* out, int n);
float oracle_dot_iq4_xs(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq3_s(const uint8_t* src, float* out, int n);
float oracle_dot_iq3_s(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq3_xxs(const uint8_t* src, float* out, int n);
float oracle_dot_iq3_xxs(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq2_xs(const uint8_t* src, float* out, int n);
float oracle_dot_iq2_xs(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq2_xxs(const uint8_t* src, float* out, int n);
float oracle_dot_iq2_xxs(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq2_s(const uint8_t* src, float* out, int n);
float oracle_dot_iq2_s(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq1_s(const uint8_t* src, float* out, int n);
float oracle_dot_iq1_s(const uint8_t* row, const float* x, int n);
void oracle_dequant_iq1_m(const uint8_t* src, float* out, int n);
float oracle_dot_iq1_m(const uint8_t* row, const float* x, int n);
float oracle_dot_f32(const float* a, const float* b, int n);

/* y[m] = dot(W row m, x) for m < M (MatVecMulByType semantics). Returns 0 or -3
 * for an unsupported type. */
int oracle_matvec(uint32_t type, const void* W, const float* x, float* y, int M, int K);

void oracle_rmsnorm(const float* x, const float* w, float* out, int n, float eps);
void oracle_softmax(float* data, int n);
void oracle_silu_mul(float* gate, const float* up, int n);
void oracle_add(float* a, const float* b, int n);
void oracle_rope(float* q, float* k, int position, int head_dim, int n_heads, int n_kv_heads,
                 float freq_base);
void oracle_rope_neox(float* q, float* k, int position, int head_dim, int n_heads, int n_kv_heads,
                      float freq_base);
int oracle_argmax(const float* logits, int n);

/* System.Random(int seed) of the .NET BCL (the seeded compat generator). */
typedef struct oracle_net_random {
  int32_t seed_array[56];
  int32_t inext, inextp;
} oracle_net_random;
void oracle_net_random_init(oracle_net_random* r, int32_t seed);
int32_t oracle_net_random_sample(oracle_net_random* r); /* InternalSample, [0, int.MaxValue) */
double oracle_net_random_next_double(oracle_net_random* r);

/* TemperatureSampler.Sample with the draw r = (float)Random.NextDouble() passed
 * in.  Returns the token (-1 for top_k < 1, where the reference indexes out of
 * range); *margin (nullable) receives the smallest distance between a quantity
 * the result depends on and the threshold it was compared with: the gap of the
 * k-th to the (k+1)-th probability relative to the k-th, and in probability
 * units cumulative vs top_p and draw vs running sum. */
int oracle_temperature_sample(const float* logits, int n, float temperature, int top_k, float top_p, float r,
                              float* margin);

/* Whole model.  Tensor pointers are borrowed host pointers (like the mmap). */
enum { ORACLE_ARCH_LLAMA = 0, ORACLE_ARCH_QWEN2 = 1 };
typedef struct oracle_config {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size, context_length;
  float rope_freq_base, rms_norm_eps;
  int32_t arch; /* ORACLE_ARCH_LLAMA (Llama, Mistral) or ORACLE_ARCH_QWEN2 */
} oracle_config;

typedef struct oracle_llama oracle_llama;
oracle_llama* oracle_llama_create(const oracle_config* cfg);
int oracle_llama_set_tensor(oracle_llama* m, const char* name, uint32_t type, const void* data);
int oracle_llama_forward(oracle_llama* m, const int32_t* tokens, int n, int position, float* logits);
/* Copies layer `layer`'s cached K (which=0) or V (which=1) at `position`
 * (kv_dim floats) to out. */
int oracle_llama_kv(oracle_llama* m, int layer, int position, int which, float* out);
void oracle_llama_destroy(oracle_llama* m);

#ifdef __cplusplus
}
#endif

#endif
