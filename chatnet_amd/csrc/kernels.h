// kernels.h — host-side launch interface of the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

// A kernel may use more than 64 KB of dynamic LDS only after its maximum was
// raised, per device.  allow_full_lds raises it to the CU's whole 160 KB (so
// every later launch of the kernel fits, whatever its size) the first time a
// device launches the kernel; `done` holds one bit per device ordinal < 64
// (higher ordinals set the attribute on every call).  Concurrent first calls
// both set the same value.
constexpr int kCuLdsBytes = 160 * 1024;
inline hipError_t allow_full_lds(const void* kern, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, kCuLdsBytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

// STORE and LOGITS write y = W x; LOGITS is the LM-head instance (a separate
// kernel so its launches are told apart from stand-alone GEMVs in profiles).
// GEMV_EPI_ADD_MERGE: GEMV_EPI_ADD whose x is the decode attention's output,
// combined from its per-chunk partials while it is staged (the O projection
// of a position bucket with 2..kFoldMaxSplits chunks; no merge launch).
enum { GEMV_EPI_STORE = 0, GEMV_EPI_ADD = 1, GEMV_EPI_QKV = 2, GEMV_EPI_SWIGLU = 3, GEMV_EPI_LOGITS = 4,
       GEMV_EPI_ADD_MERGE = 5 };
constexpr int kFoldMaxSplits = 8;

// One fused GEMV launch over up to three weight segments of the same type.
// Virtual rows: STORE/ADD use segment 0 only; QKV concatenates q|k|v rows;
// SWIGLU interleaves gate (even) and up (odd) rows.
struct GemvArgs {
  const uint8_t* w[3];
  int seg_rows[3];
  int n_vrows;
  int K;
  const float* x;       // K fp32 inputs
  const float* norm_w;  // optional fused RMSNorm weight (K), nullptr = none
  float eps;
  float* out[3];  // out[0]: y / q / h
  // QKV epilogue
  const int* pos;  // device position of the token
  int head_dim;
  const float2* rope;       // RoPE table [context][head_dim/2] of (cos, sin)
  void* kcache;             // layer base of the K cache
  void* vcache;             // layer base of the V cache
  int kv_dim;
  int kv_f16;
  const float* bias;  // QKV: optional per-row bias added before RoPE, indexed by virtual row
  // ADD_MERGE: attention partials [heads][msplits][head_dim] and (max, sum)
  // pairs, chunks of mchunk positions of which those below *pos + 1 count
  const float* part_o;
  const float* part_ml;
  int msplits, mchunk;
  // Decode loops: the stop flag of the device decode state (kDecStop); when it
  // is set the launch returns after staging x, writing nothing.  nullptr
  // elsewhere.
  const int* stop;
};

// Weight types: Q4_0, Q8_0 (K % 64 == 0), Q4_K, Q5_K, Q6_K (K % 256 == 0), and
// F32 / F16 (K % 64 == 0, gemv_float.hip); K <= 16384.  gemv_float_launch
// also takes kGemvPacked: w[] holding packed units (gemm_pack_launch), how the
// model runs Q4_1, Q5_0, Q5_1, IQ4_NL (K % 64 == 0), Q2_K, Q8_K and the other
// IQ types (K % 256 == 0).
constexpr int kGemvPacked = -1;
bool gemv_supports(int qtype, int K);
// True for the types gemv_supports accepts only as packed units.
bool gemv_needs_pack(int qtype);
// Q4_0 rows against N columns of x (N x K fp32, row-major) in launches of up to
// gemv_cols_max(K) columns: y (N x M) column c = the single-column GEMV of x[c]
// (bit for bit outside 4096 < K <= 8192).  K % 64 == 0, K <= 16384.
int gemv_cols_max(int K);
hipError_t gemv_cols_launch(const void* w, const float* x, float* y, int M, int K, int N, int num_cus,
                            hipStream_t st);
size_t gemv_lds_bytes(int qtype, int K);
hipError_t gemv_launch(int qtype, int epi, const GemvArgs& a, int num_cus, hipStream_t st);
hipError_t gemv_float_launch(int qtype, int epi, const GemvArgs& a, int num_cus, hipStream_t st);

// Batched quantized GEMM on the matrix cores (gemm.hip):
//   acc[n][vr] = sum_k W_vr[k] * xb[n][k],  0 <= n < N, 0 <= vr < M
// epilogue `epi`: GEMV_EPI_STORE y[n*ldy+vr] = acc, GEMV_EPI_ADD y += acc,
// GEMV_EPI_SWIGLU h[n][vr/2] = silu(acc[vr even]) * acc[vr odd] as fp16 hi + lo
// planes (hb, hb_lo) in the cn_span_pos order.
enum { GEMM_SEG_SINGLE = 0, GEMM_SEG_CONCAT = 1, GEMM_SEG_INTERLEAVE = 2 };
// How W is stored (GemmArgs::packed): raw Q4_0 blocks, gemm_pack_launch units
// (any packable type), or (the span kernel only) rows of F16 / F32 values or
// raw Q4_K super-blocks.
enum { GEMM_W_Q4_0 = 0, GEMM_W_PACKED = 1, GEMM_W_F16 = 2, GEMM_W_F32 = 3, GEMM_W_Q4_K = 4 };
struct GemmArgs {
  int qtype;
  int packed;             // GEMM_W_*: how w is stored
  const uint8_t* w[3];
  int seg_rows[3];
  int seg_mode;
  int M, K, N;            // M = virtual rows
  const uint16_t* xb;     // N x K, row stride K, fp16 in the cn_span_pos order: one plane scaled per
                          // column (one-plane kernel, to_f16_scaled_launch), or the high parts when precise
  const uint16_t* xb_lo;  // precise: fp16 low parts, x = xb + xb_lo
  const float* xinv;      // one-plane kernel: per-column 2^-e undoing the scale of xb (nullptr: 1)
  int precise;            // exact-weight two-plane kernel
  int epi;
  float* y;               // STORE / ADD target
  int ldy;
  uint16_t* hb;           // SWIGLU target: fp16 high parts of h (cn_span_pos order)
  uint16_t* hb_lo;        // SWIGLU target: fp16 low parts of h
  int ldh;
  float* part;            // K-split partials (stream-K: each workgroup's two part slots),
                          // gemm_workspace_bytes() bytes
  unsigned* tile_cnt;     // one-plane kernel: kGemmTileCounters arrival counters, zero before the
                          // launch and left zero by it; nullptr: no stream-K launch
  int splits;             // set by gemm_launch
  int sk_wgs, sk_dp;      // set by gemm_launch: stream-K workgroups (0: none), of them whole-tile ones
  int sk_tiles;           // set by gemm_launch: the stream-K launch's tiles
};
// Arrival counters a stream-K launch may use (one per tile).
constexpr int kGemmTileCounters = 1024;
bool gemm_supports(int qtype, int K);
// Packed weights: every 64 weights of a row become one 96-byte unit of 64 u8
// codes, 4 fp32 scales and 4 fp32 offsets (one pair per 16 weights), with
// weight k = fmaf(code[k], scale[k/16], offset[k/16]) equal to the block
// type's own dequantized value.  Types Q4_0, Q8_0 (K % 64 == 0) and Q4_K,
// Q5_K, Q6_K (K % 256 == 0).
constexpr int kGemmPackUnit = 96;
bool gemm_pack_supports(int qtype, int K);
size_t gemm_pack_bytes(int M, int K);
hipError_t gemm_pack_launch(int qtype, const void* w, int M, int K, void* dst, hipStream_t st);
// stream_k: the caller passes GemmArgs::tile_cnt (the one-plane kernel may
// then share the tiles past one per CU between workgroups).
size_t gemm_workspace_bytes(int M, int N, int K, int num_cus, bool precise, int wfmt, bool stream_k = false);
// With splits_left, a launch whose K is split leaves its partial tiles in
// a.part ([splits][N][M]) unreduced and reports the split count there (0 when
// the epilogue ran): the caller folds them into its next kernel
// (add_rmsnorm_span_launch for a residual add).
hipError_t gemm_launch(const GemmArgs& a, int num_cus, hipStream_t st, int* splits_left = nullptr);
// x [N][K] fp32 -> the one-plane GEMM's input: xh[n] = fp16(x[n] * 2^e_n) in
// the cn_span_pos order, 2^e_n bringing max|x[n]| into [2^14, 2^15), and
// xinv[n] = 2^-e_n.  K % 32 == 0, K <= 16384.
hipError_t to_f16_scaled_launch(const float* x, uint16_t* xh, float* xinv, int N, int K, hipStream_t st);
// x[r] += the K-split partials part[0..splits)[r] (summed as the GEMM's reduce
// does), then xb / xb_lo = RMSNorm(x[r]) * g as the span GEMM's input (fp16 hi
// + lo planes in the cn_span_pos order); splits 0: the norm alone.  dim % 32
// == 0, dim <= 16384, and dim <= 4096 with splits (at most 16).
hipError_t add_rmsnorm_span_launch(float* x, const float* part, int splits, const float* g, float eps, uint16_t* xb,
                                   uint16_t* xb_lo, int rows, int dim, hipStream_t st);

// Span kernels (prefill.hip).  qkv is [n][ld] fp32 with q | k | v columns.
struct RopeKvArgs {
  float* qkv;
  int ld, dim, kv_dim, head_dim, p0;
  const float2* rope;  // RoPE table [context][head_dim/2] of (cos, sin)
  void* kcache;  // layer base
  void* vcache;
  int kv_f16;
  const float* bias;  // optional [dim | kv_dim | kv_dim] added to q | k | v before RoPE
  // optional: the QKV GEMM's unreduced K-split partials [splits][n][ld]
  // (splits <= 16), read instead of qkv; q is written back to qkv either way
  const float* part;
  int splits;
  int n;  // set by rope_kv_launch
};
hipError_t rope_kv_launch(const RopeKvArgs& a, int n, hipStream_t st);
// Fills tab[p][j] = (cos, sin) of theta = p * exp(2j * dim_inv * neg_log_base),
// p < ctx, j < head_dim/2 (TensorMath.ApplyRoPE's angle, TensorMath.cs:418-432).
hipError_t rope_table_launch(float2* tab, int ctx, int head_dim, float dim_inv, float neg_log_base, hipStream_t st);

struct PrefillAttnArgs {
  const float* qkv;  // q at column 0 of each row
  int ld;
  const void* kc;    // layer base, [ctx][kv_dim]
  const void* vc;
  uint16_t* out;     // [n][ldo]: fp16 high parts, cn_span_pos order
  uint16_t* out_lo;  // [n][ldo]: fp16 low parts
  int ldo;
  int n, p0, n_heads, kv_mul, head_dim, kv_dim, kv_f16;
  float scale;
};
bool attn_prefill_supports(int head_dim, int kv_mul);
hipError_t attn_prefill_launch(const PrefillAttnArgs& a, hipStream_t st);

// Embedding row gather (LlamaModel.LoadEmbedding, LlamaModel.cs:365-394) of
// n tokens read from device memory: x[i] = row tok[i].  type: F32, F16, Q4_0,
// Q8_0 on the stored rows, or kGemvPacked on the packed units of any other
// block type (dim % 64 == 0).
hipError_t embed_launch(const void* emb, int type, int dim, const int* tok, float* x, hipStream_t st,
                        int n = 1);

// GQA decode attention over the device KV cache (LlamaModel.ComputeAttention,
// LlamaModel.cs:241-346).  Reads pos from device memory; seq = pos+1.
struct AttnArgs {
  const float* q;     // n_heads*head_dim
  const void* kc;     // layer base, [ctx][kv_dim]
  const void* vc;
  float* out;         // n_heads*head_dim
  const int* pos;
  int n_heads, kv_mul, head_dim, kv_dim, ctx, kv_f16;
  float scale;
  float* part_o;      // split partials: [n_heads][splits][head_dim]
  float* part_ml;     // [n_heads][splits][2] (max, sum)
  int splits;         // position chunks of the launch (<= kFoldMaxSplits), one workgroup per kv head each
  int chunk;          // positions per chunk: chunk c covers [c*chunk, (c+1)*chunk) below pos+1
  int hsplit;         // workgroups per kv head, each taking kv_mul / hsplit query heads
  const int* stop;    // decode loops: return at once while *stop is set (nullptr: never)
};
hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t st);
// Positions one decode-attention workgroup covers per round of wave steps
// (kv_mul: the query heads the workgroup takes).
int attn_decode_round(int head_dim, int kv_mul);
// Workgroups per kv head for a launch of `splits` position chunks.
int attn_decode_hsplit(int n_kv_heads, int kv_mul, int splits, int num_cus);

// Device decode state, kDecWords ints: the position of the token being
// forwarded, that token, the picks made so far in the current decode loop, a
// stop flag (set by a pick that returns the EOS token; the decode-step kernels
// then exit early, so the cache and logits stay as InferenceEngine.Generate
// leaves them when it breaks before forwarding EOS, InferenceEngine.cs:258-261)
// and the EOS token id of the loop (-1: none).
enum { kDecPos = 0, kDecTok = 1, kDecStep = 2, kDecStop = 3, kDecEos = 4, kDecWords = 8 };

// Greedy argmax (GreedySampler.Sample, GreedySampler.cs:13-26); writes the
// winner to state[kDecTok] and advances state[kDecPos] (the position) by one.
// With out_tokens (a decode loop) it also appends the winner to
// out_tokens[state[kDecStep]++], does nothing while state[kDecStop] is set,
// and sets it when the winner is state[kDecEos].
hipError_t argmax_launch(const float* logits, int n, int* state, int* out_tokens, int out_cap,
                         hipStream_t st);

// TemperatureSampler.Sample (TemperatureSampler.cs:33-112) over the logits with
// the parameters in device memory (so captured graphs read the current ones):
// the draw is draws[state[2]] when draws is given, else params->draw; the
// token is written like argmax_launch's.  top_k must be in [1, kSampleMaxK]
// (clamped to n); scratch holds n floats.
constexpr int kSampleMaxK = 1024;
struct SampleParams {
  float inv_temp;  // 1.0f / temperature, temperature > 0
  int top_k;
  float top_p;
  float draw;
};
hipError_t sample_launch(const float* logits, int n, const SampleParams* params, const float* draws, int* state,
                         int* out_tokens, int out_cap, float* scratch, hipStream_t st);

// System.Random(seed) of the .NET BCL, the seeded compat generator
// (TemperatureSampler.cs:29 constructs it, :97 draws NextDouble).
class NetRandom {
 public:
  explicit NetRandom(int32_t seed);
  double next_double();

 private:
  int32_t internal_sample();
  int32_t a_[56];
  int inext_, inextp_;
};

// h[i] = silu(g[i]) * u[i] (TensorMath.SiluElementwiseMul, TensorMath.cs:253-286).
hipError_t silu_mul_launch(const float* g, const float* u, float* h, int n, hipStream_t st);

// Sets state[kDecPos] = pos, state[kDecTok] = tok and, when step >= 0 (the
// start of a decode loop), state[kDecStep] = step, clears the stop flag and
// sets state[kDecEos] = eos.
hipError_t set_state_launch(int* state, int pos, int tok, int step, hipStream_t st, int eos = -1);
