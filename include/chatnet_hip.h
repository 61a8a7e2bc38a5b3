/*
 * chatnet_hip.h — C ABI of libchatnet_hip.so, the MI355X (gfx950) quantized
 * Llama forward pass that stands in for ChatNet's CPU hot path.
 *
 * The reference has no FFI; its hot path sits behind the C# interface
 * IModel (src/ChatNet.Core/Abstractions/IModel.cs:8-19) implemented by
 * LlamaModel (src/ChatNet.Core/Models/Llama/LlamaModel.cs:18-611).  Each entry
 * point below names the reference member whose behaviour it takes over.
 *
 * Conventions
 *   - Every function returns CHATNET_OK (0) or a negative chatnet_status.
 *     chatnet_last_error() returns a thread-local message for the last
 *     failure on the calling thread.
 *   - The library owns all device memory of a model handle.  Host pointers
 *     are borrowed for the duration of the call only.
 *   - One HIP stream per model handle.  A handle is not thread-safe, which is
 *     the reference's contract too (static per-kernel state in
 *     src/ChatNet.Core/Tensors/TensorMath.cs:30-37).
 *   - Only types, pointers and sizes cross the boundary; no torch types.
 */
#ifndef CHATNET_HIP_H
#define CHATNET_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define CHATNET_API __attribute__((visibility("default")))
#else
#define CHATNET_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Each maps to the .NET exception the reference throws for
 * the same condition, so a P/Invoke adapter can rethrow it. */
typedef enum chatnet_status {
  CHATNET_OK = 0,
  CHATNET_ERR_INVALID_ARG = -1,      /* ArgumentException */
  CHATNET_ERR_NOT_FOUND = -2,        /* KeyNotFoundException, MemoryMappedWeights.cs:50-53 */
  CHATNET_ERR_UNSUPPORTED_TYPE = -3, /* NotSupportedException, LlamaModel.cs:564-565 */
  CHATNET_ERR_SIZE_MISMATCH = -4,    /* byte count differs from GgufTensorInfo.ByteSize */
  CHATNET_ERR_OUT_OF_RANGE = -5,     /* IndexOutOfRangeException (position >= context, token >= vocab) */
  CHATNET_ERR_NO_DEVICE = -6,        /* no usable HIP device */
  CHATNET_ERR_HIP = -7,              /* a HIP runtime call failed */
  CHATNET_ERR_OUT_OF_MEMORY = -8     /* OutOfMemoryException */
} chatnet_status;

/* GGML tensor type codes, identical to GgmlType
 * (src/ChatNet.Core/Gguf/GgufConstants.cs:41-71). */
enum {
  CHATNET_GGML_F32 = 0,
  CHATNET_GGML_F16 = 1,
  CHATNET_GGML_Q4_0 = 2,
  CHATNET_GGML_Q4_1 = 3,
  CHATNET_GGML_Q5_0 = 6,
  CHATNET_GGML_Q5_1 = 7,
  CHATNET_GGML_Q8_0 = 8,
  CHATNET_GGML_Q2_K = 10,
  CHATNET_GGML_Q3_K = 11,
  CHATNET_GGML_Q4_K = 12,
  CHATNET_GGML_Q5_K = 13,
  CHATNET_GGML_Q6_K = 14,
  CHATNET_GGML_Q8_K = 15,
  CHATNET_GGML_IQ2_XXS = 16,
  CHATNET_GGML_IQ2_XS = 17,
  CHATNET_GGML_IQ3_XXS = 18,
  CHATNET_GGML_IQ1_S = 19,
  CHATNET_GGML_IQ4_NL = 20,
  CHATNET_GGML_IQ3_S = 21,
  CHATNET_GGML_IQ2_S = 22,
  CHATNET_GGML_IQ4_XS = 23,
  CHATNET_GGML_IQ1_M = 29
};

/* KV-cache element type. */
enum { CHATNET_KV_F32 = 0, CHATNET_KV_F16 = 1 };

/* Forward-pass variant, chosen by GGUF general.architecture the way
 * ModelFactory.DetectArchitecture / CreateModel do
 * (src/ChatNet.Core/Models/ModelFactory.cs:23-82):
 *   CHATNET_ARCH_LLAMA  "llama" and "mistral": LlamaModel.Forward
 *                       (LlamaModel.cs:93-238); MistralModel.Forward
 *                       (Models/Mistral/MistralModel.cs:67-154) is the same
 *                       computation (no sliding window).
 *   CHATNET_ARCH_QWEN2  "qwen2" and "qwen": QwenModel.Forward
 *                       (Models/Qwen/QwenModel.cs:69-178): optional F32 biases
 *                       added to q, k and v after their projections, and
 *                       split-half (NeoX) RoPE, TensorMath.ApplyRoPENeox
 *                       (TensorMath.cs:475-520). */
enum { CHATNET_ARCH_LLAMA = 0, CHATNET_ARCH_QWEN2 = 1 };

/* Model hyper-parameters.  Mirrors LlamaConfig
 * (src/ChatNet.Core/Models/Llama/LlamaConfig.cs:8-38), which is derived from
 * ModelConfig (src/ChatNet.Core/Abstractions/ModelConfig.cs:6-27). */
typedef struct chatnet_config {
  int32_t dim;            /* LlamaConfig.Dim        (embedding_length)      */
  int32_t hidden_dim;     /* LlamaConfig.HiddenDim  (feed_forward_length)   */
  int32_t n_layers;       /* LlamaConfig.LayerCount                         */
  int32_t n_heads;        /* LlamaConfig.HeadCount                          */
  int32_t n_kv_heads;     /* LlamaConfig.KvHeadCount                        */
  int32_t head_dim;       /* LlamaConfig.HeadDim                            */
  int32_t vocab_size;     /* LlamaConfig.VocabSize                          */
  int32_t context_length; /* LlamaConfig.ContextLength = KV-cache capacity  */
  float rope_freq_base;   /* LlamaConfig.RopeFreqBase                       */
  float rms_norm_eps;     /* LlamaConfig.RmsNormEps                         */
  int32_t kv_dtype;       /* CHATNET_KV_F32 (reference) or CHATNET_KV_F16   */
  int32_t arch;           /* CHATNET_ARCH_LLAMA or CHATNET_ARCH_QWEN2       */
} chatnet_config;

typedef struct chatnet_model chatnet_model;

/* Creates a model on HIP device `device`: allocates the KV cache
 * (n_layers x context_length x n_kv_heads*head_dim per K and V) and all
 * activation scratch in HBM.  Replaces the constructor
 * LlamaModel(ModelConfig, LlamaWeights) (LlamaModel.cs:48-88). */
CHATNET_API int chatnet_create(const chatnet_config* cfg, int device, chatnet_model** out);

/* Copies one GGUF tensor's raw bytes host->device once, in its on-disk block
 * layout (no host-side dequantization).  `name` is the GGUF tensor name the
 * reference resolves in LlamaWeights.ResolveAll (LlamaWeights.cs:78-145):
 * token_embd.weight, output.weight, output_norm.weight and
 * blk.{l}.{attn_norm,ffn_norm,attn_q,attn_k,attn_v,attn_output,
 * ffn_gate,ffn_up,ffn_down}.weight, plus for CHATNET_ARCH_QWEN2 the optional
 * F32 biases blk.{l}.{attn_q,attn_k,attn_v}.bias (QwenWeights.cs:158-170: a
 * layer that has the q bias must have all three).  Weight matrices may be
 * of every type LlamaModel.MatVecMulByType dispatches (LlamaModel.cs:470-567):
 * F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K
 * and IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_M
 * (as DequantIQ.cs decodes them), each dispatched on its own type.  Q4_1,
 * Q5_0, Q5_1, Q2_K, Q8_K and the IQ types are also re-encoded on the
 * device at upload (u8 codes with an fp32 scale and offset per 16 weights,
 * M*(K/64)*96 bytes beside the stored blocks), the form the GEMV reads them
 * in.  An IQ3_S row's last block reads 28 bytes past the row, as the
 * reference does (DequantIQ.cs:255-283): the next row's first bytes, or for
 * the last row zeros (the reference reads whatever follows the tensor in the
 * file).  Without output.weight the LM head is token_embd.weight, of whatever
 * type (the tied fallback of LlamaWeights.cs:89-98 and QwenWeights.cs:102-112).
 * Embeddings may be of any of those types but IQ3_S (LlamaModel.LoadEmbedding,
 * LlamaModel.cs:365-394; the reference's IQ3_S row dequantize throws,
 * CHATNET_ERR_OUT_OF_RANGE); a block type other than Q4_0 and Q8_0 is
 * re-encoded the same way at upload.
 * `dims` is GGUF order (ne0 = inner).
 * `nbytes` must equal GgufTensorInfo.ByteSize (GgufTensorInfo.cs:30-113).
 * Replaces MemoryMappedWeights.GetTensorPointer (MemoryMappedWeights.cs:76-84)
 * as the source of weight bytes for the forward pass. */
CHATNET_API int chatnet_upload_tensor(chatnet_model* m, const char* name, uint32_t ggml_type,
                          const uint64_t* dims, int ndims, const void* host,
                          uint64_t nbytes);

/* IModel.Forward(ReadOnlySpan<int> tokenIds, int position, Span<float> logits)
 * (IModel.cs:18, LlamaModel.cs:93-238).  Processes tokens[0..n) at positions
 * position..position+n-1, writing their K/V into the cache; logits of the last
 * token stay on the device and are copied to `logits_host` (vocab_size
 * floats) when it is non-NULL.  Spans of 8 or more tokens run as batches of
 * up to 512 tokens when head_dim is 64 or 128 and n_heads / n_kv_heads is at
 * most 64: MFMA GEMMs on fp16 operands (activations as fp16 hi + lo planes)
 * and causal attention over the cache.  Each GEMM of a layer (q|k|v, o,
 * gate|up, down) reads its matrices in one format: F16 rows as stored (two
 * products per step, exact weights), F32 rows split into fp16 hi + lo as
 * read (three products, ~22 bits), block types from their stored blocks when
 * every matrix of that GEMM is Q4_0 (each weight exact as two fp16 planes) or
 * every one is Q4_K (~22 bits), otherwise re-encoded once into packed units
 * kept for the model's lifetime (~22 bits).  Shorter spans, and models whose
 * layers give one GEMM matrices of both a float and a block type (ffn_gate
 * Q4_0 with ffn_up F16), run token by token. */
CHATNET_API int chatnet_forward(chatnet_model* m, const int32_t* tokens, int n, int position,
                    float* logits_host);

/* GreedySampler.Sample (src/ChatNet.Core/Samplers/GreedySampler.cs:13-26) on
 * the device-resident logits of the last forward: index of the first maximum. */
CHATNET_API int chatnet_argmax(chatnet_model* m, int32_t* out_token);

/* Greedy generation loop of InferenceEngine.Generate
 * (src/ChatNet.Core/InferenceEngine.cs:234-307) with the tokenizer and
 * stop-string checks left to the caller: forwards the prompt at positions
 * 0..n_prompt-1, then emits up to max_tokens greedy tokens, feeding each back
 * at the next position.  As in the reference, a token is emitted before the
 * context check, so the loop stops after emitting the token at position
 * context_length - 1 without forwarding it (InferenceEngine.cs:295-298), and a
 * prompt that fills the context still yields one token.  The loop stops before
 * the first `eos_token` and never forwards it (InferenceEngine.cs:258-261):
 * the cache, the position and the logits stay those of the last token before
 * it, so a later chatnet_decode_greedy continues from there.  eos_token < 0
 * disables the check.  The decode loop stays on the device (one HIP graph per
 * step, token fed back through device memory; the steps after an EOS return
 * at once).  Writes the generated ids to out_tokens (room for max_tokens ids)
 * and their count to *n_out. */
CHATNET_API int chatnet_generate_greedy(chatnet_model* m, const int32_t* prompt, int n_prompt,
                            int max_tokens, int32_t eos_token, int32_t* out_tokens,
                            int* n_out);

/* The decode half of InferenceEngine.Generate (InferenceEngine.cs:241-307):
 * continues after a chatnet_forward of positions ..p-1 by sampling greedily
 * from its logits, emitting the token, forwarding it at position p, and so on,
 * with the same context and EOS rules as chatnet_generate_greedy.  Every
 * decode step is one replay of a captured HIP graph; the host synchronizes
 * once, at the end. */
CHATNET_API int chatnet_decode_greedy(chatnet_model* m, int max_tokens, int32_t eos_token,
                                      int32_t* out_tokens, int* n_out);

/* TemperatureSampler.Sample (src/ChatNet.Core/Samplers/TemperatureSampler.cs:33-112)
 * on the device-resident logits of the last forward, with the draw `r` that the
 * reference takes from its Random, (float)NextDouble() (:97).  temperature <= 0
 * is the reference's greedy fallback (:37-41, same result as chatnet_argmax);
 * otherwise softmax(logits / temperature), the top_k most probable tokens
 * (1 <= top_k <= 1024; the reference throws for top_k < 1), the shortest prefix
 * reaching top_p, renormalised, and the first token whose running sum exceeds r. */
CHATNET_API int chatnet_sample(chatnet_model* m, float temperature, int top_k, float top_p, float r,
                               int32_t* out_token);

/* InferenceEngine.Generate (InferenceEngine.cs:234-307) with
 * TemperatureSampler(temperature, top_k, top_p, seed)
 * (TemperatureSampler.cs:25-31): like chatnet_generate_greedy, but every token
 * is drawn by chatnet_sample's rule, the k-th draw being the k-th NextDouble()
 * of System.Random(seed) (seed < 0: a nondeterministic seed, as
 * `new Random()`).  The draws are made on the host before the loop (they do
 * not depend on the logits); the loop itself stays on the device. */
CHATNET_API int chatnet_generate_sampled(chatnet_model* m, const int32_t* prompt, int n_prompt,
                                         int max_tokens, float temperature, int top_k, float top_p,
                                         int32_t seed, int32_t eos_token, int32_t* out_tokens,
                                         int* n_out);

/* The first n values of System.Random(seed).NextDouble() (the .NET BCL's seeded
 * generator that TemperatureSampler uses, TemperatureSampler.cs:29), for callers
 * that drive chatnet_sample one token at a time.  No counterpart to bind in the
 * reference (it is the BCL's); provided so a host loop can reproduce the draws. */
CHATNET_API int chatnet_net_random(int32_t seed, int n, double* out);

/* Copies the device logits of the last forward to the host (vocab_size floats). */
CHATNET_API int chatnet_get_logits(chatnet_model* m, float* logits_host);

/* Matrix product on caller-owned device buffers, the batched form of
 * TensorMath.MatVecMulQ4_0 / MatVecMulQ6K / MatVecMulGeneric / MatVecMul and
 * LlamaModel.MatVecMulF16 (TensorMath.cs:527-656, LlamaModel.cs:570-598) as
 * dispatched by LlamaModel.MatVecMulByType (LlamaModel.cs:470-567):
 *   y[n][m] = sum_k W[m][k] * x[n][k],  0 <= n < N, 0 <= m < M
 * W is M rows of raw GGUF blocks (row stride K/block*bytes_per_block), x is
 * N x K fp32 row-major, y is N x M fp32 row-major; w_dev and x_dev 16-byte
 * aligned.  Types F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL and
 * K % 64 == 0, or Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K and the other IQ types
 * and K % 256 == 0, with K <= 16384 (IQ3_S: bytes past W's last row read as
 * zero).
 * Q4_0 with 2 <= N < 8, or N <= 16 with M*K*N <= 8*4096*4096, runs one
 * multi-column GEMV (each column the N = 1 product's exact arithmetic).  Other
 * calls with N >= 8 and a block type run the dequant-to-LDS fp16 MFMA GEMM (x
 * rounded to fp16 after scaling each column by a power of two that keeps it
 * inside fp16's range, each weight rounded once to fp16; Q4_0 read as raw
 * blocks, the other types first re-encoded
 * into the workspace as u8 codes with an fp32 scale and offset per 16 weights,
 * M*(K/64)*96 bytes, giving the same dequantized values); any other call
 * (N < 8, F32, F16) runs the fused GEMV once per column, which reads Q4_1,
 * Q5_0, Q5_1, Q2_K, Q8_K and the IQ types from that same re-encoded
 * copy, made in the workspace first.  A GEMM whose grid of 128 x 128 tiles
 * is just over one tile per CU (e.g. 11008 x 4096 at N = 512) runs as a
 * stream-K launch: one whole tile per CU, the other tiles' K chunks shared
 * out evenly, a shared tile summed in K order by its last contributor (the
 * result does not depend on arrival order) with arrival counters kept at the
 * start of the workspace.  The GEMM's workspace is allocated on first use
 * per (device, stream) and kept until the process ends (a buffer it outgrows
 * is retired, not freed, since a captured graph may still read it).  A call
 * on a stream under HIP graph capture cannot allocate: it fails with
 * CHATNET_ERR_INVALID_ARG if the stream's workspace is too small, so a
 * capturing caller first makes one uncaptured call of the largest size, or
 * uses chatnet_matmul_noalloc.  `stream` is a hipStream_t (NULL = default
 * stream).  Asynchronous on `stream`. */
CHATNET_API int chatnet_matmul(uint32_t ggml_type, const void* w_dev, const float* x_dev,
                   float* y_dev, int M, int K, int N, void* stream);

/* chatnet_matmul without any allocation, for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  No counterpart in the reference.  Same arguments,
 * kernels and results as chatnet_matmul for Q4_0 and for the types read
 * only as packed units (Q4_1, Q5_0, Q5_1, Q2_K, Q8_K and the IQ types,
 * whose packed copy of W, M*(K/64)*96 bytes, goes into the scratch), except
 * that it runs no stream-K launch: where chatnet_matmul shares tiles it runs
 * the plain tile grid, the same product summed in another order.  Q8_0,
 * Q3_K, Q4_K, Q5_K and Q6_K run the fused GEMV once per column on their stored
 * blocks.  The scratch (fp16 x, its per-column scales, the K-split partials
 * and the packed W) lives
 * in a fixed 64 MiB array per device, held by the library from load to
 * process exit, instead of a per-stream workspace.  Calls needing more
 * scratch than that (N*K*2 bytes of x for N >= 8 and N*4 bytes of scales,
 * each rounded up to 256, plus the partials, plus the packed W) fail with CHATNET_ERR_INVALID_ARG before
 * launching anything.  Every call on one device shares that device's array:
 * calls that may overlap on one device (different streams, threads) race and
 * must be serialized by the caller. */
CHATNET_API int chatnet_matmul_noalloc(uint32_t ggml_type, const void* w_dev, const float* x_dev,
                                       float* y_dev, int M, int K, int N, void* stream);

/* Bytes of one GGUF tensor of `ggml_type` with `n_elements` elements, per
 * GgufTensorInfo.ByteSize (GgufTensorInfo.cs:30-113); 0 for an unknown type. */
CHATNET_API uint64_t chatnet_tensor_nbytes(uint32_t ggml_type, uint64_t n_elements);

/* Frees every device buffer of the model.  Replaces LlamaModel.Dispose
 * (LlamaModel.cs:606-609).  NULL is accepted. */
CHATNET_API void chatnet_destroy(chatnet_model* m);

/* Thread-local message describing the last error on this thread ("" if none). */
CHATNET_API const char* chatnet_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* CHATNET_HIP_H */
