// chatnet_api.hip — the C ABI of libchatnet_hip (declared in include/chatnet_hip.h).
//
// Host-side orchestration of the per-token schedule of LlamaModel.Forward
// (src/ChatNet.Core/Models/Llama/LlamaModel.cs:93-238), six launches per layer:
//   1. QKV GEMV   : RMSNorm (fused prologue) -> Wq|Wk|Wv -> RoPE -> K/V cache write
//   2. attention  : GQA decode attention over the cache, split over positions,
//                   then a merge of the splits
//   3. O GEMV     : x += Wo * attn           (residual fused)
//   4. gate/up    : RMSNorm -> Wg|Wu -> silu(g)*u
//   5. down GEMV  : x += Wd * h              (residual fused)
// then the LM head (final RMSNorm fused) only for the last token of a span.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <random>
#include <string>
#include <utility>
#include <vector>

#include "../../include/chatnet_hip.h"
#include "kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(expr)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess) return fail(CHATNET_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

struct DevTensor {
  void* ptr = nullptr;
  uint32_t type = 0;
  uint64_t nbytes = 0;
  uint64_t ne0 = 0, ne1 = 1;  // GGUF dims: ne0 = inner (K), ne1 = rows (M)
  // The matrix re-encoded for the batched GEMM (gemm_pack_launch), made by the
  // first span that needs it and dropped when the tensor is uploaded again.
  void* pk = nullptr;
};

struct Layer {
  DevTensor attn_norm, ffn_norm, wq, wk, wv, wo, wg, wu, wd;
  // QKV biases (Qwen2), one fp32 buffer [dim | kv_dim | kv_dim] in the row
  // order of the stored q/k/v weights; bias_have: bits 0/1/2 = q/k/v uploaded.
  float* bias = nullptr;
  unsigned bias_have = 0;
};

// CU count per device ordinal, cached (threads may race to fill an entry; they
// store the same value).
int device_cus(int dev) {
  static std::atomic<int> cache[64];
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c) return c;
  }
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64) cache[dev].store(p.multiProcessorCount, std::memory_order_relaxed);
  return p.multiProcessorCount;
}

// Weight types the GEMV serves (LlamaModel.MatVecMulByType, LlamaModel.cs:470-567):
// F32, F16, Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K from the stored blocks, and
// Q4_1, Q5_0, Q5_1, Q2_K, Q8_K and the nine IQ types (the reference's
// MatVecMulGeneric branches, LlamaModel.cs:488-562) from packed units made at
// upload.
bool is_matrix_type(uint32_t t) {
  return t == CHATNET_GGML_F32 || t == CHATNET_GGML_F16 || t == CHATNET_GGML_Q4_0 || t == CHATNET_GGML_Q8_0 ||
         t == CHATNET_GGML_Q3_K || t == CHATNET_GGML_Q4_K || t == CHATNET_GGML_Q5_K || t == CHATNET_GGML_Q6_K ||
         gemv_needs_pack((int)t);
}

// Embedding rows read in their stored form; every other block type is
// gathered from packed units made at upload.
bool embed_raw_type(uint32_t t) {
  return t == CHATNET_GGML_F32 || t == CHATNET_GGML_F16 || t == CHATNET_GGML_Q4_0 || t == CHATNET_GGML_Q8_0;
}

// A matrix as the GEMV reads it: its packed units for the types the GEMV
// takes only in that form, else the stored blocks.
int gemv_qt(const DevTensor& t) { return gemv_needs_pack((int)t.type) ? kGemvPacked : (int)t.type; }
const uint8_t* gemv_w(const DevTensor& t) {
  return (const uint8_t*)(gemv_needs_pack((int)t.type) ? t.pk : t.ptr);
}
int embed_qt(const DevTensor& t) { return embed_raw_type(t.type) ? (int)t.type : kGemvPacked; }
const void* embed_w(const DevTensor& t) { return embed_raw_type(t.type) ? t.ptr : t.pk; }

// Workspace of chatnet_matmul's batched path (fp16 copy of x + K-split
// partials), one per (device, stream): work queued on one stream runs in
// order, so calls sharing a stream can share it.  Grown on demand and kept
// until the process ends; a buffer it outgrows is retired, not freed, because
// a graph the caller captured earlier may still read it.  Growing needs a
// hipMalloc, which a stream under capture cannot take: a capturing caller gets
// an error unless an uncaptured call of the same or a larger size came first.
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, std::pair<char*, size_t>> g_ws;
std::vector<char*> g_ws_retired;

// The first kMatmulCounterBytes of a stream's workspace are the one-plane
// GEMM's stream-K tile counters: zeroed when the workspace is allocated, and
// every launch leaves them zero.
constexpr size_t kMatmulCounterBytes = (size_t)kGemmTileCounters * sizeof(unsigned);

int matmul_workspace(int dev, hipStream_t st, size_t bytes, char** out) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto& e = g_ws[{dev, st}];
  bytes = std::max(bytes, kMatmulCounterBytes);
  if (e.second < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return fail(CHATNET_ERR_INVALID_ARG,
                  "chatnet_matmul: the stream is capturing and its workspace (%zu bytes) is smaller than the %zu "
                  "this call needs; make one uncaptured call of this size first, or use chatnet_matmul_noalloc",
                  e.second, bytes);
    char* p = nullptr;
    if (hipMalloc((void**)&p, bytes) != hipSuccess)
      return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes (matmul workspace) failed", bytes);
    const hipError_t z = hipMemsetAsync(p, 0, kMatmulCounterBytes, st);
    if (z != hipSuccess) {
      (void)hipFree(p);
      return fail(CHATNET_ERR_HIP, "hipMemsetAsync of the matmul workspace's counters: %s", hipGetErrorString(z));
    }
    if (e.first) g_ws_retired.push_back(e.first);
    e = {p, bytes};
  }
  *out = e.first;
  return CHATNET_OK;
}

// Scratch of chatnet_matmul_noalloc: a fixed array in the library's code
// object, so every device the library runs on holds its own copy from module
// load to process exit and no call allocates.  Host code never uses the
// array's name as an address (on the host it names a stand-in, not device
// memory): the device address comes from hipGetSymbolAddress, taken once per
// device with that device current, and is passed to the kernels.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
char* g_scratch_dev[kMaxDevices] = {};

int noalloc_scratch(int dev, char** out) {
  if (dev < 0 || dev >= kMaxDevices) return fail(CHATNET_ERR_NO_DEVICE, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(CHATNET_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_dev[dev];
  return CHATNET_OK;
}

}  // namespace

struct chatnet_model {
  chatnet_config cfg{};
  int device = 0;
  int num_cus = 256;
  int kv_dim = 0;
  size_t kv_elt = 4;
  hipStream_t stream = nullptr;
  DevTensor emb, out, out_norm;
  std::vector<Layer> layers;
  void* kcache = nullptr;
  void* vcache = nullptr;
  float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr;
  float* gu = nullptr;  // [2][hidden]: gate and up of a layer whose two types differ
  int* state = nullptr;  // device decode state, kDecWords ints (kernels.h)
  float* attn_part_o = nullptr;   // split partials of the decode attention
  float* attn_part_ml = nullptr;
  int attn_splits_max = 1;  // most chunks any decode-attention launch uses

  float2* rope = nullptr;  // [context_length][head_dim/2] (cos, sin), filled at creation
  int* out_tokens = nullptr;
  int out_cap = 0;
  // Decode-step graphs, one per position bucket (sequence lengths up to
  // min(ctx, 64 << k) for bucket k), captured on first use.
  static constexpr int kBuckets = 16;
  hipGraphExec_t graphs[kBuckets] = {};
  // The same steps with the temperature sampler in place of the argmax; the
  // sampler's parameters and draws are read from device memory at replay.
  hipGraphExec_t sgraphs[kBuckets] = {};
  SampleParams* sparams = nullptr;  // device
  float* sample_p = nullptr;        // [vocab] probabilities scratch
  float* draws = nullptr;           // [draws_cap] draw of each step
  int draws_cap = 0;
  bool have_logits = false;
  int next_pos = 0;  // position after the last forwarded token
  int last_tok = 0;  // last forwarded token
  // Batched span buffers (allocated by the first span of >= kSpanMin tokens):
  // up to span_cap tokens per pass.
  int span_cap = 0;
  float* sp_x = nullptr;       // [cap][dim] residual stream
  // GEMM inputs as fp16 hi + lo planes in the span order (x = hi + lo to ~2^-22)
  uint16_t* sp_xb = nullptr;   // [2][cap][dim]: normed x, then attention output
  uint16_t* sp_hb = nullptr;   // [2][cap][hidden]: silu(gate)*up
  float* sp_qkv = nullptr;     // [cap][dim + 2*kv_dim]
  int* sp_tok = nullptr;       // [cap]
  float* sp_part = nullptr;    // GEMM K-split partials
  size_t sp_part_bytes = 0;
};

namespace {

// Most decode-attention chunks per kv head the CUs call for: up to two
// workgroups per CU over the kv heads, at most 64 (the model then caps it by
// what the O projection folds).
int attn_max_splits(int n_kv_heads, int num_cus) {
  int s = 1;
  while (s < 64 && s * 2 * n_kv_heads <= 2 * num_cus) s *= 2;
  return s;
}

// Position bucket of a sequence length: bucket k covers lengths up to
// min(ctx, 64 << k).  A decode graph serves one bucket; its attention launch is
// sized for the bucket's largest length.
int bucket_index(const chatnet_model* m, int seq) {
  int k = 0;
  while ((64 << k) < seq && (64 << k) < m->cfg.context_length && k + 1 < chatnet_model::kBuckets) k++;
  return k;
}

int bucket_cap(const chatnet_model* m, int seq) {
  const int cap = 64 << bucket_index(m, seq);
  return cap < m->cfg.context_length ? cap : m->cfg.context_length;
}

// Decode-attention launch for sequence lengths up to cap: chunks of at least
// one round of the workgroup's wave steps, as many as attn_max_splits allows;
// chunk * splits >= cap, and every chunk starts below cap.  Where two chunks
// would do, one chunk of two rounds is used instead: its second round costs
// less than the merge launch a second chunk needs.
struct AttnPlan {
  int splits, chunk;
};
AttnPlan attn_plan(const chatnet_model* m, int cap) {
  const int smax = m->attn_splits_max;
  const int round = attn_decode_round(m->cfg.head_dim, m->cfg.n_heads / m->cfg.n_kv_heads);
  int chunk = (cap + smax - 1) / smax;
  if (chunk < round) chunk = round;
  const int splits = (cap + chunk - 1) / chunk;
  if (splits <= 2 && cap <= 2 * round) return {1, cap};
  return {splits, chunk};
}

// Row order of the stored q and k weights of a split-half (NeoX) RoPE model
// (TensorMath.ApplyRoPENeox, TensorMath.cs:475-520, rotates element j of a head
// with element j + hd/2): stored row 2j of a head is source row j and stored
// row 2j+1 is source row j + hd/2.  The interleaved rotation of stored rows
// (2j, 2j+1), with the angle of pair j, is then the split-half rotation, and
// ApplyRoPENeox's angle for j, exp(j * (2/hd) * -ln base), equals ApplyRoPE's
// for the pair at 2j, exp(2j * (1/hd) * -ln base), bit for bit (scaling by 2 is
// exact).  q and the K cache keep this order: a q.k dot product does not depend
// on a permutation applied to both.
int neox_source_row(int r, int hd) {
  const int t = r % hd;
  return r - t + t / 2 + (t & 1) * (hd / 2);
}

void drop_graphs(chatnet_model* m) {
  for (auto& g : m->graphs) {
    if (g) (void)hipGraphExecDestroy(g);
    g = nullptr;
  }
  for (auto& g : m->sgraphs) {
    if (g) (void)hipGraphExecDestroy(g);
    g = nullptr;
  }
}

// QwenWeights' optional biases (QwenWeights.cs:158-170), kept in one buffer
// per layer [dim | kv_dim | kv_dim] in the stored row order of q/k/v.
int upload_bias(chatnet_model* m, Layer& L, int which, const char* name, uint32_t type, uint64_t ne0,
                uint64_t ne1, const void* host) {
  const chatnet_config& c = m->cfg;
  if (type != CHATNET_GGML_F32) return fail(CHATNET_ERR_UNSUPPORTED_TYPE, "tensor %s: biases must be F32", name);
  const int n = which == 0 ? c.dim : m->kv_dim;
  if (ne0 != (uint64_t)n || ne1 != 1)
    return fail(CHATNET_ERR_SIZE_MISMATCH, "tensor %s: dims [%llu, %llu], expected [%d]", name,
                (unsigned long long)ne0, (unsigned long long)ne1, n);
  HIP_TRY(hipSetDevice(m->device));
  HIP_TRY(hipStreamSynchronize(m->stream));
  if (!L.bias) {
    const size_t bytes = sizeof(float) * (size_t)(c.dim + 2 * m->kv_dim);
    if (hipMalloc(&L.bias, bytes) != hipSuccess) return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of bias failed");
    HIP_TRY(hipMemset(L.bias, 0, bytes));
  }
  const float* src = (const float*)host;
  std::vector<float> v(src, src + n);
  if (which < 2)
    for (int r = 0; r < n; r++) v[r] = src[neox_source_row(r, c.head_dim)];
  const size_t off = which == 0 ? 0 : (size_t)c.dim + (which == 2 ? m->kv_dim : 0);
  HIP_TRY(hipMemcpy(L.bias + off, v.data(), sizeof(float) * n, hipMemcpyHostToDevice));
  L.bias_have |= 1u << which;
  drop_graphs(m);
  g_err.clear();
  return CHATNET_OK;
}

}  // namespace

extern "C" {

const char* chatnet_last_error(void) { return g_err.c_str(); }

// GgufTensorInfo.ByteSize (src/ChatNet.Core/Gguf/GgufTensorInfo.cs:30-113).
uint64_t chatnet_tensor_nbytes(uint32_t t, uint64_t n) {
  auto blocks = [n](uint64_t b) { return (n + b - 1) / b; };
  switch (t) {
    case 0: return n * 4;                 // F32
    case 1: return n * 2;                 // F16
    case 2: return blocks(32) * 18;       // Q4_0
    case 3: return blocks(32) * 20;       // Q4_1
    case 6: return blocks(32) * 22;       // Q5_0
    case 7: return blocks(32) * 24;       // Q5_1
    case 8: return blocks(32) * 34;       // Q8_0
    case 9: return blocks(32) * 36;       // Q8_1
    case 10: return blocks(256) * 84;     // Q2_K
    case 11: return blocks(256) * 110;    // Q3_K
    case 12: return blocks(256) * 144;    // Q4_K
    case 13: return blocks(256) * 176;    // Q5_K
    case 14: return blocks(256) * 210;    // Q6_K
    case 15: return blocks(256) * 292;    // Q8_K
    case 16: return blocks(256) * 66;     // IQ2_XXS
    case 17: return blocks(256) * 74;     // IQ2_XS
    case 18: return blocks(256) * 98;     // IQ3_XXS
    case 19: return blocks(256) * 50;     // IQ1_S
    case 20: return blocks(32) * 18;      // IQ4_NL
    case 21: return blocks(256) * 110;    // IQ3_S
    case 22: return blocks(256) * 82;     // IQ2_S
    case 23: return blocks(256) * 136;    // IQ4_XS
    case 24: return n;                    // I8
    case 25: return n * 2;                // I16
    case 26: return n * 4;                // I32
    case 27: return n * 8;                // I64
    case 28: return n * 8;                // F64
    case 29: return blocks(256) * 56;     // IQ1_M
    default: return 0;
  }
}

int chatnet_create(const chatnet_config* cfg, int device, chatnet_model** out) {
  if (!cfg || !out) return fail(CHATNET_ERR_INVALID_ARG, "cfg and out must be non-null");
  *out = nullptr;
  const chatnet_config& c = *cfg;
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
      c.head_dim <= 0 || c.vocab_size <= 0 || c.context_length <= 0)
    return fail(CHATNET_ERR_INVALID_ARG, "all dimensions must be positive");
  if (c.n_heads % c.n_kv_heads != 0)
    return fail(CHATNET_ERR_INVALID_ARG, "n_heads (%d) must be a multiple of n_kv_heads (%d)", c.n_heads, c.n_kv_heads);
  if (c.n_heads * c.head_dim != c.dim)
    return fail(CHATNET_ERR_INVALID_ARG, "n_heads*head_dim (%d) must equal dim (%d)", c.n_heads * c.head_dim, c.dim);
  if (c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
    return fail(CHATNET_ERR_INVALID_ARG, "head_dim %d not supported (32, 64, 128, 256)", c.head_dim);
  if (c.dim % 64 != 0 || c.hidden_dim % 64 != 0)
    return fail(CHATNET_ERR_INVALID_ARG, "dim and hidden_dim must be multiples of 64");
  if (c.context_length > 16384)
    return fail(CHATNET_ERR_INVALID_ARG, "context_length %d exceeds 16384", c.context_length);
  if (c.kv_dtype != CHATNET_KV_F32 && c.kv_dtype != CHATNET_KV_F16)
    return fail(CHATNET_ERR_INVALID_ARG, "kv_dtype %d unknown", c.kv_dtype);
  if (c.arch != CHATNET_ARCH_LLAMA && c.arch != CHATNET_ARCH_QWEN2)
    return fail(CHATNET_ERR_INVALID_ARG, "arch %d unknown", c.arch);
  if (!(c.rope_freq_base > 0.f) || !(c.rms_norm_eps >= 0.f))
    return fail(CHATNET_ERR_INVALID_ARG, "rope_freq_base must be > 0 and rms_norm_eps >= 0");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return fail(CHATNET_ERR_NO_DEVICE, "no HIP device available");
  if (device < 0 || device >= ndev) return fail(CHATNET_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, ndev);
  HIP_TRY(hipSetDevice(device));

  chatnet_model* m = new chatnet_model();
  m->cfg = c;
  m->device = device;
  m->num_cus = device_cus(device);
  m->kv_dim = c.n_kv_heads * c.head_dim;
  m->kv_elt = c.kv_dtype == CHATNET_KV_F16 ? 2 : 4;
  m->layers.resize(c.n_layers);
  const size_t kv_bytes = (size_t)c.n_layers * c.context_length * m->kv_dim * m->kv_elt;
  m->attn_splits_max = attn_max_splits(c.n_kv_heads, m->num_cus);
  {
    // Every workgroup of the O projection reads all chunk partials while it
    // stages x (n_heads * splits * head_dim floats): at most 64 KB of them,
    // and never more chunks than it can fold, so no merge launch is needed.
    int fold_cap = (int)((64 << 10) / ((size_t)c.n_heads * c.head_dim * sizeof(float)));
    fold_cap = fold_cap < 2 ? 2 : (fold_cap > kFoldMaxSplits ? kFoldMaxSplits : fold_cap);
    if (m->attn_splits_max > fold_cap) m->attn_splits_max = fold_cap;
  }
  const size_t attn_slots = (size_t)c.n_heads * m->attn_splits_max;
  auto cleanup = [m]() { chatnet_destroy(m); };
  if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
    cleanup();
    return fail(CHATNET_ERR_HIP, "hipStreamCreate failed");
  }
  struct { void** p; size_t n; } allocs[] = {
      {&m->kcache, kv_bytes},
      {&m->vcache, kv_bytes},
      {(void**)&m->x, sizeof(float) * c.dim},
      {(void**)&m->q, sizeof(float) * c.dim},
      {(void**)&m->att, sizeof(float) * c.dim},
      {(void**)&m->h, sizeof(float) * c.hidden_dim},
      {(void**)&m->gu, sizeof(float) * 2 * c.hidden_dim},
      {(void**)&m->logits, sizeof(float) * c.vocab_size},
      {(void**)&m->state, sizeof(int) * kDecWords},
      {(void**)&m->attn_part_o, sizeof(float) * attn_slots * c.head_dim},
      {(void**)&m->attn_part_ml, sizeof(float) * attn_slots * 2},
      {(void**)&m->rope, sizeof(float2) * (size_t)c.context_length * (c.head_dim / 2)},
      {(void**)&m->sparams, sizeof(SampleParams)},
      {(void**)&m->sample_p, sizeof(float) * c.vocab_size},
  };
  for (auto& a : allocs) {
    if (hipMalloc(a.p, a.n) != hipSuccess) {
      cleanup();
      return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes failed", a.n);
    }
  }
  // Zero the caches once so unwritten positions hold 0 like the managed arrays.
  if (hipMemset(m->kcache, 0, kv_bytes) != hipSuccess || hipMemset(m->vcache, 0, kv_bytes) != hipSuccess ||
      hipMemset(m->state, 0, sizeof(int) * kDecWords) != hipSuccess) {
    cleanup();
    return fail(CHATNET_ERR_HIP, "hipMemset failed");
  }
  // RoPE angles of every position (TensorMath.cs:418-432), computed once.
  if (rope_table_launch(m->rope, c.context_length, c.head_dim, 1.0f / (float)c.head_dim, -logf(c.rope_freq_base),
                        m->stream) != hipSuccess ||
      hipStreamSynchronize(m->stream) != hipSuccess) {
    cleanup();
    return fail(CHATNET_ERR_HIP, "RoPE table initialisation failed");
  }
  *out = m;
  g_err.clear();
  return CHATNET_OK;
}

void chatnet_destroy(chatnet_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->device);
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  drop_graphs(m);
  auto fr = [](void* p) { if (p) (void)hipFree(p); };
  fr(m->emb.ptr); fr(m->out.ptr); fr(m->out_norm.ptr); fr(m->emb.pk); fr(m->out.pk);
  for (auto& l : m->layers) {
    fr(l.attn_norm.ptr); fr(l.ffn_norm.ptr); fr(l.wq.ptr); fr(l.wk.ptr); fr(l.wv.ptr);
    fr(l.wo.ptr); fr(l.wg.ptr); fr(l.wu.ptr); fr(l.wd.ptr); fr(l.bias);
    fr(l.wq.pk); fr(l.wk.pk); fr(l.wv.pk); fr(l.wo.pk); fr(l.wg.pk); fr(l.wu.pk); fr(l.wd.pk);
  }
  fr(m->kcache); fr(m->vcache); fr(m->x); fr(m->q); fr(m->att); fr(m->h); fr(m->gu); fr(m->logits);
  fr(m->state); fr(m->out_tokens);
  fr(m->attn_part_o); fr(m->attn_part_ml); fr(m->rope);
  fr(m->sparams); fr(m->sample_p); fr(m->draws);
  fr(m->sp_x); fr(m->sp_xb); fr(m->sp_hb); fr(m->sp_qkv); fr(m->sp_tok); fr(m->sp_part);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

int chatnet_upload_tensor(chatnet_model* m, const char* name, uint32_t type, const uint64_t* dims,
                          int ndims, const void* host, uint64_t nbytes) {
  if (!m || !name || !dims || !host || ndims < 1 || ndims > 4)
    return fail(CHATNET_ERR_INVALID_ARG, "invalid arguments to chatnet_upload_tensor");
  const chatnet_config& c = m->cfg;
  uint64_t n = 1;
  for (int i = 0; i < ndims; i++) n *= dims[i];
  const uint64_t want = chatnet_tensor_nbytes(type, n);
  if (want == 0) return fail(CHATNET_ERR_UNSUPPORTED_TYPE, "tensor %s: unknown ggml type %u", name, type);
  if (want != nbytes)
    return fail(CHATNET_ERR_SIZE_MISMATCH, "tensor %s: %llu bytes given, ByteSize is %llu", name,
                (unsigned long long)nbytes, (unsigned long long)want);
  const uint64_t ne0 = dims[0], ne1 = ndims > 1 ? dims[1] : 1;
  for (int i = 2; i < ndims; i++)
    if (dims[i] != 1) return fail(CHATNET_ERR_INVALID_ARG, "tensor %s: more than 2 non-unit dims", name);

  DevTensor* slot = nullptr;
  uint64_t want0 = 0, want1 = 0;
  bool matrix = true;
  int layer = -1;
  char suffix[64] = {0};
  if (!strcmp(name, "token_embd.weight")) {
    slot = &m->emb; want0 = c.dim; want1 = c.vocab_size; matrix = false;
    if (!embed_raw_type(type) && !gemm_pack_supports((int)type, 256))
      return fail(CHATNET_ERR_UNSUPPORTED_TYPE, "token_embd.weight: type %u not supported", type);
    if (type == CHATNET_GGML_IQ3_S)  // IQ3S.Dequantize indexes past the row it is given (DequantIQ.cs:266, :280)
      return fail(CHATNET_ERR_OUT_OF_RANGE,
                  "token_embd.weight: IQ3_S rows cannot be dequantized one at a time (the reference's "
                  "IQ3S.Dequantize reads 28 bytes past the row and throws IndexOutOfRangeException)");
    if (!embed_raw_type(type) && !gemm_pack_supports((int)type, c.dim))
      return fail(CHATNET_ERR_INVALID_ARG, "token_embd.weight: dim %d not a multiple of the type's block", c.dim);
    if ((type == CHATNET_GGML_Q4_0 || type == CHATNET_GGML_Q8_0) && c.dim % 32 != 0)
      return fail(CHATNET_ERR_INVALID_ARG, "token_embd.weight: dim %d not a multiple of 32", c.dim);
  } else if (!strcmp(name, "output.weight")) {
    slot = &m->out; want0 = c.dim; want1 = c.vocab_size;
  } else if (!strcmp(name, "output_norm.weight")) {
    slot = &m->out_norm; want0 = c.dim; want1 = 1; matrix = false;
  } else if (sscanf(name, "blk.%d.%63s", &layer, suffix) == 2) {
    if (layer < 0 || layer >= c.n_layers) return fail(CHATNET_ERR_NOT_FOUND, "tensor %s: layer out of range", name);
    Layer& L = m->layers[layer];
    const uint64_t kvd = (uint64_t)m->kv_dim;
    struct { const char* s; DevTensor* t; uint64_t k, r; bool mat; } tab[] = {
        {"attn_norm.weight", &L.attn_norm, (uint64_t)c.dim, 1, false},
        {"ffn_norm.weight", &L.ffn_norm, (uint64_t)c.dim, 1, false},
        {"attn_q.weight", &L.wq, (uint64_t)c.dim, (uint64_t)c.dim, true},
        {"attn_k.weight", &L.wk, (uint64_t)c.dim, kvd, true},
        {"attn_v.weight", &L.wv, (uint64_t)c.dim, kvd, true},
        {"attn_output.weight", &L.wo, (uint64_t)c.dim, (uint64_t)c.dim, true},
        {"ffn_gate.weight", &L.wg, (uint64_t)c.dim, (uint64_t)c.hidden_dim, true},
        {"ffn_up.weight", &L.wu, (uint64_t)c.dim, (uint64_t)c.hidden_dim, true},
        {"ffn_down.weight", &L.wd, (uint64_t)c.hidden_dim, (uint64_t)c.dim, true},
    };
    for (auto& e : tab)
      if (!strcmp(suffix, e.s)) { slot = e.t; want0 = e.k; want1 = e.r; matrix = e.mat; }
    const char* bias_names[3] = {"attn_q.bias", "attn_k.bias", "attn_v.bias"};
    for (int which = 0; which < 3 && !slot && c.arch == CHATNET_ARCH_QWEN2; which++)
      if (!strcmp(suffix, bias_names[which])) return upload_bias(m, L, which, name, type, ne0, ne1, host);
  }
  if (!slot) return fail(CHATNET_ERR_NOT_FOUND, "tensor %s is not part of the Llama layout", name);
  if (ne0 != want0 || ne1 != want1)
    return fail(CHATNET_ERR_SIZE_MISMATCH, "tensor %s: dims [%llu, %llu], expected [%llu, %llu]", name,
                (unsigned long long)ne0, (unsigned long long)ne1, (unsigned long long)want0,
                (unsigned long long)want1);
  if (matrix) {
    if (!is_matrix_type(type))
      return fail(CHATNET_ERR_UNSUPPORTED_TYPE,
                  "tensor %s: weight type %u not supported (F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, "
                  "Q4_K, Q5_K, Q6_K, Q8_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_M)",
                  name, type);
    if (!gemv_supports((int)type, (int)ne0))
      return fail(CHATNET_ERR_INVALID_ARG, "tensor %s: inner dim %llu not a multiple of the block", name,
                  (unsigned long long)ne0);
  } else if (slot != &m->emb && type != CHATNET_GGML_F32) {
    return fail(CHATNET_ERR_UNSUPPORTED_TYPE, "tensor %s: norm weights must be F32", name);
  }
  HIP_TRY(hipSetDevice(m->device));
  if (slot->ptr) {
    HIP_TRY(hipStreamSynchronize(m->stream));
    (void)hipFree(slot->ptr);
    slot->ptr = nullptr;
    if (slot->pk) (void)hipFree(slot->pk);
    slot->pk = nullptr;
  }
  // 256 bytes of tail padding keep every vector load of the kernels in bounds.
  if (hipMalloc(&slot->ptr, nbytes + 256) != hipSuccess)
    return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %llu bytes for %s failed", (unsigned long long)nbytes, name);
  const bool neox_rows = c.arch == CHATNET_ARCH_QWEN2 && layer >= 0 &&
                         (slot == &m->layers[layer].wq || slot == &m->layers[layer].wk);
  // Types the GEMV (or the embedding gather) reads only as packed units are
  // packed below, one pass over the uploaded rows; the stored blocks stay for
  // the other readers.  Their stored rows keep the file's order even where the
  // Qwen2 row order applies (an IQ3_S row reads into the row after it in the
  // file, DequantIQ.cs:255-283): the packed rows are put in that order instead.
  const bool pack_now = (matrix && gemv_needs_pack((int)type)) || (slot == &m->emb && !embed_raw_type(type));
  if (neox_rows && !pack_now) {
    const size_t bpr = (size_t)(nbytes / ne1);
    std::vector<uint8_t> rows(nbytes);
    for (uint64_t r = 0; r < ne1; r++)
      memcpy(rows.data() + r * bpr, (const uint8_t*)host + (size_t)neox_source_row((int)r, c.head_dim) * bpr, bpr);
    HIP_TRY(hipMemcpy(slot->ptr, rows.data(), nbytes, hipMemcpyHostToDevice));
  } else {
    HIP_TRY(hipMemcpy(slot->ptr, host, nbytes, hipMemcpyHostToDevice));
  }
  HIP_TRY(hipMemset((char*)slot->ptr + nbytes, 0, 256));
  slot->type = type;
  slot->nbytes = nbytes;
  slot->ne0 = ne0;
  slot->ne1 = ne1;
  if (pack_now) {
    const size_t pk_bytes = gemm_pack_bytes((int)ne1, (int)ne0);
    if (hipMalloc(&slot->pk, pk_bytes) != hipSuccess) {
      slot->pk = nullptr;
      return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes (packed %s) failed", pk_bytes, name);
    }
    if (neox_rows) {
      void* tmp = nullptr;
      if (hipMalloc(&tmp, pk_bytes) != hipSuccess)
        return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes (packed %s) failed", pk_bytes, name);
      const size_t prow = pk_bytes / ne1;
      hipError_t e = gemm_pack_launch((int)type, slot->ptr, (int)ne1, (int)ne0, tmp, m->stream);
      for (uint64_t r = 0; r < ne1 && e == hipSuccess; r++)
        e = hipMemcpyAsync((char*)slot->pk + r * prow,
                           (const char*)tmp + (size_t)neox_source_row((int)r, c.head_dim) * prow, prow,
                           hipMemcpyDeviceToDevice, m->stream);
      const hipError_t es = hipStreamSynchronize(m->stream);
      (void)hipFree(tmp);
      HIP_TRY(e);
      HIP_TRY(es);
    } else {
      HIP_TRY(gemm_pack_launch((int)type, slot->ptr, (int)ne1, (int)ne0, slot->pk, m->stream));
      HIP_TRY(hipStreamSynchronize(m->stream));
    }
  }
  drop_graphs(m);
  g_err.clear();
  return CHATNET_OK;
}

}  // extern "C"

namespace {

int check_complete(const chatnet_model* m) {
  if (!m->emb.ptr) return fail(CHATNET_ERR_NOT_FOUND, "tensor token_embd.weight not uploaded");
  if (!m->out_norm.ptr) return fail(CHATNET_ERR_NOT_FOUND, "tensor output_norm.weight not uploaded");
  if (!m->out.ptr && (!is_matrix_type(m->emb.type) || !gemv_supports((int)m->emb.type, m->cfg.dim))) {
    // LlamaWeights.cs:89-98 / QwenWeights.cs:103-112 fall back to the tied
    // embedding, which the GEMV then reads as the LM head
    return fail(CHATNET_ERR_INVALID_ARG,
                "output.weight missing: the tied token_embd.weight (type %u) cannot be the LM head at dim %d",
                m->emb.type, m->cfg.dim);
  }
  for (size_t l = 0; l < m->layers.size(); l++) {
    const Layer& L = m->layers[l];
    const DevTensor* ts[] = {&L.attn_norm, &L.ffn_norm, &L.wq, &L.wk, &L.wv, &L.wo, &L.wg, &L.wu, &L.wd};
    const char* nm[] = {"attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    for (int i = 0; i < 9; i++)
      if (!ts[i]->ptr) return fail(CHATNET_ERR_NOT_FOUND, "tensor blk.%zu.%s.weight not uploaded", l, nm[i]);
    // QwenWeights.cs:164-169: with the q bias present, k and v are looked up too
    const char* bn[3] = {"attn_q", "attn_k", "attn_v"};
    if (L.bias_have)
      for (int i = 0; i < 3; i++)
        if (!(L.bias_have & (1u << i)))
          return fail(CHATNET_ERR_NOT_FOUND, "tensor blk.%zu.%s.bias not uploaded", l, bn[i]);
  }
  return CHATNET_OK;
}

// output.weight, or the tied embedding when it is absent (LlamaWeights.cs:89-98).
const DevTensor& lm_head_tensor(const chatnet_model* m) { return m->out.ptr ? m->out : m->emb; }

GemvArgs base_args(const chatnet_model* m, bool decode = false) {
  GemvArgs a;
  memset(&a, 0, sizeof(a));
  a.stop = decode ? m->state + kDecStop : nullptr;
  a.eps = m->cfg.rms_norm_eps;
  a.pos = m->state;
  a.head_dim = m->cfg.head_dim;
  a.rope = m->rope;
  a.kv_dim = m->kv_dim;
  a.kv_f16 = m->cfg.kv_dtype == CHATNET_KV_F16;
  return a;
}

// Launches the forward of the token held in m->state (pos, token); the
// attention covers sequence lengths up to cap (the position's bucket).  In a
// decode loop (`decode`) every launch but the embedding gather exits early
// once the loop's stop flag is set.
int launch_token(chatnet_model* m, bool lm_head, int cap, bool decode = false) {
  const chatnet_config& c = m->cfg;
  hipStream_t st = m->stream;
  const int kvd = m->kv_dim;
  HIP_TRY(embed_launch(embed_w(m->emb), embed_qt(m->emb), c.dim, m->state + 1, m->x, st));
  for (int l = 0; l < c.n_layers; l++) {
    const Layer& L = m->layers[l];
    const size_t loff = (size_t)l * c.context_length * kvd * m->kv_elt;
    GemvArgs a = base_args(m, decode);
    a.K = c.dim;
    a.x = m->x;
    a.norm_w = (const float*)L.attn_norm.ptr;
    a.out[0] = m->q;
    a.kcache = (char*)m->kcache + loff;
    a.vcache = (char*)m->vcache + loff;
    a.bias = L.bias_have ? L.bias : nullptr;  // QwenModel.cs:104-120
    if (L.wq.type == L.wk.type && L.wk.type == L.wv.type) {
      a.w[0] = gemv_w(L.wq);
      a.w[1] = gemv_w(L.wk);
      a.w[2] = gemv_w(L.wv);
      a.seg_rows[0] = c.dim;
      a.seg_rows[1] = kvd;
      a.seg_rows[2] = kvd;
      a.n_vrows = c.dim + 2 * kvd;
      HIP_TRY(gemv_launch(gemv_qt(L.wq), GEMV_EPI_QKV, a, m->num_cus, st));
    } else {
      const DevTensor* ts[3] = {&L.wq, &L.wk, &L.wv};
      const int rows[3] = {c.dim, kvd, kvd};
      for (int s = 0; s < 3; s++) {
        GemvArgs b = a;
        b.w[0] = b.w[1] = b.w[2] = gemv_w(*ts[s]);
        b.seg_rows[0] = s == 0 ? rows[0] : 0;
        b.seg_rows[1] = s == 1 ? rows[1] : 0;
        b.seg_rows[2] = s == 2 ? rows[2] : 0;
        b.n_vrows = rows[s];
        if (b.bias) b.bias += s == 0 ? 0 : c.dim + (s == 2 ? kvd : 0);
        HIP_TRY(gemv_launch(gemv_qt(*ts[s]), GEMV_EPI_QKV, b, m->num_cus, st));
      }
    }
    AttnArgs at;
    memset(&at, 0, sizeof(at));
    at.q = m->q;
    at.kc = a.kcache;
    at.vc = a.vcache;
    at.out = m->att;
    at.pos = m->state;
    at.n_heads = c.n_heads;
    at.kv_mul = c.n_heads / c.n_kv_heads;
    at.head_dim = c.head_dim;
    at.kv_dim = kvd;
    at.ctx = c.context_length;
    at.kv_f16 = a.kv_f16;
    at.scale = 1.0f / sqrtf((float)c.head_dim);  // LlamaModel.cs:248
    const AttnPlan plan = attn_plan(m, cap);
    at.splits = plan.splits;
    at.chunk = plan.chunk;
    at.part_o = m->attn_part_o;
    at.part_ml = m->attn_part_ml;
    at.stop = a.stop;
    at.hsplit = attn_decode_hsplit(c.n_kv_heads, at.kv_mul, plan.splits, m->num_cus);
    HIP_TRY(attn_decode_launch(at, st));

    GemvArgs o = base_args(m, decode);
    o.K = c.dim;
    o.x = m->att;
    o.w[0] = gemv_w(L.wo);
    o.seg_rows[0] = c.dim;
    o.n_vrows = c.dim;
    o.out[0] = m->x;
    const bool fold = plan.splits > 1;  // the O GEMV combines the chunks as it stages x
    if (fold) {
      o.part_o = m->attn_part_o;
      o.part_ml = m->attn_part_ml;
      o.msplits = plan.splits;
      o.mchunk = plan.chunk;
    }
    HIP_TRY(gemv_launch(gemv_qt(L.wo), fold ? GEMV_EPI_ADD_MERGE : GEMV_EPI_ADD, o, m->num_cus, st));

    GemvArgs g = base_args(m, decode);
    g.K = c.dim;
    g.x = m->x;
    g.norm_w = (const float*)L.ffn_norm.ptr;
    if (L.wg.type == L.wu.type) {  // one launch, gate and up rows interleaved
      g.w[0] = gemv_w(L.wg);
      g.w[1] = gemv_w(L.wu);
      g.seg_rows[0] = c.hidden_dim;
      g.seg_rows[1] = c.hidden_dim;
      g.n_vrows = 2 * c.hidden_dim;
      g.out[0] = m->h;
      HIP_TRY(gemv_launch(gemv_qt(L.wg), GEMV_EPI_SWIGLU, g, m->num_cus, st));
    } else {
      // gate and up of different types (each dispatched on its own type,
      // LlamaModel.cs:175-179): two normed GEMVs, then SiLU(gate) * up
      const DevTensor* ts[2] = {&L.wg, &L.wu};
      for (int s = 0; s < 2; s++) {
        GemvArgs b = g;
        b.w[0] = b.w[1] = b.w[2] = gemv_w(*ts[s]);
        b.seg_rows[0] = c.hidden_dim;
        b.n_vrows = c.hidden_dim;
        b.out[0] = m->gu + (size_t)s * c.hidden_dim;
        HIP_TRY(gemv_launch(gemv_qt(*ts[s]), GEMV_EPI_LOGITS, b, m->num_cus, st));
      }
      HIP_TRY(silu_mul_launch(m->gu, m->gu + c.hidden_dim, m->h, c.hidden_dim, st));
    }

    GemvArgs d = base_args(m, decode);
    d.K = c.hidden_dim;
    d.x = m->h;
    d.w[0] = gemv_w(L.wd);
    d.seg_rows[0] = c.dim;
    d.n_vrows = c.dim;
    d.out[0] = m->x;
    HIP_TRY(gemv_launch(gemv_qt(L.wd), GEMV_EPI_ADD, d, m->num_cus, st));
  }
  if (lm_head) {
    GemvArgs o = base_args(m, decode);  // final RMSNorm fused (LlamaModel.cs:203-213)
    o.K = c.dim;
    o.x = m->x;
    o.norm_w = (const float*)m->out_norm.ptr;
    o.w[0] = gemv_w(lm_head_tensor(m));
    o.seg_rows[0] = c.vocab_size;
    o.n_vrows = c.vocab_size;
    o.out[0] = m->logits;
    HIP_TRY(gemv_launch(gemv_qt(lm_head_tensor(m)), GEMV_EPI_LOGITS, o, m->num_cus, st));
  }
  return CHATNET_OK;
}

int ensure_out_tokens(chatnet_model* m, int cap) {
  if (m->out_cap >= cap) return CHATNET_OK;
  if (m->out_tokens) {
    HIP_TRY(hipStreamSynchronize(m->stream));
    (void)hipFree(m->out_tokens);
    m->out_tokens = nullptr;
    m->out_cap = 0;
  }
  if (hipMalloc(&m->out_tokens, sizeof(int) * (size_t)cap) != hipSuccess)
    return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of token buffer failed");
  m->out_cap = cap;
  drop_graphs(m);  // the captured argmax nodes point at the old buffer
  return CHATNET_OK;
}

// Spans of at least this many tokens run as one batch on the MFMA GEMM.
constexpr int kSpanMin = 8;
constexpr int kSpanCap = 512;

// The seven projection matrices of a layer.
struct LayerMats {
  DevTensor* t[7];
};
LayerMats layer_mats(Layer& L) { return {{&L.wq, &L.wk, &L.wv, &L.wo, &L.wg, &L.wu, &L.wd}}; }

// How a span's projections read their weights, per GEMM of the layer (QKV,
// O, gate/up, down): F16 and F32 matrices as their own rows (GEMM_W_F16 /
// GEMM_W_F32), block types from their stored blocks when every matrix of that
// GEMM in every layer is Q4_0 (GEMM_W_Q4_0) or every one is Q4_K
// (GEMM_W_Q4_K), else as packed units (block types mixed freely, made once
// per model).  The matrices one GEMM concatenates (q|k|v) or interleaves
// (gate/up) must share a class (float type or block type); a span whose layers
// cannot (ffn_gate Q4_0 with ffn_up F16, a type neither packable nor float)
// runs token by token.
enum { SG_QKV = 0, SG_O = 1, SG_GU = 2, SG_D = 3 };
struct SpanPlan {
  bool ok = false;
  int fmt[4] = {};
};

SpanPlan span_plan(chatnet_model* m, int n) {
  SpanPlan p;
  if (n < kSpanMin) return p;
  const char* e = getenv("CHATNET_SPAN_BATCH");  // "0": per-token schedule for every span
  if (e && e[0] == '0') return p;
  const chatnet_config& c = m->cfg;
  if (!attn_prefill_supports(c.head_dim, c.n_heads / c.n_kv_heads)) return p;
  // the class of a matrix: a float format, 1 for any block type, -1 for none
  auto cls = [](const DevTensor* t) -> int {
    if (t->type == CHATNET_GGML_F16) return GEMM_W_F16;
    if (t->type == CHATNET_GGML_F32) return GEMM_W_F32;
    if (t->ne0 % 64 == 0 && gemm_pack_supports((int)t->type, (int)t->ne0)) return GEMM_W_PACKED;
    return -1;
  };
  const int group_of[7] = {SG_QKV, SG_QKV, SG_QKV, SG_O, SG_GU, SG_GU, SG_D};
  int gcls[4] = {0, 0, 0, 0};  // 0: not seen yet
  bool all_q4_0[4] = {true, true, true, true}, all_q4_k[4] = {true, true, true, true};
  for (Layer& L : m->layers) {
    const LayerMats lm = layer_mats(L);
    for (int i = 0; i < 7; i++) {
      const DevTensor* t = lm.t[i];
      const int k = cls(t), gi = group_of[i];
      if (k < 0) return p;
      int& g = gcls[gi];
      if (g == 0) g = k;
      else if (g != k) return p;
      if (t->type != CHATNET_GGML_Q4_0 || !gemm_supports(CHATNET_GGML_Q4_0, (int)t->ne0)) all_q4_0[gi] = false;
      if (t->type != CHATNET_GGML_Q4_K || t->ne0 % 256) all_q4_k[gi] = false;
    }
  }
  for (int g = 0; g < 4; g++) {
    if (gcls[g] != GEMM_W_PACKED) p.fmt[g] = gcls[g];
    else p.fmt[g] = all_q4_0[g] ? GEMM_W_Q4_0 : (all_q4_k[g] ? GEMM_W_Q4_K : GEMM_W_PACKED);
  }
  p.ok = true;
  return p;
}

// Packs every projection matrix of a packed-unit GEMM not yet packed (once
// per upload).
int ensure_span_packs(chatnet_model* m, const SpanPlan& plan) {
  const int group_of[7] = {SG_QKV, SG_QKV, SG_QKV, SG_O, SG_GU, SG_GU, SG_D};
  for (Layer& L : m->layers) {
    const LayerMats lm = layer_mats(L);
    for (int i = 0; i < 7; i++) {
      DevTensor* t = lm.t[i];
      if (t->pk || plan.fmt[group_of[i]] != GEMM_W_PACKED) continue;
      const size_t bytes = gemm_pack_bytes((int)t->ne1, (int)t->ne0);
      if (hipMalloc(&t->pk, bytes) != hipSuccess) {
        t->pk = nullptr;
        return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes (packed weights) failed", bytes);
      }
      HIP_TRY(gemm_pack_launch((int)t->type, t->ptr, (int)t->ne1, (int)t->ne0, t->pk, m->stream));
    }
  }
  return CHATNET_OK;
}

int ensure_span_buffers(chatnet_model* m) {
  if (m->span_cap) return CHATNET_OK;
  const chatnet_config& c = m->cfg;
  const int cap = c.context_length < kSpanCap ? c.context_length : kSpanCap;
  struct { void** p; size_t n; } allocs[] = {
      {(void**)&m->sp_x, sizeof(float) * cap * c.dim},
      {(void**)&m->sp_xb, sizeof(uint16_t) * 2 * cap * c.dim},
      {(void**)&m->sp_hb, sizeof(uint16_t) * 2 * cap * c.hidden_dim},
      {(void**)&m->sp_qkv, sizeof(float) * cap * (c.dim + 2 * m->kv_dim)},
      {(void**)&m->sp_tok, sizeof(int) * cap},
  };
  for (auto& a : allocs) {
    if (hipMalloc(a.p, a.n) != hipSuccess) return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes failed", a.n);
  }
  m->span_cap = cap;
  return CHATNET_OK;
}

int span_gemm(chatnet_model* m, GemmArgs& g, int* splits_left = nullptr) {
  g.precise = 1;
  const size_t need = gemm_workspace_bytes(g.M, g.N, g.K, m->num_cus, true, g.packed);
  if (need > m->sp_part_bytes) {
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (m->sp_part) (void)hipFree(m->sp_part);
    m->sp_part = nullptr;
    m->sp_part_bytes = 0;
    if (hipMalloc(&m->sp_part, need) != hipSuccess)
      return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of %zu bytes failed", need);
    m->sp_part_bytes = need;
  }
  g.part = m->sp_part;
  HIP_TRY(gemm_launch(g, m->num_cus, m->stream, splits_left));
  return CHATNET_OK;
}

// LlamaModel.Forward (LlamaModel.cs:93-238) over tokens[0..n) at positions
// position.. as batches of up to span_cap tokens: every projection is one
// MFMA GEMM over the batch (its weights read as `plan` says), attention
// is causal over the cache, and the LM head runs for the last token only
// (LlamaModel.cs:207).
int run_span(chatnet_model* m, const int32_t* tokens, int n, int position, const SpanPlan& plan) {
  int rc = ensure_span_buffers(m);
  if (rc) return rc;
  if ((rc = ensure_span_packs(m, plan))) return rc;
  auto wsrc = [&plan](const DevTensor& t, int grp) {
    return (const uint8_t*)(plan.fmt[grp] == GEMM_W_PACKED ? t.pk : t.ptr);
  };
  const chatnet_config& c = m->cfg;
  hipStream_t st = m->stream;
  const int kvd = m->kv_dim, qkv_ld = c.dim + 2 * kvd;
  uint16_t* xb_lo = m->sp_xb + (size_t)m->span_cap * c.dim;
  uint16_t* hb_lo = m->sp_hb + (size_t)m->span_cap * c.hidden_dim;
  int last_rows = 0;
  int pending = 0;  // K splits of a residual-add GEMM whose partials the next norm folds in
  int* defer = c.dim <= 4096 ? &pending : nullptr;  // the fold's register budget
  for (int s0 = 0; s0 < n; s0 += m->span_cap) {
    const int cn = n - s0 < m->span_cap ? n - s0 : m->span_cap;
    const int p0 = position + s0;
    HIP_TRY(hipMemcpyAsync(m->sp_tok, tokens + s0, sizeof(int) * cn, hipMemcpyHostToDevice, st));
    HIP_TRY(embed_launch(embed_w(m->emb), embed_qt(m->emb), c.dim, m->sp_tok, m->sp_x, st, cn));
    for (int l = 0; l < c.n_layers; l++) {
      const Layer& L = m->layers[l];
      const size_t loff = (size_t)l * c.context_length * kvd * m->kv_elt;
      void* kc = (char*)m->kcache + loff;
      void* vc = (char*)m->vcache + loff;
      // the previous layer's down projection may have left its K-split
      // partials: the residual add completes here, with the norm
      HIP_TRY(add_rmsnorm_span_launch(m->sp_x, m->sp_part, pending, (const float*)L.attn_norm.ptr, c.rms_norm_eps,
                                      m->sp_xb, xb_lo, cn, c.dim, st));
      pending = 0;
      GemmArgs g;
      memset(&g, 0, sizeof(g));
      g.qtype = CHATNET_GGML_Q4_0;
      g.packed = plan.fmt[SG_QKV];
      g.w[0] = wsrc(L.wq, SG_QKV);
      g.w[1] = wsrc(L.wk, SG_QKV);
      g.w[2] = wsrc(L.wv, SG_QKV);
      g.seg_rows[0] = c.dim;
      g.seg_rows[1] = kvd;
      g.seg_rows[2] = kvd;
      g.seg_mode = GEMM_SEG_CONCAT;
      g.M = qkv_ld;
      g.K = c.dim;
      g.N = cn;
      g.xb = m->sp_xb;
      g.xb_lo = xb_lo;
      g.epi = GEMV_EPI_STORE;
      g.y = m->sp_qkv;
      g.ldy = qkv_ld;
      int qkv_splits = 0;  // partials the RoPE/KV kernel sums itself
      if ((rc = span_gemm(m, g, &qkv_splits))) return rc;

      RopeKvArgs r;
      memset(&r, 0, sizeof(r));
      r.qkv = m->sp_qkv;
      r.ld = qkv_ld;
      r.dim = c.dim;
      r.kv_dim = kvd;
      r.head_dim = c.head_dim;
      r.p0 = p0;
      r.rope = m->rope;
      r.kcache = kc;
      r.vcache = vc;
      r.kv_f16 = c.kv_dtype == CHATNET_KV_F16;
      r.bias = L.bias_have ? L.bias : nullptr;
      r.part = m->sp_part;
      r.splits = qkv_splits;
      HIP_TRY(rope_kv_launch(r, cn, st));

      PrefillAttnArgs at;
      memset(&at, 0, sizeof(at));
      at.qkv = m->sp_qkv;
      at.ld = qkv_ld;
      at.kc = kc;
      at.vc = vc;
      at.out = m->sp_xb;
      at.out_lo = xb_lo;
      at.ldo = c.dim;
      at.n = cn;
      at.p0 = p0;
      at.n_heads = c.n_heads;
      at.kv_mul = c.n_heads / c.n_kv_heads;
      at.head_dim = c.head_dim;
      at.kv_dim = kvd;
      at.kv_f16 = r.kv_f16;
      at.scale = 1.0f / sqrtf((float)c.head_dim);  // LlamaModel.cs:248
      HIP_TRY(attn_prefill_launch(at, st));

      GemmArgs o;
      memset(&o, 0, sizeof(o));
      o.qtype = CHATNET_GGML_Q4_0;
      o.packed = plan.fmt[SG_O];
      o.w[0] = wsrc(L.wo, SG_O);
      o.seg_rows[0] = c.dim;
      o.M = c.dim;
      o.K = c.dim;
      o.N = cn;
      o.xb = m->sp_xb;
      o.xb_lo = xb_lo;
      o.epi = GEMV_EPI_ADD;
      o.y = m->sp_x;
      o.ldy = c.dim;
      if ((rc = span_gemm(m, o, defer))) return rc;

      HIP_TRY(add_rmsnorm_span_launch(m->sp_x, m->sp_part, pending, (const float*)L.ffn_norm.ptr, c.rms_norm_eps,
                                      m->sp_xb, xb_lo, cn, c.dim, st));
      pending = 0;
      GemmArgs gu;
      memset(&gu, 0, sizeof(gu));
      gu.qtype = CHATNET_GGML_Q4_0;
      gu.packed = plan.fmt[SG_GU];
      gu.w[0] = wsrc(L.wg, SG_GU);
      gu.w[1] = wsrc(L.wu, SG_GU);
      gu.seg_rows[0] = c.hidden_dim;
      gu.seg_rows[1] = c.hidden_dim;
      gu.seg_mode = GEMM_SEG_INTERLEAVE;
      gu.M = 2 * c.hidden_dim;
      gu.K = c.dim;
      gu.N = cn;
      gu.xb = m->sp_xb;
      gu.xb_lo = xb_lo;
      gu.epi = GEMV_EPI_SWIGLU;
      gu.hb = m->sp_hb;
      gu.hb_lo = hb_lo;
      gu.ldh = c.hidden_dim;
      if ((rc = span_gemm(m, gu))) return rc;

      GemmArgs d;
      memset(&d, 0, sizeof(d));
      d.qtype = CHATNET_GGML_Q4_0;
      d.packed = plan.fmt[SG_D];
      d.w[0] = wsrc(L.wd, SG_D);
      d.seg_rows[0] = c.dim;
      d.M = c.dim;
      d.K = c.hidden_dim;
      d.N = cn;
      d.xb = m->sp_hb;
      d.xb_lo = hb_lo;
      d.epi = GEMV_EPI_ADD;
      d.y = m->sp_x;
      d.ldy = c.dim;
      // the last layer's residual add completes here (the LM head reads x)
      if ((rc = span_gemm(m, d, l + 1 < c.n_layers ? defer : nullptr))) return rc;
    }
    last_rows = cn;
  }
  // final RMSNorm + LM head of the last token (LlamaModel.cs:203-213)
  GemvArgs o = base_args(m);
  o.K = c.dim;
  o.x = m->sp_x + (size_t)(last_rows - 1) * c.dim;
  o.norm_w = (const float*)m->out_norm.ptr;
  o.w[0] = gemv_w(lm_head_tensor(m));
  o.seg_rows[0] = c.vocab_size;
  o.n_vrows = c.vocab_size;
  o.out[0] = m->logits;
  HIP_TRY(gemv_launch(gemv_qt(lm_head_tensor(m)), GEMV_EPI_LOGITS, o, m->num_cus, st));
  m->have_logits = true;
  m->next_pos = position + n;
  m->last_tok = tokens[n - 1];
  return CHATNET_OK;
}

int run_prompt(chatnet_model* m, const int32_t* tokens, int n, int position) {
  const SpanPlan plan = span_plan(m, n);
  if (plan.ok) return run_span(m, tokens, n, position, plan);
  for (int t = 0; t < n; t++) {
    HIP_TRY(set_state_launch(m->state, position + t, tokens[t], -1, m->stream));
    int rc = launch_token(m, t == n - 1, bucket_cap(m, position + t + 1));
    if (rc) return rc;
  }
  m->have_logits = true;
  m->next_pos = position + n;
  m->last_tok = tokens[n - 1];
  return CHATNET_OK;
}

// chatnet_matmul and chatnet_matmul_noalloc: the same kernels; the batched
// path's scratch (fp16 x and its column scales, then the K-split partials) comes from the per-stream
// workspace, or with `noalloc` from the fixed per-device scratch array.
int matmul_impl(uint32_t type, const void* w_dev, const float* x_dev, float* y_dev, int M, int K, int N, void* stream,
                bool noalloc) {
  if (!w_dev || !x_dev || !y_dev) return fail(CHATNET_ERR_INVALID_ARG, "null device pointer");
  if (M <= 0 || K <= 0 || N <= 0) return fail(CHATNET_ERR_INVALID_ARG, "M, K, N must be positive");
  if (!is_matrix_type(type)) return fail(CHATNET_ERR_UNSUPPORTED_TYPE, "matmul type %u not supported", type);
  if (!gemv_supports((int)type, K))
    return fail(CHATNET_ERR_INVALID_ARG, "K=%d not supported for type %u (block multiple, at most 16384)", K, type);
  if ((reinterpret_cast<uintptr_t>(w_dev) & 15) || (reinterpret_cast<uintptr_t>(x_dev) & 15))
    return fail(CHATNET_ERR_INVALID_ARG, "w_dev and x_dev must be 16-byte aligned");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  const int cus = device_cus(dev);
  hipStream_t st = (hipStream_t)stream;
  // Q4_0 reads its raw blocks; the other block types (not in the no-allocation
  // variant) are packed into the workspace first, one pass over W.  The types
  // the GEMV reads only as packed units are packed for every N, in both
  // variants.
  // Q4_0 with a few columns: the GEMV over all of them at once, one pass over W.
  // Its digit dots cost ALU and LDS time per column, so from 8 columns on it
  // is taken only up to the size where it measured faster than the MFMA GEMM
  // (8 columns of a 4096 x 4096 matrix: 14.8 against 17.2 us; 11008 x 4096:
  // 27.6 against 23.4 us).
  if (type == CHATNET_GGML_Q4_0 && N >= 2 && gemv_cols_max(K) >= 2 &&
      (N < 8 || (N <= 16 && (long long)M * K * N <= 8LL * 4096 * 4096))) {
    HIP_TRY(gemv_cols_launch(w_dev, x_dev, y_dev, M, K, N, cus, st));
    g_err.clear();
    return CHATNET_OK;
  }
  const bool raw = gemm_supports((int)type, K);
  const bool must_pack = gemv_needs_pack((int)type);
  const bool batched = N >= 8 && (raw || must_pack || (!noalloc && gemm_pack_supports((int)type, K)));
  const bool pack = must_pack || (batched && !raw);
  const uint8_t* wp = (const uint8_t*)w_dev;
  if (batched || pack) {
    // [stream-K tile counters | fp16 x | per-column x scales | K-split or
    // stream-K partials | packed W]: the counters in the per-stream workspace
    // only (the no-allocation variant runs no stream-K launch), the next
    // three for the batched path only
    const size_t cnt_bytes = noalloc ? 0 : kMatmulCounterBytes;
    const size_t xh_bytes = cnt_bytes + (batched ? ((size_t)N * K * sizeof(uint16_t) + 255) & ~(size_t)255 : 0);
    const size_t xb_bytes = batched ? xh_bytes + (((size_t)N * sizeof(float) + 255) & ~(size_t)255) : cnt_bytes;
    const size_t part_bytes =
        batched ? (gemm_workspace_bytes(M, N, K, cus, false, pack, !noalloc) + 255) & ~(size_t)255 : 0;
    const size_t pack_bytes = pack ? gemm_pack_bytes(M, K) : 0;
    const size_t need = xb_bytes + part_bytes + pack_bytes;
    char* ws = nullptr;
    int rc;
    if (noalloc) {
      if (need > kNoAllocScratchBytes)
        return fail(CHATNET_ERR_INVALID_ARG,
                    "chatnet_matmul_noalloc: M=%d K=%d N=%d needs %zu bytes of scratch, more than its %zu", M, K, N,
                    need, kNoAllocScratchBytes);
      rc = noalloc_scratch(dev, &ws);
    } else {
      rc = matmul_workspace(dev, st, need, &ws);
    }
    if (rc) return rc;
    if (pack) {
      HIP_TRY(gemm_pack_launch((int)type, w_dev, M, K, ws + xb_bytes + part_bytes, st));
      wp = (const uint8_t*)(ws + xb_bytes + part_bytes);
    }
    if (batched) {
      // x -> per-column scaled fp16 into the scratch, then the MFMA GEMM
      HIP_TRY(to_f16_scaled_launch(x_dev, (uint16_t*)(ws + cnt_bytes), (float*)(ws + xh_bytes), N, K, st));
      GemmArgs g;
      memset(&g, 0, sizeof(g));
      g.qtype = (int)type;
      g.packed = pack;
      g.w[0] = g.w[1] = g.w[2] = wp;
      g.seg_rows[0] = M;
      g.seg_mode = GEMM_SEG_SINGLE;
      g.M = M;
      g.K = K;
      g.N = N;
      g.xb = (const uint16_t*)(ws + cnt_bytes);
      g.xinv = (const float*)(ws + xh_bytes);
      g.epi = GEMV_EPI_STORE;
      g.y = y_dev;
      g.ldy = M;
      g.part = part_bytes ? (float*)(ws + xb_bytes) : nullptr;
      g.tile_cnt = noalloc ? nullptr : (unsigned*)ws;
      HIP_TRY(gemm_launch(g, cus, st));
      g_err.clear();
      return CHATNET_OK;
    }
  }
  const int qt = pack ? kGemvPacked : (int)type;
  for (int n = 0; n < N; n++) {  // one fused GEMV per column
    GemvArgs a;
    memset(&a, 0, sizeof(a));
    a.w[0] = a.w[1] = a.w[2] = wp;
    a.seg_rows[0] = M;
    a.n_vrows = M;
    a.K = K;
    a.x = x_dev + (size_t)n * K;
    a.out[0] = y_dev + (size_t)n * M;
    HIP_TRY(gemv_launch(qt, GEMV_EPI_STORE, a, cus, st));
  }
  g_err.clear();
  return CHATNET_OK;
}

int validate_tokens(const chatnet_model* m, const int32_t* tokens, int n, int position) {
  if (!tokens || n <= 0) return fail(CHATNET_ERR_INVALID_ARG, "tokens must be non-empty");
  if (position < 0 || (long long)position + n > m->cfg.context_length)
    return fail(CHATNET_ERR_OUT_OF_RANGE, "positions %d..%d exceed context_length %d", position,
                position + n - 1, m->cfg.context_length);
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size)
      return fail(CHATNET_ERR_OUT_OF_RANGE, "token id %d at index %d outside [0, %d)", tokens[i], i, m->cfg.vocab_size);
  return CHATNET_OK;
}

}  // namespace

extern "C" {

int chatnet_forward(chatnet_model* m, const int32_t* tokens, int n, int position, float* logits_host) {
  if (!m) return fail(CHATNET_ERR_INVALID_ARG, "null model");
  int rc = validate_tokens(m, tokens, n, position);
  if (rc) return rc;
  if ((rc = check_complete(m))) return rc;
  HIP_TRY(hipSetDevice(m->device));
  if ((rc = run_prompt(m, tokens, n, position))) return rc;
  if (logits_host)
    HIP_TRY(hipMemcpyAsync(logits_host, m->logits, sizeof(float) * m->cfg.vocab_size, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  g_err.clear();
  return CHATNET_OK;
}

int chatnet_get_logits(chatnet_model* m, float* logits_host) {
  if (!m || !logits_host) return fail(CHATNET_ERR_INVALID_ARG, "null argument");
  if (!m->have_logits) return fail(CHATNET_ERR_INVALID_ARG, "no forward has produced logits yet");
  HIP_TRY(hipSetDevice(m->device));
  HIP_TRY(hipMemcpyAsync(logits_host, m->logits, sizeof(float) * m->cfg.vocab_size, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  return CHATNET_OK;
}

int chatnet_argmax(chatnet_model* m, int32_t* out_token) {
  if (!m || !out_token) return fail(CHATNET_ERR_INVALID_ARG, "null argument");
  if (!m->have_logits) return fail(CHATNET_ERR_INVALID_ARG, "no forward has produced logits yet");
  HIP_TRY(hipSetDevice(m->device));
  HIP_TRY(argmax_launch(m->logits, m->cfg.vocab_size, m->state, nullptr, 0, m->stream));
  int st[4];
  HIP_TRY(hipMemcpyAsync(st, m->state, sizeof(st), hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  *out_token = st[1];
  return CHATNET_OK;
}

// The decode half of InferenceEngine.Generate (InferenceEngine.cs:241-307):
// each token is picked by the argmax or, when `sampled`, by the temperature
// sampler (parameters in m->sparams, the i-th pick's draw in m->draws[i]).
static int decode_loop(chatnet_model* m, int max_tokens, int32_t eos_token, int32_t* out_tokens, int* n_out,
                       bool sampled) {
  *n_out = 0;
  if (!m->have_logits) return fail(CHATNET_ERR_INVALID_ARG, "no forward has produced logits yet");
  int rc = check_complete(m);
  if (rc) return rc;
  HIP_TRY(hipSetDevice(m->device));
  if (max_tokens == 0) {  // InferenceEngine.cs:256: the loop body never runs
    g_err.clear();
    return CHATNET_OK;
  }
  const int ctx = m->cfg.context_length;
  const int p0 = m->next_pos;  // position of the first generated token
  // InferenceEngine.cs:256-307: token i is emitted unless it is EOS, then the
  // loop stops if its position p0+i >= ctx-1; otherwise it is forwarded there
  // and the next one sampled.  So at most `room` tokens are forwarded and
  // room + 1 emitted (one, the first pick, when the cache is already full).
  const int room = ctx - 1 - p0;
  const int forwards = max_tokens < room ? max_tokens : (room > 0 ? room : 0);
  const int emitted = max_tokens < (room > 0 ? room : 0) + 1 ? max_tokens : (room > 0 ? room : 0) + 1;
  if ((rc = ensure_out_tokens(m, max_tokens + 2))) return rc;
  // step counter = 0, stop flag cleared, then the first pick from the last
  // forward's logits.  A pick of EOS sets the stop flag: every later launch of
  // the loop returns early, so the cache, the logits and the state stay those
  // of the last token forwarded before it (InferenceEngine.cs:258-261 breaks
  // before forwarding EOS).
  auto pick = [m, sampled]() {
    return sampled ? sample_launch(m->logits, m->cfg.vocab_size, m->sparams, m->draws, m->state, m->out_tokens,
                                   m->out_cap, m->sample_p, m->stream)
                   : argmax_launch(m->logits, m->cfg.vocab_size, m->state, m->out_tokens, m->out_cap, m->stream);
  };
  hipGraphExec_t* graphs = sampled ? m->sgraphs : m->graphs;
  HIP_TRY(set_state_launch(m->state, p0 - 1, m->last_tok, 0, m->stream, eos_token >= 0 ? eos_token : -1));
  HIP_TRY(pick());
  // CHATNET_DECODE_GRAPH=0 issues the same per-step launches directly instead
  // of replaying the captured graph (the kernels and their order are
  // identical; kernel-trace profiles of the decode step are taken this way).
  const char* ge = getenv("CHATNET_DECODE_GRAPH");
  const bool use_graph = !(ge && ge[0] == '0');
  // Step i forwards the token at position p0+i (sequence length p0+i+1).
  if (forwards > 0 && !use_graph) {
    for (int i = 0; i < forwards; i++) {
      if ((rc = launch_token(m, true, bucket_cap(m, p0 + i + 1), true))) return rc;
      HIP_TRY(pick());
    }
  } else if (forwards > 0) {
    for (int i = 0; i < forwards; i++) {
      const int k = bucket_index(m, p0 + i + 1);
      if (!graphs[k]) {
        hipGraph_t g = nullptr;
        HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        const int lrc = launch_token(m, true, bucket_cap(m, p0 + i + 1), true);
        const hipError_t ae = lrc ? hipSuccess : pick();
        // the capture is always ended, so the stream leaves capture mode, and
        // the graph it returns is destroyed on every path
        const hipError_t ee = hipStreamEndCapture(m->stream, &g);
        hipError_t ie = hipSuccess;
        if (!lrc && ae == hipSuccess && ee == hipSuccess) ie = hipGraphInstantiate(&graphs[k], g, nullptr, nullptr, 0);
        if (g) (void)hipGraphDestroy(g);
        if (lrc) return lrc;
        if (ae != hipSuccess) return fail(CHATNET_ERR_HIP, "sampler capture: %s", hipGetErrorString(ae));
        if (ee != hipSuccess) return fail(CHATNET_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(ee));
        if (ie != hipSuccess) {
          graphs[k] = nullptr;
          return fail(CHATNET_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(ie));
        }
      }
      HIP_TRY(hipGraphLaunch(graphs[k], m->stream));
    }
  }
  std::vector<int> buf((size_t)emitted + 2);
  HIP_TRY(hipMemcpyAsync(buf.data(), m->out_tokens, sizeof(int) * emitted, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  int nout = 0;
  while (nout < emitted && !(eos_token >= 0 && buf[nout] == eos_token)) {  // InferenceEngine.cs:258-261
    out_tokens[nout] = buf[nout];
    nout++;
  }
  *n_out = nout;
  // tokens 0 .. done-1 were forwarded (EOS never is): the cache holds
  // positions < p0 + done and the logits are those of token done-1
  const int done = nout < forwards ? nout : forwards;
  if (done > 0) {
    m->next_pos = p0 + done;
    m->last_tok = buf[done - 1];
  }
  g_err.clear();
  return CHATNET_OK;
}

int chatnet_decode_greedy(chatnet_model* m, int max_tokens, int32_t eos_token, int32_t* out_tokens, int* n_out) {
  if (!m || !out_tokens || !n_out) return fail(CHATNET_ERR_INVALID_ARG, "null argument");
  *n_out = 0;
  if (max_tokens < 0) return fail(CHATNET_ERR_INVALID_ARG, "max_tokens must be >= 0");
  return decode_loop(m, max_tokens, eos_token, out_tokens, n_out, false);
}

int chatnet_generate_greedy(chatnet_model* m, const int32_t* prompt, int n_prompt, int max_tokens,
                            int32_t eos_token, int32_t* out_tokens, int* n_out) {
  if (!m || !out_tokens || !n_out) return fail(CHATNET_ERR_INVALID_ARG, "null argument");
  *n_out = 0;
  if (max_tokens < 0) return fail(CHATNET_ERR_INVALID_ARG, "max_tokens must be >= 0");
  int rc = validate_tokens(m, prompt, n_prompt, 0);
  if (rc) return rc;
  if ((rc = check_complete(m))) return rc;
  HIP_TRY(hipSetDevice(m->device));
  if ((rc = run_prompt(m, prompt, n_prompt, 0))) return rc;  // InferenceEngine.cs:235-239
  return chatnet_decode_greedy(m, max_tokens, eos_token, out_tokens, n_out);
}

int chatnet_sample(chatnet_model* m, float temperature, int top_k, float top_p, float r, int32_t* out_token) {
  if (!m || !out_token) return fail(CHATNET_ERR_INVALID_ARG, "null argument");
  if (temperature <= 0.0f) return chatnet_argmax(m, out_token);  // TemperatureSampler.cs:37-41
  if (!m->have_logits) return fail(CHATNET_ERR_INVALID_ARG, "no forward has produced logits yet");
  if (top_k < 1 || top_k > kSampleMaxK) return fail(CHATNET_ERR_INVALID_ARG, "top_k must be in [1, %d]", kSampleMaxK);
  HIP_TRY(hipSetDevice(m->device));
  const SampleParams sp{1.0f / temperature, top_k, top_p, r};  // invTemp as TemperatureSampler.cs:50
  HIP_TRY(hipMemcpyAsync(m->sparams, &sp, sizeof(sp), hipMemcpyHostToDevice, m->stream));
  HIP_TRY(sample_launch(m->logits, m->cfg.vocab_size, m->sparams, nullptr, m->state, nullptr, 0, m->sample_p,
                        m->stream));
  int st[4];
  HIP_TRY(hipMemcpyAsync(st, m->state, sizeof(st), hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  *out_token = st[1];
  return CHATNET_OK;
}

int chatnet_generate_sampled(chatnet_model* m, const int32_t* prompt, int n_prompt, int max_tokens, float temperature,
                             int top_k, float top_p, int32_t seed, int32_t eos_token, int32_t* out_tokens,
                             int* n_out) {
  if (temperature <= 0.0f)  // greedy fallback, no draws consumed (TemperatureSampler.cs:37-41)
    return chatnet_generate_greedy(m, prompt, n_prompt, max_tokens, eos_token, out_tokens, n_out);
  if (!m || !out_tokens || !n_out) return fail(CHATNET_ERR_INVALID_ARG, "null argument");
  *n_out = 0;
  if (max_tokens < 0) return fail(CHATNET_ERR_INVALID_ARG, "max_tokens must be >= 0");
  if (top_k < 1 || top_k > kSampleMaxK) return fail(CHATNET_ERR_INVALID_ARG, "top_k must be in [1, %d]", kSampleMaxK);
  int rc = validate_tokens(m, prompt, n_prompt, 0);
  if (rc) return rc;
  if ((rc = check_complete(m))) return rc;
  HIP_TRY(hipSetDevice(m->device));
  // pick i takes the i-th NextDouble of the sampler's Random (TemperatureSampler.cs:29, :97)
  const int ndraw = max_tokens + 2;
  if (m->draws_cap < ndraw) {
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (m->draws) (void)hipFree(m->draws);
    m->draws = nullptr;
    m->draws_cap = 0;
    if (hipMalloc(&m->draws, sizeof(float) * (size_t)ndraw) != hipSuccess)
      return fail(CHATNET_ERR_OUT_OF_MEMORY, "hipMalloc of the draw buffer failed");
    m->draws_cap = ndraw;
    drop_graphs(m);  // captured sampler nodes point at the old buffer
  }
  NetRandom rng(seed >= 0 ? seed : (int32_t)(std::random_device{}() & 0x7FFFFFFFu));
  std::vector<float> d((size_t)ndraw);
  for (auto& v : d) v = (float)rng.next_double();
  const SampleParams sp{1.0f / temperature, top_k, top_p, 0.0f};
  HIP_TRY(hipMemcpyAsync(m->draws, d.data(), sizeof(float) * d.size(), hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipMemcpyAsync(m->sparams, &sp, sizeof(sp), hipMemcpyHostToDevice, m->stream));
  if ((rc = run_prompt(m, prompt, n_prompt, 0))) return rc;  // InferenceEngine.cs:235-239
  return decode_loop(m, max_tokens, eos_token, out_tokens, n_out, true);
}

int chatnet_net_random(int32_t seed, int n, double* out) {
  if (n < 0 || (n > 0 && !out)) return fail(CHATNET_ERR_INVALID_ARG, "invalid arguments to chatnet_net_random");
  NetRandom rng(seed);
  for (int i = 0; i < n; i++) out[i] = rng.next_double();
  return CHATNET_OK;
}

int chatnet_matmul(uint32_t type, const void* w_dev, const float* x_dev, float* y_dev, int M, int K, int N,
                   void* stream) {
  return matmul_impl(type, w_dev, x_dev, y_dev, M, K, N, stream, false);
}

int chatnet_matmul_noalloc(uint32_t type, const void* w_dev, const float* x_dev, float* y_dev, int M, int K, int N,
                           void* stream) {
  return matmul_impl(type, w_dev, x_dev, y_dev, M, K, N, stream, true);
}

}  // extern "C"
