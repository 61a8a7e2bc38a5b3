// probe_span_gemm.hip — the span GEMM (gemm_s_kernel through gemm_launch, as
// the forward pass runs it) at the four TinyLlama-shaped projections of a
// 512-token span, in a stand-alone program (not part of the library) that a
// counter run can profile without the Python host.
//
// Per shape: 22 distinct weight copies (one per layer, random Q4_0 blocks
// with scales over six octaves), x as the fp16 hi + lo planes in the
// cn_span_pos order a producer writes.  First a check: the STORE epilogue on
// layer 0 against a double-precision dot of the same dequantized weights and
// planes on 2000 sampled outputs (max |error| / sum |w x| must stay below
// 1e-6).  Then the timing: 22 launches with the shape's real epilogue (STORE
// for QKV, residual ADD for O and down, SWIGLU for gate/up) between HIP
// events; K-split shapes include their reduce launch.
#include "gemm.hip"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define CK(x)                                                              \
  do {                                                                     \
    hipError_t e_ = (x);                                                   \
    if (e_ != hipSuccess) {                                                \
      printf("%s: %s\n", #x, hipGetErrorString(e_));                       \
      exit(1);                                                             \
    }                                                                      \
  } while (0)

namespace {

uint16_t host_f2h(float f) {
  _Float16 h = (_Float16)f;
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}
float host_h2f(uint16_t u) {
  _Float16 h;
  memcpy(&h, &u, 2);
  return (float)h;
}

struct Shape {
  const char* name;
  int M, K, epi, seg;
};

// splitmix64: the probe's weights and inputs
uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t next_u64() {
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

int main() {
  const int L = 22, N = 512;
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  hipStream_t st;
  CK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  const Shape shapes[] = {{"QKV", 2560, 2048, GEMV_EPI_STORE, GEMM_SEG_SINGLE},
                          {"O", 2048, 2048, GEMV_EPI_ADD, GEMM_SEG_SINGLE},
                          {"gate/up", 11264, 2048, GEMV_EPI_SWIGLU, GEMM_SEG_INTERLEAVE},
                          {"down", 2048, 5632, GEMV_EPI_ADD, GEMM_SEG_SINGLE}};
  const int KM = 5632, MM = 11264;
  std::vector<float> xf((size_t)N * KM);
  for (float& v : xf) v = (float)((double)(next_u64() >> 11) * (4.0 / 9007199254740992.0) - 2.0);
  uint16_t *xh, *xl, *hb, *hbl;
  float *y, *part;
  CK(hipMalloc(&xh, xf.size() * 2));
  CK(hipMalloc(&xl, xf.size() * 2));
  CK(hipMalloc(&y, (size_t)N * MM * 4));
  CK(hipMalloc(&hb, (size_t)N * (MM / 2) * 2));
  CK(hipMalloc(&hbl, (size_t)N * (MM / 2) * 2));
  CK(hipMemset(y, 0, (size_t)N * MM * 4));
  size_t part_bytes = 256;
  for (const Shape& s : shapes) part_bytes = std::max(part_bytes, gemm_workspace_bytes(s.M, N, s.K, cus, true, false));
  CK(hipMalloc(&part, part_bytes));

  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  printf("device: %d CUs; N = %d, %d weight copies per shape\n", cus, N, L);
  int bad = 0;
  double total_us = 0;
  for (const Shape& s : shapes) {
    // x rows of length K from the first N*K values, in the span order
    std::vector<uint16_t> ph((size_t)N * s.K), pl((size_t)N * s.K);
    for (int n = 0; n < N; n++)
      for (int k = 0; k < s.K; k++) {
        const float v = xf[(size_t)n * s.K + k];
        const uint16_t h = host_f2h(v);
        ph[(size_t)n * s.K + cn_span_pos(k)] = h;
        pl[(size_t)n * s.K + cn_span_pos(k)] = host_f2h(v - host_h2f(h));
      }
    CK(hipMemcpy(xh, ph.data(), ph.size() * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(xl, pl.data(), pl.size() * 2, hipMemcpyHostToDevice));
    const int nseg = s.seg == GEMM_SEG_INTERLEAVE ? 2 : 1;
    const size_t bytes = (size_t)(s.M / nseg) * (s.K / 32) * 18;
    std::vector<uint8_t> hw(bytes);
    for (size_t b = 0; b < bytes; b += 18) {
      const float base = 0.0005f * (float)(1 << (next_u64() % 6));
      const uint16_t d = host_f2h(base * (1.0f + (float)(next_u64() & 1023) / 1024.0f));
      memcpy(&hw[b], &d, 2);
      for (int j = 2; j < 18; j++) hw[b + j] = (uint8_t)next_u64();
    }
    std::vector<uint8_t*> w(L * nseg);
    for (uint8_t*& p : w) {
      CK(hipMalloc(&p, bytes));
      CK(hipMemcpy(p, hw.data(), bytes, hipMemcpyHostToDevice));
    }
    auto args = [&](int l, int epi) {
      GemmArgs a{};
      a.qtype = 2;
      a.w[0] = w[nseg * l];
      a.w[1] = a.w[2] = w[nseg * l + nseg - 1];
      a.seg_rows[0] = a.seg_rows[1] = s.M / nseg;
      a.seg_mode = s.seg;
      a.M = s.M;
      a.K = s.K;
      a.N = N;
      a.xb = xh;
      a.xb_lo = xl;
      a.precise = 1;
      a.epi = epi;
      a.y = y;
      a.ldy = s.M;
      a.hb = hb;
      a.hb_lo = hbl;
      a.ldh = s.M / 2;
      a.part = part;
      return a;
    };
    // check (both interleaved segments hold the same bytes)
    CK(gemm_launch(args(0, GEMV_EPI_STORE), cus, st));
    CK(hipStreamSynchronize(st));
    std::vector<float> hy((size_t)N * s.M);
    CK(hipMemcpy(hy.data(), y, hy.size() * 4, hipMemcpyDeviceToHost));
    double worst = 0;
    for (int t = 0; t < 2000; t++) {
      const int n = (int)(next_u64() % N), m = (int)(next_u64() % s.M);
      const uint8_t* row = hw.data() + (size_t)(nseg == 2 ? m >> 1 : m) * (s.K / 32) * 18;
      double acc = 0, mag = 0;
      for (int k = 0; k < s.K; k++) {
        const uint8_t* blk = row + (k / 32) * 18;
        uint16_t dbits;
        memcpy(&dbits, blk, 2);
        const int j = k % 32;
        const int q = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
        const size_t xi = (size_t)n * s.K + cn_span_pos(k);
        const double wx = (double)host_h2f(dbits) * (q - 8) * ((double)host_h2f(ph[xi]) + (double)host_h2f(pl[xi]));
        acc += wx;
        mag += fabs(wx);
      }
      worst = std::max(worst, fabs((double)hy[(size_t)n * s.M + m] - acc) / (mag + 1e-30));
    }
    const bool ok = worst < 1e-6;
    bad += !ok;
    // timing
    for (int l = 0; l < 2; l++) CK(gemm_launch(args(l, s.epi), cus, st));
    CK(hipEventRecord(e0, st));
    for (int l = 0; l < L; l++) CK(gemm_launch(args(l, s.epi), cus, st));
    CK(hipEventRecord(e1, st));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    const double us = ms * 1000.0 / L;
    total_us += us;
    const GemmShape gs = pick_gemm(s.M, N, s.K, cus, true, false);
    const double tf = 2.0 * s.M * (double)N * s.K / us * 1e-6;
    printf("%-8s %5dx%-5d tiles of %d columns, %d-stage ring, K split %d: %8.2f us per call, useful %5.0f TFLOP/s "
           "(%.3f of 2.5 PFLOP/s, %.3f issued); check max |err|/sum|w x| %.2e %s\n",
           s.name, s.M, s.K, 32 * gs.tn, gs.stages, gs.splits, us, tf, tf / 2500.0, 3.0 * tf / 2500.0, worst,
           ok ? "ok" : "FAILED");
    fflush(stdout);
    for (uint8_t* p : w) CK(hipFree(p));
  }
  printf("per layer: %.2f us of span GEMMs\n", total_us);
  printf(bad ? "FAILED\n" : "done\n");
  return bad ? 1 : 0;
}
