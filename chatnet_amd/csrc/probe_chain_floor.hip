// probe_chain_floor.hip — the floor of a chain of dependent kernels inside one
// HIP graph on this device (a stand-alone measurement program, not part of
// the library).  A decode step is such a chain: every GEMV reads the vector
// the previous kernel wrote, so the step time is bounded below by what one
// dependent launch costs before it has moved any useful bytes.
//
//  empty   : kernels that do nothing (1 workgroup; one and two per CU)
//  stream  : each kernel streams S bytes (2 workgroups per CU), cold (a
//            distinct buffer per kernel, >= 1 GiB in rotation, so the 256 MB
//            memory-side cache cannot serve it) and warm (one buffer re-read)
//  shared x: as cold stream, but every workgroup first reads the whole of an
//            x vector of X bytes written by the previous kernel, the way a
//            GEMV stages its input; all workgroups walk x from element 0, or
//            each from its own rotated start
// Times are HIP events around three replays of the captured chain.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CK(x)                                                              \
  do {                                                                     \
    hipError_t e_ = (x);                                                   \
    if (e_ != hipSuccess) {                                                \
      printf("%s: %s\n", #x, hipGetErrorString(e_));                       \
      exit(1);                                                             \
    }                                                                      \
  } while (0)

__global__ void empty_kernel(int* p) {
  if (threadIdx.x == 0 && blockIdx.x == 0 && p[1] == 12345) p[0] = 1;
}

// Streams n4 float4 of buf (4 loads per lane in flight), after reading x
// (xn float4, the previous kernel's output) from start r0 = blockIdx.x * rot,
// and writes its own x for the next kernel.
__global__ __launch_bounds__(256) void stream_kernel(const float4* __restrict__ buf, size_t n4, const float4* x,
                                                      int xn, int rot, float4* xout, float* sink) {
  float xs = 0.f;
  const int r0 = xn > 0 ? (int)(((long long)blockIdx.x * rot) % xn) : 0;
  for (int i = threadIdx.x; i < xn; i += 256) {
    int j = i + r0;
    if (j >= xn) j -= xn;
    const float4 v = x[j];
    xs += v.x + v.y + v.z + v.w;
  }
  float acc = 0.f;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride * 4) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const size_t j = i + u * stride;
      v[u] = j < n4 ? buf[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) acc += v[u].x + v[u].y + v[u].z + v[u].w;
  }
  acc += xs * 1e-30f;
  if (acc == 123.456f) sink[blockIdx.x] = acc;
  const int gi = blockIdx.x * 256 + threadIdx.x;
  if (gi < 4096) xout[gi] = make_float4(acc, 0.f, 0.f, 0.f);
}

int main() {
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  printf("device: %d CUs\n", cus);
  hipStream_t st;
  CK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  int* flag;
  float* sink;
  float4* xb;  // two x vectors of up to 4096 float4 (64 KB), ping-pong
  CK(hipMalloc(&flag, 64));
  CK(hipMalloc(&sink, 1 << 20));
  CK(hipMalloc(&xb, 2 * 4096 * sizeof(float4)));
  CK(hipMemset(flag, 0, 64));
  CK(hipMemset(xb, 0, 2 * 4096 * sizeof(float4)));
  const size_t pool_bytes = (size_t)1536 << 20;
  char* pool;
  CK(hipMalloc(&pool, pool_bytes));
  CK(hipMemset(pool, 0, pool_bytes));
  CK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));

  auto time_graph = [&](auto issue, int nk, const char* what) {
    hipGraph_t g;
    hipGraphExec_t ge;
    CK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    issue();
    CK(hipStreamEndCapture(st, &g));
    CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CK(hipGraphLaunch(ge, st));
    CK(hipStreamSynchronize(st));
    const int reps = 3;
    CK(hipEventRecord(e0, st));
    for (int r = 0; r < reps; r++) CK(hipGraphLaunch(ge, st));
    CK(hipEventRecord(e1, st));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    printf("%-58s %8.3f us per kernel (%d kernels)\n", what, ms * 1000.f / (reps * nk), nk);
    fflush(stdout);
    CK(hipGraphExecDestroy(ge));
    CK(hipGraphDestroy(g));
  };

  const int NK = 400;
  for (int wg : {1, cus, 2 * cus}) {
    char what[96];
    snprintf(what, sizeof what, "empty, %d workgroups", wg);
    time_graph([&]() {
      for (int i = 0; i < NK; i++) hipLaunchKernelGGL(empty_kernel, dim3(wg), dim3(256), 0, st, flag);
    }, NK, what);
  }

  // stream S bytes per kernel; shared x of xn float4 read first (rot: float4
  // by which each workgroup's start moves)
  struct Case {
    size_t kb;
    int xn, rot;
    bool warm;
  };
  const Case cases[] = {
      {3500, 0, 0, false},   {3500, 0, 0, true},    {9400, 0, 0, false},    {25400, 0, 0, false},
      {9400, 1024, 0, false}, {9400, 1024, 64, false}, {25400, 1024, 0, false}, {25400, 1024, 64, false},
      {25400, 2752, 0, false}, {25400, 2752, 64, false}, {25400, 4096, 0, false}, {25400, 4096, 64, false},
  };
  for (const Case& c : cases) {
    const size_t bytes = c.kb * 1000, stride = (bytes + 65535) & ~(size_t)65535;
    int copies = (int)((((size_t)1 << 30) + stride - 1) / stride);
    if ((size_t)copies * stride > pool_bytes) copies = (int)(pool_bytes / stride);
    const int nk = c.warm ? 200 : copies;
    char what[96];
    snprintf(what, sizeof what, "stream %5zu KB %s, x %5d B%s", c.kb, c.warm ? "warm" : "cold", 16 * c.xn,
             c.xn ? (c.rot ? " (rotated start)" : " (same start)") : "");
    time_graph([&]() {
      for (int i = 0; i < nk; i++)
        hipLaunchKernelGGL(stream_kernel, dim3(2 * cus), dim3(256), 0, st,
                           (const float4*)(pool + (c.warm ? 0 : (size_t)i * stride)), bytes / 16,
                           xb + 4096 * (i & 1), c.xn, c.rot, xb + 4096 * ((i + 1) & 1), sink);
    }, nk, what);
  }
  CK(hipFree(pool));
  CK(hipFree(xb));
  CK(hipFree(sink));
  CK(hipFree(flag));
  printf("done\n");
  return 0;
}
