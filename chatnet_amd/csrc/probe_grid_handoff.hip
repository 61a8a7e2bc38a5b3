// probe_grid_handoff.hip — the cost of a grid-wide handoff inside one
// persistent kernel on this device (a stand-alone measurement program, not part
// of the library).  A decode step could run as one kernel whose workgroups pass
// each projection's output to the next through memory instead of through a
// kernel boundary; this measures what one such handoff costs, to set beside
// the 1.56 us of a dependent kernel launch in a graph (probe_chain_floor).
//
// Protocol, without fences: each workgroup writes its slice of a payload with
// device-scope stores (sc1: written through past the XCD's L2), waits for its
// own stores, then stores its round number into its flag; every workgroup then
// polls all the flags with device-scope loads until each shows the round, and
// reads the whole payload with device-scope loads (so no L2 line of another XCD
// can serve it stale), checking every element.  One round = one handoff.
//
// Every poll is bounded by 0.5 s of the 100 MHz real-time counter: a workgroup
// that times out records it and leaves its loop, so the kernel always ends
// (all workgroups of each case are resident: at most two 256-thread
// workgroups per CU).
//
// Cases: workgroups G (64..512), flag stride (packed or one 128-byte line per
// flag), payload floats read by every workgroup per round (0, 2048 = a
// TinyLlama x, 4096 = a 7B x), polling waves per workgroup.
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

__device__ __forceinline__ unsigned ld_dev(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stf_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// flags: gridDim.x entries at stride fs dwords; payload: two buffers of xn
// floats (round r writes buffer r & 1: a workgroup can be at most one round
// ahead of the slowest reader, so it never overwrites what is still read).
// err[0]: 0x80000000 | round of a timed-out poll; err[1]: payload mismatches.
__global__ __launch_bounds__(256) void handoff_kernel(unsigned* flags, int fs, float* payload, int xn, int rounds,
                                                      unsigned* err, int pollers) {
  const int G = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
  const int slice = xn / G;
  __shared__ int s_fail;
  if (tid == 0) s_fail = 0;
  __syncthreads();
  const unsigned long long t_limit = 50000000ull;  // 0.5 s of the 100 MHz counter
  for (int r = 1; r <= rounds; r++) {
    float* pb = payload + (size_t)(r & 1) * xn;
    for (int i = tid; i < slice; i += 256) stf_dev(pb + wg * slice + i, (float)(r * 7 + wg * slice + i));
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
    __syncthreads();
    if (tid == 0) st_dev(flags + (size_t)wg * fs, (unsigned)r);
    if (tid < 64 * pollers) {  // whole waves: every lane of a polling wave runs the loop
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      bool done = false;
      while (!done) {
        bool mine = true;
        for (int j = tid; j < G; j += 64 * pollers) mine &= ld_dev(flags + (size_t)j * fs) >= (unsigned)r;
        done = __all(mine);
        if (!done && __builtin_amdgcn_s_memrealtime() - t0 > t_limit) {
          if ((tid & 63) == 0) {
            st_dev(err, 0x80000000u | r);
            s_fail = 1;
          }
          break;
        }
      }
    }
    __syncthreads();
    if (s_fail) return;  // uniform: read after the barrier, never reset
    if (xn > 0) {
      float s = 0.f, want = 0.f;
      for (int i = tid; i < xn; i += 256) {
        s += ldf_dev(pb + i);
        want += (float)(r * 7 + i);
      }
      if (s != want) st_dev(err + 1, 1u);
    }
  }
}

int main() {
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  printf("device: %d CUs\n", prop.multiProcessorCount);
  unsigned* flags;
  float* payload;
  unsigned* err;
  CK(hipMalloc(&flags, 1024 * 64 * 4));
  CK(hipMalloc(&payload, 2 * 16384 * 4));
  CK(hipMalloc(&err, 64));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  struct Case {
    int G, fs, xn, pollers;
  };
  const Case cases[] = {{64, 1, 0, 1},    {128, 1, 0, 1},   {256, 1, 0, 1},  {256, 32, 0, 1},
                        {256, 1, 0, 4},   {512, 1, 0, 1},   {512, 32, 0, 1}, {256, 1, 2048, 1},
                        {256, 1, 4096, 1}, {512, 1, 4096, 1}};
  for (const Case& c : cases) {
    if (c.G > 2 * prop.multiProcessorCount) continue;  // every workgroup must be resident
    const int rounds = 2000;
    CK(hipMemset(flags, 0, 1024 * 64 * 4));
    CK(hipMemset(err, 0, 64));
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(handoff_kernel, dim3(c.G), dim3(256), 0, 0, flags, c.fs, payload, c.xn, rounds, err,
                       c.pollers);
    CK(hipGetLastError());
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    unsigned h[2];
    CK(hipMemcpy(h, err, 8, hipMemcpyDeviceToHost));
    printf("workgroups %4d, flag stride %2d dwords, payload %5d floats, polling waves %d: %7.3f us per handoff%s%s\n",
           c.G, c.fs, c.xn, c.pollers, ms * 1000.f / rounds, h[0] ? " (POLL TIMED OUT)" : "",
           h[1] ? " (STALE PAYLOAD)" : "");
    fflush(stdout);
  }
  printf("done\n");
  return 0;
}
