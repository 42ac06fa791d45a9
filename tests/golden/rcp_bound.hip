// Exhaustive bound of the hardware reciprocal v_rcp_f32 (__builtin_amdgcn_rcpf) over every
// float d in [lo, hi] (bit patterns; default [1, 2^24], which holds every denominator of the
// selection chain: (float)(1 + N) and (float)N + VL with N < 2^24).  Prints the largest
// |rcp(d) * d - 1| (the product is exact in double) and how many d exceed 2^-23.  Built by
// __graft_entry__.build(); run by tests/test_gpu_rcp_bound.py.  Test code: the selection
// chain relies on the bound it prints.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

__global__ void rcp_bound_kernel(uint32_t lo, uint32_t n, unsigned long long* max_bits,
                                 unsigned long long* over) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float d = __uint_as_float(lo + (uint32_t)i);
  const float r = __builtin_amdgcn_rcpf(d);
  const double e = fabs((double)r * (double)d - 1.0);
  unsigned long long eb;
  memcpy(&eb, &e, sizeof eb);  // non-negative doubles order as their bits
  atomicMax(max_bits, eb);
  if (e > 0x1p-23) atomicAdd(over, 1ull);
}

static int fail(const char* what, hipError_t e) {
  fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return 2;
}

int main(int argc, char** argv) {
  uint32_t lo = 0x3F800000u, hi = 0x4B800000u;  // 1.0 and 2^24
  if (argc == 3) {
    lo = (uint32_t)strtoul(argv[1], nullptr, 0);
    hi = (uint32_t)strtoul(argv[2], nullptr, 0);
  }
  if (hi < lo || hi - lo >= 0x40000000u) {
    fprintf(stderr, "bad range\n");
    return 2;
  }
  const uint32_t n = hi - lo + 1;
  unsigned long long* dev = nullptr;
  hipError_t e = hipMalloc(&dev, 2 * sizeof(unsigned long long));
  if (e != hipSuccess) return fail("hipMalloc", e);
  if ((e = hipMemset(dev, 0, 2 * sizeof(unsigned long long))) != hipSuccess)
    return fail("hipMemset", e);
  const uint32_t bs = 256, nb = (n + bs - 1) / bs;
  hipLaunchKernelGGL(rcp_bound_kernel, dim3(nb), dim3(bs), 0, 0, lo, n, dev, dev + 1);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return fail("kernel", e);
  unsigned long long host[2] = {0, 0};
  if ((e = hipMemcpy(host, dev, sizeof host, hipMemcpyDeviceToHost)) != hipSuccess)
    return fail("hipMemcpy", e);
  hipFree(dev);
  double m;
  memcpy(&m, &host[0], sizeof m);
  printf("floats %u max_rel_err %.9e log2 %.4f over_2^-23 %llu\n", n, m,
         m > 0 ? std::log2(m) : -1000.0, host[1]);
  return 0;
}
