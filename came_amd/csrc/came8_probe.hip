// HBM access-mix probes for bench.py --probes: kernels that stream the byte mixes of the optimizer's
// passes with no arithmetic to speak of, so that a pass's measured rate can be set against what its
// access mix alone reaches on the device.  Built into a library of its own (libcame8probe.so); nothing
// in libcame8.so uses it.
//
// Per 8-element chunk of a 16-bit gradient (the C4 case):
//   mode 0  read 16 B                                   (pass 1: the gradient)
//   mode 1  read 16 B + 8 B                             (pass 2: gradient and momentum codes)
//   mode 2  read 16 B, read+write 16 B, read+write 8 B  (pass 3: gradient, parameter, codes)
//   mode 3  read 16 B, write 16 B                       (a copy)
// Modes 4-7 are modes 0-3 with the nontemporal hint on every load and store (`global_load ... nt`,
// `global_store ... nt`); each wavefront instruction covers 1 KiB (or 512 B) of whole lines.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;

typedef uint32_t U4 __attribute__((ext_vector_type(4)));
typedef uint32_t U2 __attribute__((ext_vector_type(2)));

template <bool NT, typename T>
__device__ __forceinline__ T ld(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename T>
__device__ __forceinline__ void st(T* p, T v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// kIlp: chunks per thread in flight; MODE & 3: the access mix, MODE & 4: the nontemporal hint
template <int MODE, int kIlp>
__global__ __launch_bounds__(kThreads) void k_probe(const U4* __restrict__ a, U4* __restrict__ b, U2* __restrict__ c,
                                                    int64_t n, uint32_t* __restrict__ sink) {
  constexpr int MIX = MODE & 3;
  constexpr bool NT = (MODE & 4) != 0;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  uint32_t acc = 0;
  for (int64_t i0 = int64_t(blockIdx.x) * kThreads + threadIdx.x; i0 < n; i0 += stride * kIlp) {
    U4 va[kIlp], vb[kIlp];
    U2 vc[kIlp];
#pragma unroll
    for (int u = 0; u < kIlp; ++u) {
      const int64_t i = i0 + u * stride;
      if (i < n) {
        va[u] = ld<NT>(a + i);
        if constexpr (MIX == 1) vc[u] = ld<NT>(c + i);
        if constexpr (MIX == 2) {
          vb[u] = ld<NT>(b + i);
          vc[u] = ld<NT>(c + i);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kIlp; ++u) {
      const int64_t i = i0 + u * stride;
      if (i < n) {
        if constexpr (MIX == 0) acc ^= va[u].x ^ va[u].y ^ va[u].z ^ va[u].w;
        if constexpr (MIX == 1) acc ^= va[u].x ^ va[u].w ^ vc[u].x ^ vc[u].y;
        if constexpr (MIX == 2) {
          st<NT>(b + i, U4{vb[u].x + va[u].x, vb[u].y + va[u].y, vb[u].z + va[u].z, vb[u].w + va[u].w});
          st<NT>(c + i, U2{vc[u].x ^ va[u].y, vc[u].y ^ va[u].z});
        }
        if constexpr (MIX == 3) st<NT>(b + i, va[u]);
      }
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads of the read-only modes
}

}  // namespace

extern "C" {

// Runs mode `mode` (0-7) over n chunks nrep times on `stream` and writes the average duration of one run
// (HIP events on that stream) to *ms.  a: n * 16 bytes; b: n * 16 bytes (modes 2, 3, 6, 7);
// c: n * 8 bytes (modes 1, 2, 5, 6); sink: 4 bytes.  Launch shape: wgs_per_cu workgroups of 256 threads per CU, ilp (4 or
// 8) chunks per thread in flight.  Returns 0, or -1 for a bad argument or a HIP error.
int came8_probe(int mode, const void* a, void* b, void* c, int64_t n, int nrep, int wgs_per_cu, int ilp, void* sink,
                float* ms, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  if (wgs_per_cu < 1 || wgs_per_cu > 64 || (ilp != 4 && ilp != 8)) return -1;
  const dim3 grid(unsigned(cus) * unsigned(wgs_per_cu)), blk(kThreads);
  auto* pa = static_cast<const U4*>(a);
  auto* pb = static_cast<U4*>(b);
  auto* pc = static_cast<U2*>(c);
  auto* ps = static_cast<uint32_t*>(sink);
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, blk, 0, s, pa, pb, pc, n, ps); };
  auto launch = [&]() {
    const bool i8 = ilp == 8;
    switch (mode) {
      case 0: i8 ? go(k_probe<0, 8>) : go(k_probe<0, 4>); break;
      case 1: i8 ? go(k_probe<1, 8>) : go(k_probe<1, 4>); break;
      case 2: i8 ? go(k_probe<2, 8>) : go(k_probe<2, 4>); break;
      case 3: i8 ? go(k_probe<3, 8>) : go(k_probe<3, 4>); break;
      case 4: i8 ? go(k_probe<4, 8>) : go(k_probe<4, 4>); break;
      case 5: i8 ? go(k_probe<5, 8>) : go(k_probe<5, 4>); break;
      case 6: i8 ? go(k_probe<6, 8>) : go(k_probe<6, 4>); break;
      case 7: i8 ? go(k_probe<7, 8>) : go(k_probe<7, 4>); break;
      default: break;
    }
  };
  if (mode < 0 || mode > 7 || nrep < 1) return -1;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -1;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return -1;
  }
  (void)hipEventRecord(e0, s);
  for (int r = 0; r < nrep; ++r) launch();
  (void)hipEventRecord(e1, s);
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  float t = 0.0f;
  if (err == hipSuccess) err = hipEventElapsedTime(&t, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (err != hipSuccess) return -1;
  *ms = t / float(nrep);
  return 0;
}

}  // extern "C"
