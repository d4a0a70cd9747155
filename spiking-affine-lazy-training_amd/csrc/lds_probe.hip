// libsalt_probe.so: LDS bandwidth probe for the roofline of bench.py (not part of the
// forward path).  Every CU runs work-groups that stream conflict-free reads (or writes)
// through a 32 KB LDS buffer: lane l of a wave touches element base + l, so a wave's
// access covers consecutive words and every bank once per half-wave.  The host times
// the launch with HIP events and reports bytes moved per second.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "salt_probe.h"

namespace {

constexpr int kThreads = 256;
constexpr int kBufBytes = 32 * 1024;
constexpr int kUnroll = 16;

template <typename T>
__device__ __forceinline__ T fold(T a, T b) { return a ^ b; }
template <>
__device__ __forceinline__ uint4 fold(uint4 a, uint4 b) {
  return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w);
}
template <typename T>
__device__ __forceinline__ T word(uint32_t i) { return (T)i; }
template <>
__device__ __forceinline__ uint4 word(uint32_t i) { return make_uint4(i, i + 1, i + 2, i + 3); }
template <typename T>
__device__ __forceinline__ uint32_t low(T v) { return (uint32_t)v; }
template <>
__device__ __forceinline__ uint32_t low(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// WRITE = false: each thread reads kUnroll elements per iteration, folded into a register
// that is stored once at the end (only when it has a value the host never passes, so the
// reads stay live without a store per thread).  WRITE = true: kUnroll stores per iteration.
template <typename T, bool WRITE>
__global__ void __launch_bounds__(kThreads) lds_probe_kernel(int iters, uint32_t key,
                                                             uint32_t* sink) {
  constexpr int kElems = kBufBytes / (int)sizeof(T);  // a power of two
  __shared__ T buf[kElems];
  const int t = threadIdx.x;
  for (int i = t; i < kElems; i += kThreads) buf[i] = word<T>((uint32_t)i);
  __syncthreads();
  T acc = word<T>((uint32_t)t);
  int base = t;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int idx = (base + u * (kElems / kUnroll)) & (kElems - 1);  // 16 distinct words
      if (WRITE) buf[idx] = acc;
      else acc = fold(acc, buf[idx]);
    }
    base += 64;  // next iteration: other words, same conflict-free pattern
    if (WRITE) acc = fold(acc, word<T>((uint32_t)it));
  }
  __syncthreads();
  if (WRITE) acc = fold(acc, buf[(t * 7) & (kElems - 1)]);
  if (low(acc) == key) sink[blockIdx.x * kThreads + t] = 1;
}

template <typename T, bool WRITE>
int32_t run(int32_t blocks, int32_t iters, double* seconds, double* bytes) {
  uint32_t* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0.0f;
  bool ok = hipMalloc(&sink, (size_t)blocks * kThreads * 4) == hipSuccess &&
            hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
  for (int rep = 0; ok && rep < 2; ++rep) {  // a warm-up launch, then the timed one
    ok = hipEventRecord(e0, nullptr) == hipSuccess;
    hipLaunchKernelGGL((lds_probe_kernel<T, WRITE>), dim3(blocks), dim3(kThreads), 0, nullptr,
                       iters, 0xFFFFFFFFu, sink);
    ok = ok && hipGetLastError() == hipSuccess && hipEventRecord(e1, nullptr) == hipSuccess &&
         hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
  }
  if (e0) ok = hipEventDestroy(e0) == hipSuccess && ok;
  if (e1) ok = hipEventDestroy(e1) == hipSuccess && ok;
  if (sink) ok = hipFree(sink) == hipSuccess && ok;
  if (!ok) return -2;
  *seconds = ms * 1e-3;
  *bytes = (double)blocks * kThreads * (double)iters * kUnroll * (double)sizeof(T);
  return 0;
}

}  // namespace

extern "C" int32_t salt_probe_lds(int32_t kind, int32_t blocks, int32_t iters, double* seconds,
                                  double* bytes) {
  if (blocks < 1 || iters < 1 || !seconds || !bytes) return -1;
  switch (kind) {
    case SALT_PROBE_READ_B32: return run<uint32_t, false>(blocks, iters, seconds, bytes);
    case SALT_PROBE_READ_B64: return run<uint64_t, false>(blocks, iters, seconds, bytes);
    case SALT_PROBE_READ_B128: return run<uint4, false>(blocks, iters, seconds, bytes);
    case SALT_PROBE_WRITE_B32: return run<uint32_t, true>(blocks, iters, seconds, bytes);
    default: return -1;
  }
}
