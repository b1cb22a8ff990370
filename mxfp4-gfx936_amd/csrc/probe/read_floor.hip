// Measurement aid for bench.py (not part of the operator library): the
// time a single launch needs just to read N bytes from HBM, the floor that
// a decode GEMV over N bytes of weights cannot beat.  Every workgroup of
// 256 threads issues all of its loads -- kLoads 16-byte loads per thread,
// consecutive threads on consecutive 16-byte chunks -- before it uses any,
// then folds them into one word (so the loads are not dropped) and writes
// that word.  Out-of-range chunks are not read.
#include <hip/hip_runtime.h>
#include <cstdint>

namespace {

constexpr int kThreads = 256;
constexpr int kLoads = 4;

__global__ __launch_bounds__(kThreads) void read_floor(const uint4* __restrict__ p, int64_t chunks,
                                                       uint32_t* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * (kThreads * kLoads) + threadIdx.x;
  uint4 v[kLoads];
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
    const int64_t i = base + (int64_t)u * kThreads;
    v[u] = i < chunks ? p[i] : uint4{0u, 0u, 0u, 0u};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < kLoads; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  // one word per workgroup: the lanes' words folded through LDS
  __shared__ uint32_t red[kThreads];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kThreads / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0];
}

}  // namespace

// Reads `bytes` (a multiple of 16, 16-byte aligned) at p; sink must hold
// mxfp4_probe_read_floor_sink_words(bytes) words.  0 on success.
extern "C" int64_t mxfp4_probe_read_floor_sink_words(int64_t bytes) {
  const int64_t chunks = bytes / 16;
  return (chunks + kThreads * kLoads - 1) / (kThreads * kLoads);
}

extern "C" int mxfp4_probe_read_floor(const void* p, int64_t bytes, uint32_t* sink, void* stream) {
  if (p == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 ||
      (reinterpret_cast<uintptr_t>(p) & 15))
    return 1;
  const int64_t chunks = bytes / 16;
  const int64_t blocks = mxfp4_probe_read_floor_sink_words(bytes);
  if (blocks > 0x7FFFFFFF) return 1;
  read_floor<<<(unsigned)blocks, kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(p), chunks, sink);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
