// Read-rate probes for the measurement: how fast this device reads a buffer
// streamed once, and a set of chunks in a given order (the access pattern of
// a kernel under study, e.g. the decode's block-table reads).  Each thread
// folds what it read into one word of `sink`, so the loads are kept.
//
// Measurement support with no counterpart in the reference, exported for the
// benchmark's own binding and not declared in the library's header:
//   int cs_read_probe(const void* base, int64_t bytes, const int64_t* chunks,
//                     int64_t n_chunks, int32_t per_wg, int32_t chunk_bytes,
//                     uint32_t* sink, int64_t sink_words, void* stream);
// reads a buffer streamed once (chunks == NULL), or chunks of chunk_bytes at
// the byte offsets chunks[0 .. n_chunks), per_wg chunks per 256-thread
// workgroup in order (a chunk outside the buffer or not 16-byte aligned is
// skipped); sink holds one uint32 device word per thread (at most 16384 x 256
// in streaming mode).

#include "common.h"

namespace cs {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) stream_read_kernel(const uint4* src, int64_t n16, uint32_t* sink) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  uint32_t acc = 0;
  int64_t i = tid;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  sink[tid] = acc;
}

// Workgroup g reads chunks[g * per_wg .. + per_wg) (byte offsets into base);
// a chunk outside [0, bytes) or not 16-byte aligned is skipped.
__global__ void __launch_bounds__(kThreads) chunk_read_kernel(const char* base, int64_t bytes, const int64_t* chunks,
                                                              int32_t per_wg, int32_t chunk_bytes, uint32_t* sink) {
  uint32_t acc = 0;
  const int per_chunk = chunk_bytes / 16;
  for (int j = 0; j < per_wg; ++j) {
    const int64_t off = chunks[static_cast<int64_t>(blockIdx.x) * per_wg + j];
    if (off < 0 || off > bytes - chunk_bytes || off % 16 != 0) continue;
    const uint4* c = reinterpret_cast<const uint4*>(base + off);
    for (int t = threadIdx.x; t < per_chunk; t += kThreads) {
      const uint4 a = c[t];
      acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
  }
  sink[static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x] = acc;
}

}  // namespace
}  // namespace cs

using namespace cs;

extern "C" int cs_read_probe(const void* base, int64_t bytes, const int64_t* chunks, int64_t n_chunks,
                             int32_t per_wg, int32_t chunk_bytes, uint32_t* sink, int64_t sink_words,
                             void* stream) {
  CS_REQUIRE(base && sink && bytes >= 16 && (reinterpret_cast<uintptr_t>(base) % 16) == 0 && bytes % 16 == 0,
             "the probe reads a 16-byte aligned buffer of whole 16-byte words");
  hipStream_t s = as_stream(stream);
  if (chunks == nullptr) {
    int64_t grid = sink_words / kThreads;
    if (grid > 16384) grid = 16384;
    CS_REQUIRE(grid >= 1, "the sink holds fewer than %d words", kThreads);
    hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, s,
                       static_cast<const uint4*>(base), bytes / 16, sink);
  } else {
    CS_REQUIRE(per_wg > 0 && n_chunks % per_wg == 0 && chunk_bytes > 0 && chunk_bytes % 16 == 0 &&
                   chunk_bytes <= bytes,
               "chunks must be whole groups of per_wg chunks of whole 16-byte words");
    const int64_t grid = n_chunks / per_wg;
    CS_REQUIRE(grid < (int64_t(1) << 31) && grid * kThreads <= sink_words, "the sink holds %lld words, "
               "the probe writes %lld", static_cast<long long>(sink_words), static_cast<long long>(grid * kThreads));
    hipLaunchKernelGGL(chunk_read_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, s,
                       static_cast<const char*>(base), bytes, chunks, per_wg, chunk_bytes, sink);
  }
  CS_LAUNCH_CHECK("read_probe");
  return CS_OK;
}
