// Layer snapshots between host memory and HBM (src/cacheslide_vllm/runtime.py:192-256).
//
// The reference decodes a snapshot page with safetensors into CPU tensors,
// scans them for non-finite values on the CPU and then copies them to the
// device with `.to(device, dtype)`; writing a snapshot copies the device rows
// to pageable host memory first.  Here the page's data region moves in one
// DMA between pinned host staging and HBM (`cs_copy_async`, on a stream of
// the caller's choosing, so it overlaps the compute stream), and the finite
// check plus the dtype conversion run on the device in one pass
// (`cs_snapshot_convert`).
#include "common.h"

namespace cs {

// One pass over a contiguous source: flag non-finite values and write the
// destination dtype.  Conversions round as torch's copy kernel does
// (load_as_double/store_from_double: double -> float -> 16-bit, each step
// round-to-nearest-even), so the result equals `src.to(dtype)`.
__global__ void snapshot_convert_kernel(const void* __restrict__ src, int src_dt, void* __restrict__ dst,
                                        int dst_dt, int64_t n, int32_t bit, int32_t* flags) {
  bool bad = false;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const double v = load_as_double(src, src_dt, i);
    bad |= !__builtin_isfinite(v);
    store_from_double(dst, dst_dt, i, v);
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flags, bit);
}

static bool contiguous_view(const cs_view* v, int64_t* numel) {
  int64_t expect = 1;
  bool ok = true;
  for (int i = v->ndim - 1; i >= 0; --i) {
    if (v->shape[i] != 1 && v->stride[i] != expect) ok = false;
    expect *= v->shape[i];
  }
  *numel = expect;
  return ok;
}

}  // namespace cs

using namespace cs;

extern "C" int cs_copy_async(void* dst, const void* src, int64_t bytes, int32_t kind, void* stream) {
  CS_REQUIRE(bytes >= 0, "negative byte count");
  if (bytes == 0) return CS_OK;
  CS_REQUIRE(dst && src, "null arguments");
  hipMemcpyKind k;
  switch (kind) {
    case CS_COPY_H2D: k = hipMemcpyHostToDevice; break;
    case CS_COPY_D2H: k = hipMemcpyDeviceToHost; break;
    case CS_COPY_D2D: k = hipMemcpyDeviceToDevice; break;
    default: CS_REQUIRE(false, "unknown copy kind %d", kind);
  }
  const hipError_t err = hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), k, as_stream(stream));
  if (err != hipSuccess) {
    set_error("cs_copy_async: %s", hipGetErrorString(err));
    return CS_ELAUNCH;
  }
  return CS_OK;
}

extern "C" int cs_snapshot_convert(const cs_view* src, const cs_view* dst, int32_t bit, int32_t* flags,
                                   void* stream) {
  CS_REQUIRE(src && flags, "null arguments");
  CS_REQUIRE(is_float_dtype(src->dtype), "snapshot tensors must be floating point");
  int64_t n = 0;
  CS_REQUIRE(contiguous_view(src, &n), "snapshot source must be contiguous");
  const bool same = !present(dst) || (dst->data == src->data && dst->dtype == src->dtype);
  if (!same) {
    int64_t m = 0;
    CS_REQUIRE(is_float_dtype(dst->dtype), "snapshot destination must be floating point");
    CS_REQUIRE(contiguous_view(dst, &m) && m == n, "snapshot destination must be contiguous, same size");
    const bool overlap = static_cast<const char*>(dst->data) < static_cast<const char*>(src->data) +
                                                                     n * dtype_size(src->dtype) &&
                         static_cast<const char*>(src->data) < static_cast<const char*>(dst->data) +
                                                                    n * dtype_size(dst->dtype);
    CS_REQUIRE(!overlap || n == 0, "snapshot source and destination overlap");
  }
  if (n == 0 || !src->data) return CS_OK;
  if (same) return cs_check_finite(src, bit, flags, stream);
  const int grid = static_cast<int>(std::min<int64_t>(ceil_div(n, 256 * 4), 8192));
  hipLaunchKernelGGL(snapshot_convert_kernel, dim3(grid), dim3(256), 0, as_stream(stream), src->data,
                     src->dtype, dst->data, dst->dtype, n, bit, flags);
  CS_LAUNCH_CHECK("snapshot_convert");
  return CS_OK;
}
