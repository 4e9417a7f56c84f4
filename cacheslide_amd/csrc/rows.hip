// Row bookkeeping of the selective prefill (src/cacheslide_vllm/runtime.py:408-456).
//
// Between two layers the reference carries the hidden and residual rows of the
// tokens that stay active, restores newly active tokens from the layer's input
// snapshot (stored for the fixed tokens only), and at the end scatters the last
// layer's rows into a zero-filled [n, H] output.  It builds two length-n lookup
// tables and indexes with boolean masks, which costs host syncs.  Here each
// output row is one wavefront: it finds its source by binary search in the
// ascending token lists (previous layer's active tokens, fixed tokens) and
// copies the row in the widest chunk that every pointer and stride allows.
// Rows are moved bit for bit (any dtype).  A token found in neither list is
// "lost": its rows are written as zeros and CS_FLAG_ROW_LOST is raised (the
// reference raises ReuseFailure there).

#include "common.h"

namespace cs {
namespace {

template <int W> struct word_t;
template <> struct word_t<16> { using type = uint4; };
template <> struct word_t<8> { using type = uint2; };
template <> struct word_t<4> { using type = uint32_t; };
template <> struct word_t<2> { using type = uint16_t; };
template <> struct word_t<1> { using type = uint8_t; };

struct rows2 {  // [rows, H] with contiguous H, in bytes; base == nullptr: absent
  char* base;
  int64_t s_row;
  int64_t n_rows;
};

// Position of x in the ascending list a[0..n), or -1.
__device__ inline int64_t find_sorted(const int64_t* a, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    const int64_t v = a[mid];
    if (v < x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return (lo < n && a[lo] == x) ? lo : -1;
}

// Ascending-and-distinct check of a[0..n) and b[0..m) (and, with a_bound > 0,
// 0 <= a[j] < a_bound), spread over every thread of the grid.
__device__ inline void check_lists(const int64_t* a, int64_t n, const int64_t* b, int64_t m, int64_t a_bound,
                                   int32_t* flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t j = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; j < n || j < m; j += stride) {
    if ((j + 1 < n && a[j] >= a[j + 1]) || (j + 1 < m && b[j] >= b[j + 1]))
      atomicOr(flags, CS_FLAG_ROWS_UNSORTED);
    if (a_bound > 0 && j < n && (a[j] < 0 || a[j] >= a_bound)) atomicOr(flags, CS_FLAG_ROW_INDEX);
  }
}

// Copies one row (src == nullptr: zeros), and optionally a second one, in
// batches of 8 words per lane whose loads are all issued before any store.
constexpr int kBatch = 8;

// Position of x in the ascending a[0..n), or -1, for x uniform across the
// wavefront: the 64 lanes probe 64 evenly spaced entries per step (the probes
// not above x form a prefix), so a list of 64^k entries takes k dependent
// loads instead of k * 6.
__device__ inline int64_t find_sorted_wave(const int64_t* a, int64_t n, int64_t x, int lane) {
  int64_t lo = 0, hi = n;  // x, if present, lies in [lo, hi)
  while (hi - lo > 64) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t p = lo + lane * step;
    const unsigned long long le = __ballot(p < hi && a[p] <= x);
    const int c = __popcll(le);
    if (c == 0) return -1;  // x < a[lo]
    lo += (c - 1) * step;
    hi = lo + step < hi ? lo + step : hi;
  }
  const unsigned long long eq = __ballot(lo + lane < hi && a[lo + lane] == x);
  return eq ? lo + __ffsll(static_cast<long long>(eq)) - 1 : -1;
}

template <int W>
__device__ inline void copy_rows(char* dst0, const char* src0, char* dst1, const char* src1, int64_t words,
                                 int lane) {
  using T = typename word_t<W>::type;
  T* d0 = reinterpret_cast<T*>(dst0);
  T* d1 = reinterpret_cast<T*>(dst1);
  const T* s0 = reinterpret_cast<const T*>(src0);
  const T* s1 = reinterpret_cast<const T*>(src1);
  for (int64_t base = lane; base < words; base += 64 * kBatch) {
    T v0[kBatch], v1[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t c = base + 64 * u;
      v0[u] = (s0 && c < words) ? s0[c] : T{};
      v1[u] = (s1 && c < words) ? s1[c] : T{};
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t c = base + 64 * u;
      if (c < words) {
        d0[c] = v0[u];
        if (d1) d1[c] = v1[u];
      }
    }
  }
}

constexpr int kWaves = 4;  // wavefronts (rows) per workgroup

// Output row i holds token active[i]: continuing rows come from the previous
// layer's rows, restored rows from the snapshot of the fixed tokens.
template <int W>
__global__ void __launch_bounds__(64 * kWaves)
rows_remap_kernel(rows2 hid_in, rows2 res_in, rows2 snap_h, rows2 snap_r, rows2 hid_out, rows2 res_out,
                  const int64_t* previous, int64_t n_prev, const int64_t* active, int64_t n_act,
                  const int64_t* fixed, int64_t n_fixed, int64_t words, int64_t* restored,
                  int32_t* flags) {
  check_lists(previous, n_prev, fixed, n_fixed, 0, flags);
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (i >= n_act) return;
  const int64_t t = active[i];
  const char* sh = nullptr;
  const char* sr = nullptr;
  const int64_t r = find_sorted_wave(previous, n_prev, t, lane);
  if (r >= 0) {
    sh = hid_in.base + r * hid_in.s_row;
    sr = res_in.base ? res_in.base + r * res_in.s_row : nullptr;
  } else {
    const int64_t o = find_sorted_wave(fixed, n_fixed, t, lane);
    if (o >= 0 && o < snap_h.n_rows && snap_h.base) {
      sh = snap_h.base + o * snap_h.s_row;
      sr = snap_r.base ? snap_r.base + o * snap_r.s_row : nullptr;
      if (lane == 0) atomicAdd(reinterpret_cast<unsigned long long*>(restored), 1ull);
    } else if (lane == 0) {
      atomicOr(flags, CS_FLAG_ROW_LOST);
    }
  }
  copy_rows<W>(hid_out.base + i * hid_out.s_row, sh, res_out.base ? res_out.base + i * res_out.s_row : nullptr,
               sr, words, lane);
}

// Count of the tokens of active[] that are not in previous[] (rows the remap
// restores from the snapshot).
__global__ void rows_missing_kernel(const int64_t* previous, int64_t n_prev, const int64_t* active,
                                    int64_t n_act, int64_t* count) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  const bool miss = i < n_act && find_sorted(previous, n_prev, active[i]) < 0;
  const unsigned long long wave = __ballot(miss);
  if ((threadIdx.x & 63) == 0 && wave)
    atomicAdd(reinterpret_cast<unsigned long long*>(count), static_cast<unsigned long long>(__popcll(wave)));
}

// out[j] = rows[k] of the k with tokens[k] == j, zeros for every other j < n.
template <int W>
__global__ void __launch_bounds__(64 * kWaves)
rows_scatter_kernel(rows2 src, const int64_t* tokens, int64_t m, rows2 out, int64_t n, int64_t words,
                    int32_t* flags) {
  check_lists(tokens, m, nullptr, 0, n, flags);
  const int lane = threadIdx.x & 63;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (j >= n) return;
  const int64_t k = find_sorted_wave(tokens, m, j, lane);
  copy_rows<W>(out.base + j * out.s_row, (k >= 0 && k < src.n_rows) ? src.base + k * src.s_row : nullptr,
               nullptr, nullptr, words, lane);
}

// out[i] = src[idx[i]]; an index outside src raises CS_FLAG_ROW_INDEX and
// writes zeros.
template <int W>
__global__ void __launch_bounds__(64 * kWaves)
rows_gather_kernel(rows2 src, const int64_t* idx, int64_t m, rows2 out, int64_t words, int32_t* flags) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (i >= m) return;
  const int64_t r = idx[i];
  const bool ok = r >= 0 && r < src.n_rows;
  if (!ok && lane == 0) atomicOr(flags, CS_FLAG_ROW_INDEX);
  copy_rows<W>(out.base + i * out.s_row, ok ? src.base + r * src.s_row : nullptr, nullptr, nullptr, words, lane);
}

// ---------------------------------------------------------------- host side
int row_view(const cs_view* v, int64_t width, int es, const char* name, rows2* out, bool optional) {
  if (!present(v)) {
    CS_REQUIRE(optional, "%s is required", name);
    *out = rows2{nullptr, 0, 0};
    return CS_OK;
  }
  CS_REQUIRE(v->ndim == 2 && v->shape[1] == width, "%s must be [rows, %lld]", name,
             static_cast<long long>(width));
  CS_REQUIRE(dtype_size(v->dtype) == es, "%s has a different element size", name);
  CS_REQUIRE(v->stride[1] == 1 || v->shape[1] <= 1, "%s rows must be contiguous", name);
  CS_REQUIRE(v->stride[0] >= 0, "%s has a negative row stride", name);
  *out = rows2{static_cast<char*>(v->data), v->stride[0] * es, v->shape[0]};
  return CS_OK;
}

// Widest chunk dividing the row length, every base pointer and every row stride.
int pick_word(int64_t row_bytes, std::initializer_list<const rows2*> views) {
  for (int w = 16; w > 1; w >>= 1) {
    bool ok = row_bytes % w == 0;
    for (const rows2* v : views)
      if (v->base && (reinterpret_cast<uintptr_t>(v->base) % w || v->s_row % w)) ok = false;
    if (ok) return w;
  }
  return 1;
}

#define CS_ROWS_DISPATCH(W, KERNEL, GRID, STREAM, ...)                                         \
  switch (W) {                                                                                 \
    case 16: hipLaunchKernelGGL((KERNEL<16>), GRID, dim3(64 * kWaves), 0, STREAM, __VA_ARGS__); break; \
    case 8: hipLaunchKernelGGL((KERNEL<8>), GRID, dim3(64 * kWaves), 0, STREAM, __VA_ARGS__); break;   \
    case 4: hipLaunchKernelGGL((KERNEL<4>), GRID, dim3(64 * kWaves), 0, STREAM, __VA_ARGS__); break;   \
    case 2: hipLaunchKernelGGL((KERNEL<2>), GRID, dim3(64 * kWaves), 0, STREAM, __VA_ARGS__); break;   \
    default: hipLaunchKernelGGL((KERNEL<1>), GRID, dim3(64 * kWaves), 0, STREAM, __VA_ARGS__); break;  \
  }

dim3 row_grid(int64_t rows) { return dim3(static_cast<unsigned>(ceil_div(rows, kWaves))); }

}  // namespace
}  // namespace cs

using namespace cs;

extern "C" int cs_rows_remap(const cs_view* hidden_in, const cs_view* residual_in, const cs_view* snap_hidden,
                             const cs_view* snap_residual, cs_view* hidden_out, cs_view* residual_out,
                             const int64_t* previous, int64_t n_prev, const int64_t* active, int64_t n_active,
                             const int64_t* fixed, int64_t n_fixed, int64_t* restored, int32_t* flags,
                             void* stream) {
  CS_REQUIRE(hidden_in && hidden_out && flags && restored, "null arguments");
  CS_REQUIRE(n_prev >= 0 && n_active >= 0 && n_fixed >= 0, "negative list lengths");
  CS_REQUIRE((n_prev == 0 || previous) && (n_active == 0 || active) && (n_fixed == 0 || fixed),
             "null token lists");
  CS_REQUIRE(hidden_in->ndim == 2, "hidden must be [rows, H]");
  const int64_t width = hidden_in->shape[1];
  const int es = dtype_size(hidden_in->dtype);
  CS_REQUIRE(es > 0, "unknown dtype");
  // no active rows: nothing is read or written, and empty outputs have no data
  // pointer, so the views below would read as absent
  if (n_active == 0) return CS_OK;
  rows2 hi, ri, sh, sr, ho, ro;
  int st;
  if ((st = row_view(hidden_in, width, es, "hidden", &hi, false))) return st;
  if ((st = row_view(residual_in, width, es, "residual", &ri, true))) return st;
  if ((st = row_view(snap_hidden, width, es, "snapshot hidden", &sh, true))) return st;
  if ((st = row_view(snap_residual, width, es, "snapshot residual", &sr, true))) return st;
  if ((st = row_view(hidden_out, width, es, "hidden out", &ho, false))) return st;
  if ((st = row_view(residual_out, width, es, "residual out", &ro, true))) return st;
  CS_REQUIRE((ri.base != nullptr) == (ro.base != nullptr), "residual in and out go together");
  CS_REQUIRE(!sr.base || sh.base, "a snapshot residual needs the snapshot hidden rows");
  CS_REQUIRE(hi.n_rows >= n_prev && (!ri.base || ri.n_rows >= n_prev), "fewer rows than previous tokens");
  CS_REQUIRE(ho.n_rows >= n_active && (!ro.base || ro.n_rows >= n_active), "fewer out rows than active tokens");
  CS_REQUIRE(!sr.base || sr.n_rows >= sh.n_rows, "snapshot residual has fewer rows");
  if (ri.base && sh.base) CS_REQUIRE(sr.base != nullptr, "the snapshot needs residual rows too");
  hipStream_t s = as_stream(stream);
  if (width == 0) return CS_OK;  // nothing to move
  const int64_t row_bytes = width * es;
  const int w = pick_word(row_bytes, {&hi, &ri, &sh, &sr, &ho, &ro});
  CS_ROWS_DISPATCH(w, rows_remap_kernel, row_grid(n_active), s, hi, ri, sh, sr, ho, ro, previous, n_prev,
                   active, n_active, fixed, n_fixed, row_bytes / w, restored, flags);
  CS_LAUNCH_CHECK("rows_remap");
  return CS_OK;
}

extern "C" int cs_rows_missing(const int64_t* previous, int64_t n_prev, const int64_t* active,
                               int64_t n_active, int64_t* count, void* stream) {
  CS_REQUIRE(count && n_prev >= 0 && n_active >= 0, "bad arguments");
  CS_REQUIRE((n_prev == 0 || previous) && (n_active == 0 || active), "null token lists");
  if (n_active == 0) return CS_OK;
  hipLaunchKernelGGL(rows_missing_kernel, dim3(static_cast<unsigned>(ceil_div(n_active, 256))), dim3(256), 0,
                     as_stream(stream), previous, n_prev, active, n_active, count);
  CS_LAUNCH_CHECK("rows_missing");
  return CS_OK;
}

extern "C" int cs_rows_scatter(const cs_view* rows, const int64_t* tokens, int64_t m, cs_view* out,
                               int32_t* flags, void* stream) {
  CS_REQUIRE(rows && out && flags && m >= 0 && (m == 0 || tokens), "null arguments");
  CS_REQUIRE(out->ndim == 2 && rows->ndim == 2, "rows and out must be [rows, H]");
  const int64_t width = out->shape[1];
  const int es = dtype_size(out->dtype);
  CS_REQUIRE(es > 0, "unknown dtype");
  rows2 src, dst;
  int st;
  // no tokens: the rows are never read (and an empty tensor has no data pointer)
  if ((st = row_view(rows, width, es, "rows", &src, m == 0))) return st;
  if ((st = row_view(out, width, es, "out", &dst, false))) return st;
  CS_REQUIRE(src.n_rows >= m, "fewer rows than tokens");
  hipStream_t s = as_stream(stream);
  CS_REQUIRE(dst.n_rows > 0 || m == 0, "tokens need output rows");
  if (dst.n_rows == 0) return CS_OK;
  const int64_t row_bytes = width * es;
  const int w = pick_word(row_bytes, {&src, &dst});
  CS_ROWS_DISPATCH(w, rows_scatter_kernel, row_grid(dst.n_rows), s, src, tokens, m, dst, dst.n_rows,
                   row_bytes / w, flags);
  CS_LAUNCH_CHECK("rows_scatter");
  return CS_OK;
}

extern "C" int cs_rows_gather(const cs_view* src, const int64_t* idx, int64_t m, cs_view* out,
                              int32_t* flags, void* stream) {
  CS_REQUIRE(src && out && flags && m >= 0 && (m == 0 || idx), "null arguments");
  CS_REQUIRE(src->ndim == 2 && out->ndim == 2, "src and out must be [rows, H]");
  const int64_t width = src->shape[1];
  const int es = dtype_size(src->dtype);
  CS_REQUIRE(es > 0, "unknown dtype");
  rows2 a, b;
  int st;
  // no indices: nothing is read or written (an empty tensor has no data pointer)
  if ((st = row_view(src, width, es, "src", &a, m == 0))) return st;
  if ((st = row_view(out, width, es, "out", &b, m == 0))) return st;
  CS_REQUIRE(b.n_rows >= m, "fewer out rows than indices");
  if (m == 0 || width == 0) return CS_OK;
  const int64_t row_bytes = width * es;
  const int w = pick_word(row_bytes, {&a, &b});
  CS_ROWS_DISPATCH(w, rows_gather_kernel, row_grid(m), as_stream(stream), a, idx, m, b, row_bytes / w, flags);
  CS_LAUNCH_CHECK("rows_gather");
  return CS_OK;
}
