// SLIDE slot kernels: paged-KV scatter/gather, token and page relocation,
// token->slot map updates and the free-slot bitmap.
//
// Cache layout is the vLLM packed one used by the reference
// (src/cacheslide_vllm/paged.py:1-8): [blocks, kv_heads, block_size, 2*D] with
// K in [..., :D] and V in [..., D:].  A slot s below blocks*block_size is native
// (block s / bs, offset s % bs); s >= blocks*bs addresses the sidecar rows
// side_k/side_v [S, kv_heads, D] (paged.py:205-240).  All moves are byte copies,
// so results are bit-exact for every dtype.
//
// Every access goes through 1..16-byte "chunks"; the widest width that divides
// every base pointer, stride and row length is chosen on the host, so
// contiguous bf16 rows move as 128-bit global loads/stores.

#include "common.h"

namespace cs {
namespace {

template <int W> struct chunk_t;
template <> struct chunk_t<16> { using type = uint4; };
template <> struct chunk_t<8> { using type = uint2; };
template <> struct chunk_t<4> { using type = uint32_t; };
template <> struct chunk_t<2> { using type = uint16_t; };
template <> struct chunk_t<1> { using type = uint8_t; };

inline bool aligned(const void* p, int64_t w) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(w)) == 0;
}

// Largest chunk width (bytes) usable for rows of `row_bytes` whose base
// pointers and outer byte strides are all listed.
inline int pick_width(int64_t row_bytes, std::initializer_list<const void*> ptrs,
                      std::initializer_list<int64_t> byte_strides) {
  for (int w = 16; w >= 1; w >>= 1) {
    if (row_bytes % w) continue;
    bool ok = true;
    for (const void* p : ptrs)
      if (p && !aligned(p, w)) ok = false;
    for (int64_t s : byte_strides)
      if (s % w) ok = false;
    if (ok) return w;
  }
  return 1;
}

struct kv_rows {  // [rows, H, D] view of key or value, in bytes
  char* base;
  int64_t s_row, s_head;  // bytes
  int64_t n_rows;
  int64_t step;  // bytes between consecutive chunks along D
};

struct paged {  // [blocks, H, bs, 2D] cache + optional sidecar, in bytes
  char* cache;
  int64_t s_block, s_head, s_off;
  int64_t blocks, bs, native;
  char* side_k;
  char* side_v;
  int64_t side_rows, side_s_row, side_s_head;
  int64_t v_off;      // bytes from a record's K half to its V half
  int64_t c_step;     // bytes between chunks along D in the cache
  int64_t side_step;  // ... and in the sidecar
};

// One work item = one chunk of one (row, head, K|V) record.
template <int W, bool SCATTER>
__global__ void slot_move_kernel(paged pg, kv_rows key, kv_rows value, const int64_t* slots,
                                 const int64_t* rows, int64_t n, int64_t heads,
                                 int64_t chunks_per_row) {
  using T = typename chunk_t<W>::type;
  const int64_t total = n * heads * 2 * chunks_per_row;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t c = idx % chunks_per_row;
    int64_t t = idx / chunks_per_row;
    int64_t kv = t % 2;
    t /= 2;
    int64_t h = t % heads;
    int64_t i = t / heads;
    int64_t slot = slots[i];
    int64_t r = rows ? rows[i] : i;
    const kv_rows& src = kv ? value : key;
    if (r < 0 || r >= src.n_rows) continue;
    char* dense = src.base + r * src.s_row + h * src.s_head + c * src.step;
    char* paged_ptr;
    if (slot >= 0 && slot < pg.native) {
      int64_t blk = slot / pg.bs, off = slot % pg.bs;
      paged_ptr = pg.cache + blk * pg.s_block + h * pg.s_head + off * pg.s_off + kv * pg.v_off +
                  c * pg.c_step;
    } else if (slot >= pg.native && slot < pg.native + pg.side_rows && pg.side_k) {
      char* side = kv ? pg.side_v : pg.side_k;
      paged_ptr = side + (slot - pg.native) * pg.side_s_row + h * pg.side_s_head + c * pg.side_step;
    } else {
      continue;  // out-of-range slots are rejected on the host; never touch memory
    }
    if (SCATTER)
      *reinterpret_cast<T*>(paged_ptr) = *reinterpret_cast<const T*>(dense);
    else
      *reinterpret_cast<T*>(dense) = *reinterpret_cast<const T*>(paged_ptr);
  }
}

int grid_for(int64_t total, int threads) {
  int64_t g = ceil_div(total, threads);
  if (g > 65535 * 8) g = 65535 * 8;
  return static_cast<int>(g < 1 ? 1 : g);
}

int slot_move(const cs_view* cache, const cs_view* side_k, const cs_view* side_v,
              const int64_t* slots, const int64_t* rows, int64_t n, const cs_view* key,
              const cs_view* value, bool scatter, void* stream) {
  CS_REQUIRE(cache && cache->data && cache->ndim == 4, "cache must be a 4-d view");
  CS_REQUIRE(key && value && key->ndim == 3 && value->ndim == 3, "key/value must be 3-d views");
  CS_REQUIRE(n == 0 || (slots && key->data && value->data), "null slot or row pointers");
  const int es = dtype_size(cache->dtype);
  CS_REQUIRE(es > 0 && key->dtype == cache->dtype && value->dtype == cache->dtype,
             "key/value dtype must match the cache");
  const int64_t heads = cache->shape[1];
  const int64_t d = cache->shape[3] / 2;
  CS_REQUIRE(cache->shape[3] % 2 == 0 && key->shape[1] == heads && key->shape[2] == d &&
                 value->shape[1] == heads && value->shape[2] == d,
             "key/value must be [rows, %lld, %lld]", (long long)heads, (long long)d);
  bool side = present(side_k) && present(side_v);
  if (side) {
    CS_REQUIRE(side_k->ndim == 3 && side_v->ndim == 3 && side_k->shape[1] == heads &&
                   side_k->shape[2] == d && side_v->shape[0] == side_k->shape[0] &&
                   side_k->stride[2] == side_v->stride[2] &&
                   side_k->stride[0] == side_v->stride[0] && side_k->stride[1] == side_v->stride[1] &&
                   side_k->dtype == cache->dtype && side_v->dtype == cache->dtype,
               "sidecar must be [S, %lld, %lld] with matching strides", (long long)heads,
               (long long)d);
  }
  // Innermost strides may be arbitrary (the reference indexes actual strides);
  // contiguous rows move in wide chunks, strided ones element by element.
  const bool contiguous = cache->stride[3] == 1 && key->stride[2] == 1 && value->stride[2] == 1 &&
                          (!side || side_k->stride[2] == 1);
  if (n == 0) return CS_OK;
  paged pg{};
  pg.cache = static_cast<char*>(cache->data);
  pg.s_block = cache->stride[0] * es;
  pg.s_head = cache->stride[1] * es;
  pg.s_off = cache->stride[2] * es;
  pg.blocks = cache->shape[0];
  pg.bs = cache->shape[2];
  pg.native = pg.blocks * pg.bs;
  pg.v_off = d * cache->stride[3] * es;
  if (side) {
    pg.side_k = static_cast<char*>(side_k->data);
    pg.side_v = static_cast<char*>(side_v->data);
    pg.side_rows = side_k->shape[0];
    pg.side_s_row = side_k->stride[0] * es;
    pg.side_s_head = side_k->stride[1] * es;
  }
  kv_rows kr{static_cast<char*>(key->data), key->stride[0] * es, key->stride[1] * es, key->shape[0], 0};
  kv_rows vr{static_cast<char*>(value->data), value->stride[0] * es, value->stride[1] * es,
             value->shape[0], 0};
  const int64_t row_bytes = d * es;
  int w = es;
  if (contiguous) {
    w = pick_width(row_bytes, {pg.cache, pg.cache + pg.v_off, pg.side_k, pg.side_v, kr.base, vr.base},
                   {pg.s_block, pg.s_head, pg.s_off, pg.side_s_row, pg.side_s_head, kr.s_row,
                    kr.s_head, vr.s_row, vr.s_head});
    pg.c_step = pg.side_step = kr.step = vr.step = w;
  } else {
    pg.c_step = cache->stride[3] * es;
    pg.side_step = side ? side_k->stride[2] * es : 0;
    kr.step = key->stride[2] * es;
    vr.step = value->stride[2] * es;
  }
  int64_t chunks = row_bytes / w;
  int64_t total = n * heads * 2 * chunks;
  const int threads = 256;
  int grid = grid_for(total, threads);
  hipStream_t s = as_stream(stream);
#define CS_MOVE(WW)                                                                         \
  if (scatter)                                                                              \
    hipLaunchKernelGGL((slot_move_kernel<WW, true>), dim3(grid), dim3(threads), 0, s, pg, kr, \
                       vr, slots, rows, n, heads, chunks);                                  \
  else                                                                                      \
    hipLaunchKernelGGL((slot_move_kernel<WW, false>), dim3(grid), dim3(threads), 0, s, pg,  \
                       kr, vr, slots, rows, n, heads, chunks);
  switch (w) {
    case 16: CS_MOVE(16); break;
    case 8: CS_MOVE(8); break;
    case 4: CS_MOVE(4); break;
    case 2: CS_MOVE(2); break;
    default: CS_MOVE(1); break;
  }
#undef CS_MOVE
  CS_LAUNCH_CHECK(scatter ? "slot_scatter" : "slot_gather");
  return CS_OK;
}

// ---------------------------------------------------------------- relocation
struct stacked {  // [L, blocks, H, bs, 2D] in bytes
  char* base;
  int64_t s_layer, s_block, s_head, s_off;
  int64_t layers, blocks, heads, bs;
  int64_t rec_bytes;  // 2*D*es
};

template <int W>
__global__ void slot_copy_kernel(stacked c, const int64_t* src, const int64_t* dst, int64_t n,
                                 int64_t chunks) {
  using T = typename chunk_t<W>::type;
  const int64_t native = c.blocks * c.bs;
  const int64_t total = n * c.layers * c.heads * chunks;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t ch = idx % chunks;
    int64_t t = idx / chunks;
    int64_t h = t % c.heads;
    t /= c.heads;
    int64_t l = t % c.layers;
    int64_t i = t / c.layers;
    int64_t s = src[i], d = dst[i];
    if (s < 0 || s >= native || d < 0 || d >= native) continue;
    const char* sp = c.base + l * c.s_layer + (s / c.bs) * c.s_block + h * c.s_head +
                     (s % c.bs) * c.s_off + ch * W;
    char* dp = c.base + l * c.s_layer + (d / c.bs) * c.s_block + h * c.s_head +
               (d % c.bs) * c.s_off + ch * W;
    *reinterpret_cast<T*>(dp) = *reinterpret_cast<const T*>(sp);
  }
}

// Page copy: one work item = one chunk of one (block, layer, head, offset) row.
template <int W>
__global__ void page_copy_kernel(stacked c, const int64_t* src, const int64_t* dst, int64_t n,
                                 int64_t chunks) {
  using T = typename chunk_t<W>::type;
  const int64_t total = n * c.layers * c.heads * c.bs * chunks;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t ch = idx % chunks;
    int64_t t = idx / chunks;
    int64_t off = t % c.bs;
    t /= c.bs;
    int64_t h = t % c.heads;
    t /= c.heads;
    int64_t l = t % c.layers;
    int64_t i = t / c.layers;
    int64_t s = src[i], d = dst[i];
    if (s < 0 || s >= c.blocks || d < 0 || d >= c.blocks) continue;
    const char* sp = c.base + l * c.s_layer + s * c.s_block + h * c.s_head + off * c.s_off + ch * W;
    char* dp = c.base + l * c.s_layer + d * c.s_block + h * c.s_head + off * c.s_off + ch * W;
    *reinterpret_cast<T*>(dp) = *reinterpret_cast<const T*>(sp);
  }
}

int stacked_from(const cs_view* v, stacked* out) {
  CS_REQUIRE(v && v->data && (v->ndim == 5 || v->ndim == 4), "cache must be a 4-d or 5-d view");
  int es = dtype_size(v->dtype);
  CS_REQUIRE(es > 0, "unknown cache dtype");
  int o = v->ndim == 5 ? 1 : 0;
  CS_REQUIRE(v->stride[o + 3] == 1, "cache records must be contiguous");
  stacked c{};
  c.base = static_cast<char*>(v->data);
  c.layers = o ? v->shape[0] : 1;
  c.s_layer = o ? v->stride[0] * es : 0;
  c.blocks = v->shape[o + 0];
  c.heads = v->shape[o + 1];
  c.bs = v->shape[o + 2];
  c.s_block = v->stride[o + 0] * es;
  c.s_head = v->stride[o + 1] * es;
  c.s_off = v->stride[o + 2] * es;
  c.rec_bytes = v->shape[o + 3] * es;
  *out = c;
  return CS_OK;
}

// ---------------------------------------------------------------- maps
__global__ void mapping_scatter_kernel(int64_t* map, int64_t len, const int64_t* tokens,
                                       const int64_t* slots, int64_t n) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) {
    int64_t t = tokens[i];
    if (t >= 0 && t < len) map[t] = slots[i];
  }
}

__global__ void mapping_gather_kernel(const int64_t* map, int64_t len, const int64_t* tokens,
                                      int64_t* out, int64_t n) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) {
    int64_t t = tokens[i];
    out[i] = (t >= 0 && t < len) ? map[t] : -1;
  }
}

// ---------------------------------------------------------------- free list
__global__ void freelist_release_kernel(uint32_t* bitmap, int64_t nbits, const int64_t* slots,
                                        int64_t n) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) {
    int64_t s = slots[i];
    if (s >= 0 && s < nbits) atomicOr(&bitmap[s >> 5], 1u << (s & 31));
  }
}

// Single workgroup: each thread owns a contiguous word range; a block-wide
// exclusive scan of popcounts ranks every free bit, and the `count` lowest
// ranks are taken.  Nothing is modified when fewer than `count` are free.
constexpr int kAcqThreads = 1024;
__global__ void __launch_bounds__(kAcqThreads)
    freelist_acquire_kernel(uint32_t* bitmap, int64_t nbits, int64_t count, int64_t* out,
                            int32_t* status) {
  __shared__ int64_t partial[kAcqThreads];
  const int64_t words = (nbits + 31) >> 5;
  const int tid = threadIdx.x;
  const int64_t per = (words + kAcqThreads - 1) / kAcqThreads;
  const int64_t w0 = tid * per;
  const int64_t w1 = w0 + per < words ? w0 + per : words;
  int64_t mine = 0;
  for (int64_t w = w0; w < w1; ++w) {
    uint32_t bits = bitmap[w];
    if (w == words - 1 && (nbits & 31)) bits &= (1u << (nbits & 31)) - 1u;
    mine += __popc(bits);
  }
  partial[tid] = mine;
  __syncthreads();
  // Hillis-Steele inclusive scan over 1024 partial counts.
  for (int o = 1; o < kAcqThreads; o <<= 1) {
    int64_t v = tid >= o ? partial[tid - o] : 0;
    __syncthreads();
    partial[tid] += v;
    __syncthreads();
  }
  const int64_t total = partial[kAcqThreads - 1];
  if (total < count) {
    if (tid == 0) *status = CS_ECAPACITY;
    return;
  }
  if (tid == 0) *status = CS_OK;
  int64_t rank = partial[tid] - mine;  // exclusive prefix
  for (int64_t w = w0; w < w1 && rank < count; ++w) {
    uint32_t bits = bitmap[w];
    if (w == words - 1 && (nbits & 31)) bits &= (1u << (nbits & 31)) - 1u;
    uint32_t taken = 0;
    while (bits && rank < count) {
      int b = __ffs(bits) - 1;
      bits &= bits - 1;
      taken |= 1u << b;
      out[rank++] = (w << 5) + b;
    }
    if (taken) bitmap[w] &= ~taken;
  }
}

}  // namespace
}  // namespace cs

using namespace cs;

extern "C" int cs_slot_scatter(const cs_view* cache, const cs_view* side_k, const cs_view* side_v,
                               const int64_t* slots, const int64_t* rows, int64_t n,
                               const cs_view* key, const cs_view* value, void* stream) {
  return slot_move(cache, side_k, side_v, slots, rows, n, key, value, true, stream);
}

extern "C" int cs_slot_gather(const cs_view* cache, const cs_view* side_k, const cs_view* side_v,
                              const int64_t* slots, const int64_t* rows, int64_t n, cs_view* key,
                              cs_view* value, void* stream) {
  return slot_move(cache, side_k, side_v, slots, rows, n, key, value, false, stream);
}

extern "C" int cs_slot_copy(const cs_view* cache, const int64_t* src_slots,
                            const int64_t* dst_slots, int64_t n, void* stream) {
  stacked c;
  int st = stacked_from(cache, &c);
  if (st) return st;
  if (n == 0) return CS_OK;
  CS_REQUIRE(src_slots && dst_slots, "null slot arrays");
  int w = pick_width(c.rec_bytes, {c.base}, {c.s_layer, c.s_block, c.s_head, c.s_off});
  int64_t chunks = c.rec_bytes / w;
  int64_t total = n * c.layers * c.heads * chunks;
  int grid = grid_for(total, 256);
  hipStream_t s = as_stream(stream);
  switch (w) {
    case 16: hipLaunchKernelGGL(slot_copy_kernel<16>, dim3(grid), dim3(256), 0, s, c, src_slots, dst_slots, n, chunks); break;
    case 8: hipLaunchKernelGGL(slot_copy_kernel<8>, dim3(grid), dim3(256), 0, s, c, src_slots, dst_slots, n, chunks); break;
    case 4: hipLaunchKernelGGL(slot_copy_kernel<4>, dim3(grid), dim3(256), 0, s, c, src_slots, dst_slots, n, chunks); break;
    case 2: hipLaunchKernelGGL(slot_copy_kernel<2>, dim3(grid), dim3(256), 0, s, c, src_slots, dst_slots, n, chunks); break;
    default: hipLaunchKernelGGL(slot_copy_kernel<1>, dim3(grid), dim3(256), 0, s, c, src_slots, dst_slots, n, chunks); break;
  }
  CS_LAUNCH_CHECK("slot_copy");
  return CS_OK;
}

extern "C" int cs_page_copy(const cs_view* cache, const int64_t* src_blocks,
                            const int64_t* dst_blocks, int64_t n, void* stream) {
  stacked c;
  int st = stacked_from(cache, &c);
  if (st) return st;
  if (n == 0) return CS_OK;
  CS_REQUIRE(src_blocks && dst_blocks, "null block arrays");
  int w = pick_width(c.rec_bytes, {c.base}, {c.s_layer, c.s_block, c.s_head, c.s_off});
  int64_t chunks = c.rec_bytes / w;
  int64_t total = n * c.layers * c.heads * c.bs * chunks;
  int grid = grid_for(total, 256);
  hipStream_t s = as_stream(stream);
  switch (w) {
    case 16: hipLaunchKernelGGL(page_copy_kernel<16>, dim3(grid), dim3(256), 0, s, c, src_blocks, dst_blocks, n, chunks); break;
    case 8: hipLaunchKernelGGL(page_copy_kernel<8>, dim3(grid), dim3(256), 0, s, c, src_blocks, dst_blocks, n, chunks); break;
    case 4: hipLaunchKernelGGL(page_copy_kernel<4>, dim3(grid), dim3(256), 0, s, c, src_blocks, dst_blocks, n, chunks); break;
    case 2: hipLaunchKernelGGL(page_copy_kernel<2>, dim3(grid), dim3(256), 0, s, c, src_blocks, dst_blocks, n, chunks); break;
    default: hipLaunchKernelGGL(page_copy_kernel<1>, dim3(grid), dim3(256), 0, s, c, src_blocks, dst_blocks, n, chunks); break;
  }
  CS_LAUNCH_CHECK("page_copy");
  return CS_OK;
}

extern "C" int cs_mapping_scatter(int64_t* map, int64_t map_len, const int64_t* tokens,
                                  const int64_t* slots, int64_t n, void* stream) {
  if (n == 0) return CS_OK;
  CS_REQUIRE(map && tokens && slots, "null map arrays");
  hipLaunchKernelGGL(mapping_scatter_kernel, dim3(ceil_div(n, 256)), dim3(256), 0,
                     as_stream(stream), map, map_len, tokens, slots, n);
  CS_LAUNCH_CHECK("mapping_scatter");
  return CS_OK;
}

extern "C" int cs_mapping_gather(const int64_t* map, int64_t map_len, const int64_t* tokens,
                                 int64_t* out, int64_t n, void* stream) {
  if (n == 0) return CS_OK;
  CS_REQUIRE(map && tokens && out, "null map arrays");
  hipLaunchKernelGGL(mapping_gather_kernel, dim3(ceil_div(n, 256)), dim3(256), 0,
                     as_stream(stream), map, map_len, tokens, out, n);
  CS_LAUNCH_CHECK("mapping_gather");
  return CS_OK;
}

extern "C" int cs_freelist_release(uint32_t* bitmap, int64_t nbits, const int64_t* slots,
                                   int64_t n, void* stream) {
  if (n == 0) return CS_OK;
  CS_REQUIRE(bitmap && slots, "null free-list arrays");
  hipLaunchKernelGGL(freelist_release_kernel, dim3(ceil_div(n, 256)), dim3(256), 0,
                     as_stream(stream), bitmap, nbits, slots, n);
  CS_LAUNCH_CHECK("freelist_release");
  return CS_OK;
}

extern "C" int cs_freelist_acquire(uint32_t* bitmap, int64_t nbits, int64_t count, int64_t* out,
                                   int32_t* status_out, void* stream) {
  CS_REQUIRE(bitmap && status_out && (count == 0 || out), "null free-list arrays");
  CS_REQUIRE(count >= 0 && nbits >= 0, "negative sizes");
  hipLaunchKernelGGL(freelist_acquire_kernel, dim3(1), dim3(kAcqThreads), 0, as_stream(stream),
                     bitmap, nbits, count, out, status_out);
  CS_LAUNCH_CHECK("freelist_acquire");
  return CS_OK;
}
