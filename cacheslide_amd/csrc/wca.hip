// Weighted Correction Attention (WCA) kernels, fp64 throughout.
//
// Reference: src/cacheslide_vllm/wca.py
//   squared_deviation  :55-62   err[t]  = sum_{h,d} (new - old)^2      (fp64)
//   adaptation_weight  :65-93   alpha   = err / (sum old^2 + eps), optional clamp
//   mean_head_cosine   :96-112  mean over heads of clamped cosine of amax-scaled rows
//   WCAState._promote  :202-215 stable descending selection, ties -> lower index
//   WCAState.update    :217-304 fused = w * new + (1 - w) * old, cast to the cache dtype
//
// Per-token sums are computed exactly: every (rounded) fp64 square is added
// into a double-double accumulator and the total is rounded once, so the
// result is the correctly rounded sum and does not depend on the reduction
// order.  Torch's CPU reduction rounds partial sums and can differ from it by
// a few ulps; the oracle uses math.fsum, which is also correctly rounded.
//
// This translation unit is compiled with -ffp-contract=off so that no
// multiply/add pair is fused: the blend and the squares round exactly where
// the reference's separate tensor operations round.

#include "common.h"

namespace cs {
namespace {

constexpr int kWaves = 4;

struct dd {
  double hi, lo;
};

__device__ inline void two_sum(double a, double b, double& s, double& e) {
  s = a + b;
  double bb = s - a;
  e = (a - (s - bb)) + (b - bb);
}

__device__ inline dd dd_add_double(dd x, double y) {
  double s, e;
  two_sum(x.hi, y, s, e);
  dd r;
  r.hi = s;
  r.lo = x.lo + e;
  return r;
}

__device__ inline dd dd_add(dd x, dd y) {
  double s, e;
  two_sum(x.hi, y.hi, s, e);
  e += x.lo + y.lo;
  dd r;
  r.hi = s + e;
  r.lo = e - (r.hi - s);
  return r;
}

__device__ inline dd dd_wave_sum(dd v) {
  for (int off = 32; off > 0; off >>= 1) {
    dd o;
    o.hi = __shfl_xor(v.hi, off, 64);
    o.lo = __shfl_xor(v.lo, off, 64);
    v = dd_add(v, o);
  }
  return v;
}

__device__ inline double dd_round(dd v) {
  double s = v.hi + v.lo;
  return s;
}

// One wavefront per token.
__global__ void __launch_bounds__(64 * kWaves) wca_score_kernel(dview old_src,
                                                                const int64_t* old_rows,
                                                                dview fresh, double* err,
                                                                double* norm, int32_t* flags) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  const int64_t n = fresh.shape[0], H = fresh.shape[1], D = fresh.shape[2];
  if (i >= n) return;
  const int64_t row = old_rows ? old_rows[i] : i;
  dd e_acc{0.0, 0.0}, n_acc{0.0, 0.0};
  int bad = 0;
  const int64_t HD = H * D;
  for (int64_t x = lane; x < HD; x += 64) {
    int64_t h = x / D, d = x % D;
    double o = load_as_double(old_src.data, old_src.dtype,
                              row * old_src.stride[0] + h * old_src.stride[1] + d * old_src.stride[2]);
    double f = load_as_double(fresh.data, fresh.dtype,
                              i * fresh.stride[0] + h * fresh.stride[1] + d * fresh.stride[2]);
    if (!isfinite(o) || !isfinite(f)) bad = 1;
    double diff = f - o;
    double sq = diff * diff;
    double osq = o * o;
    e_acc = dd_add_double(e_acc, sq);
    n_acc = dd_add_double(n_acc, osq);
  }
  e_acc = dd_wave_sum(e_acc);
  n_acc = dd_wave_sum(n_acc);
  int any_bad = __any(bad);
  if (lane == 0) {
    double ev = dd_round(e_acc), nv = dd_round(n_acc);
    // an infinite term makes hi infinite and lo NaN; report it as overflow
    if (!isfinite(e_acc.hi)) ev = e_acc.hi != e_acc.hi ? e_acc.hi : INFINITY;
    if (!isfinite(n_acc.hi)) nv = n_acc.hi != n_acc.hi ? n_acc.hi : INFINITY;
    err[i] = ev;
    norm[i] = nv;
    int f = 0;
    if (any_bad) f |= 1;
    if (!isfinite(ev)) f |= 2;
    if (!isfinite(nv)) f |= 16;
    if (f) atomicOr(flags, f);
  }
}

__global__ void wca_alpha_kernel(const double* err, const double* norm, int64_t n, double eps,
                                 int32_t clamp, double* alpha, int32_t* flags) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  double num = err[i];
  double den = norm[i] + eps;
  int f = 0;
  if (!isfinite(num) || !isfinite(den)) f |= 2;
  double a = num / den;
  if (!isfinite(a)) f |= 4;
  if (clamp) a = a < 0.0 ? 0.0 : (a > 1.0 ? 1.0 : a);
  alpha[i] = a;
  if (f) atomicOr(flags, f);
}

// ------------------------------------------------------------ promotion
constexpr int kSelThreads = 1024;

__device__ inline uint64_t key_bits(double k) {
  uint64_t u = __double_as_longlong(k);
  // err >= 0, so the IEEE pattern is monotone; map -0.0 to +0.0.
  return (u >> 63) ? 0ull : u;
}

// Block-wide exclusive scan of one int per thread; returns the total.
__device__ inline int block_exclusive_scan(int v, int* tmp, int& excl) {
  const int tid = threadIdx.x;
  tmp[tid] = v;
  __syncthreads();
  for (int o = 1; o < kSelThreads; o <<= 1) {
    int add = tid >= o ? tmp[tid - o] : 0;
    __syncthreads();
    tmp[tid] += add;
    __syncthreads();
  }
  int incl = tmp[tid];
  int total = tmp[kSelThreads - 1];
  __syncthreads();
  excl = incl - v;
  return total;
}

__global__ void __launch_bounds__(kSelThreads) wca_promote_kernel(
    const double* key, const uint8_t* candidate, const uint8_t* removed, uint8_t* selected,
    int64_t n, int64_t budget, int64_t* scratch, int64_t* promoted, int64_t* count_out) {
  __shared__ int hist[256];
  __shared__ int scan_tmp[kSelThreads];
  __shared__ uint64_t s_prefix, s_mask;
  __shared__ int64_t s_remaining, s_k;
  __shared__ uint64_t tile_key[kSelThreads];
  __shared__ int tile_sel[kSelThreads];
  const int tid = threadIdx.x;

  // slots = max(0, budget - #selected); available = candidate & ~selected & ~removed
  int cnt_sel = 0, cnt_av = 0;
  for (int64_t t = tid; t < n; t += kSelThreads) {
    bool s = selected[t] != 0;
    cnt_sel += s;
    cnt_av += (candidate[t] && !s && !removed[t]);
  }
  int ex;
  int total_sel = block_exclusive_scan(cnt_sel, scan_tmp, ex);
  int total_av = block_exclusive_scan(cnt_av, scan_tmp, ex);
  int64_t slots = budget - total_sel;
  if (slots < 0) slots = 0;
  const int64_t k = slots < total_av ? slots : total_av;
  if (tid == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_remaining = k;
    s_k = k;
    *count_out = k;
  }
  __syncthreads();
  if (k == 0) return;

  // Radix select (8 x 8 bits, most significant first) of the k-th largest key.
  for (int pass = 0; pass < 8; ++pass) {
    const int shift = 56 - 8 * pass;
    for (int i = tid; i < 256; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    const uint64_t prefix = s_prefix, mask = s_mask;
    for (int64_t t = tid; t < n; t += kSelThreads) {
      if (candidate[t] && !selected[t] && !removed[t]) {
        uint64_t kb = key_bits(key[t]);
        if ((kb & mask) == prefix) atomicAdd(&hist[(kb >> shift) & 255], 1);
      }
    }
    __syncthreads();
    if (tid == 0) {
      int64_t need = s_remaining, cum = 0;
      int chosen = 0;
      for (int bin = 255; bin >= 0; --bin) {
        if (cum + hist[bin] >= need) {
          chosen = bin;
          need -= cum;
          break;
        }
        cum += hist[bin];
      }
      s_remaining = need;
      s_prefix = prefix | (static_cast<uint64_t>(chosen) << shift);
      s_mask = mask | (255ull << shift);
    }
    __syncthreads();
  }
  const uint64_t thr = s_prefix;
  const int64_t need_eq = s_remaining;  // how many keys equal to thr are taken

  // Mark the selection: all keys > thr, plus the need_eq lowest-index keys == thr.
  // The new marks go to bit 1 of selected[] until the ordering pass is done.
  int64_t eq_seen = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kSelThreads) {
    int64_t t = c0 + tid;
    int flag_gt = 0, flag_eq = 0;
    if (t < n && candidate[t] && !selected[t] && !removed[t]) {
      uint64_t kb = key_bits(key[t]);
      flag_gt = kb > thr;
      flag_eq = kb == thr;
    }
    int rank;
    int tot = block_exclusive_scan(flag_eq, scan_tmp, rank);
    if (t < n && (flag_gt || (flag_eq && eq_seen + rank < need_eq))) selected[t] |= 2;
    eq_seen += tot;
  }
  __threadfence_block();
  __syncthreads();

  // Compact the new selection (index order) into scratch[0..k).
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kSelThreads) {
    int64_t t = c0 + tid;
    int f = (t < n && (selected[t] & 2)) ? 1 : 0;
    int ex2;
    int tot = block_exclusive_scan(f, scan_tmp, ex2);
    if (f) scratch[base + ex2] = t;
    base += tot;
  }
  __threadfence_block();
  __syncthreads();
  // Order by (key desc, index asc): rank_i = #{j: key_j > key_i} + #{j: key_j == key_i, j < i}
  // over the k compacted entries, staged through LDS tiles.
  for (int64_t c0 = 0; c0 < k; c0 += kSelThreads) {
    const int64_t i = c0 + tid;
    const bool mine = i < k;
    const int64_t ti = mine ? scratch[i] : 0;
    const uint64_t ki = mine ? key_bits(key[ti]) : 0;
    int64_t rank = 0;
    for (int64_t d0 = 0; d0 < k; d0 += kSelThreads) {
      const int64_t j = d0 + tid;
      __syncthreads();
      tile_sel[tid] = j < k ? static_cast<int>(scratch[j]) : -1;
      tile_key[tid] = j < k ? key_bits(key[scratch[j]]) : 0;
      __syncthreads();
      if (mine) {
        const int lim = (k - d0) < kSelThreads ? static_cast<int>(k - d0) : kSelThreads;
        for (int x = 0; x < lim; ++x) {
          const uint64_t kj = tile_key[x];
          if (kj > ki || (kj == ki && tile_sel[x] < ti)) ++rank;
        }
      }
    }
    if (mine) promoted[rank] = ti;
  }
  __syncthreads();
  for (int64_t t = tid; t < n; t += kSelThreads)
    if (selected[t] & 2) selected[t] = 1;
}

// Ascending indices of (a[t] | b[t]) (b may be null): single workgroup.
__global__ void __launch_bounds__(kSelThreads) mask_nonzero_kernel(const uint8_t* a,
                                                                   const uint8_t* b, int64_t n,
                                                                   int64_t* out,
                                                                   int64_t* count) {
  __shared__ int scan_tmp[kSelThreads];
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kSelThreads) {
    int64_t t = c0 + threadIdx.x;
    int f = 0;
    if (t < n) f = (a[t] != 0) || (b && b[t] != 0);
    int ex;
    int tot = block_exclusive_scan(f, scan_tmp, ex);
    if (f) out[base + ex] = t;
    base += tot;
  }
  if (threadIdx.x == 0) *count = base;
}

// fused = w * new + (1 - w) * old.  One thread per element of [a, H, D].
__global__ void wca_blend_kernel(dview old_k, dview old_v, const int64_t* rows, dview new_k,
                                 dview new_v, const double* weight, const uint8_t* mandatory,
                                 dview fused_k, dview fused_v, int32_t* flags) {
  const int64_t a = new_k.shape[0], H = new_k.shape[1], D = new_k.shape[2];
  const int64_t total = a * H * D;
  int bad = 0;
  for (int64_t x = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; x < total;
       x += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t d = x % D, h = (x / D) % H, i = x / (D * H);
    int64_t row = rows ? rows[i] : i;
    double w = (mandatory && mandatory[i]) ? 1.0 : weight[i];
    double one_minus = 1.0 - w;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const dview& ov = kv ? old_v : old_k;
      const dview& nv = kv ? new_v : new_k;
      const dview& fv = kv ? fused_v : fused_k;
      double o = load_as_double(ov.data, ov.dtype, row * ov.stride[0] + h * ov.stride[1] + d * ov.stride[2]);
      double nw = load_as_double(nv.data, nv.dtype, i * nv.stride[0] + h * nv.stride[1] + d * nv.stride[2]);
      double t1 = w * nw;
      double t2 = one_minus * o;
      double f = t1 + t2;
      int64_t off = i * fv.stride[0] + h * fv.stride[1] + d * fv.stride[2];
      store_from_double(fv.data, fv.dtype, off, f);
      double back = load_as_double(fv.data, fv.dtype, off);
      if (!isfinite(back)) bad = 1;
    }
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flags, 8);
}

// mean_head_cosine: one wavefront per token.
__global__ void __launch_bounds__(64 * kWaves) wca_cosine_kernel(dview a, dview b,
                                                                 const int64_t* b_rows,
                                                                 double eps, double* out) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  const int64_t n = a.shape[0], H = a.shape[1], D = a.shape[2];
  if (i >= n) return;
  const int64_t bi = b_rows ? b_rows[i] : i;
  const double tiny = 2.2250738585072014e-308;
  double total = 0.0;
  for (int64_t h = 0; h < H; ++h) {
    double amax = 0.0, bmax = 0.0;
    for (int64_t d = lane; d < D; d += 64) {
      double x = load_as_double(a.data, a.dtype, i * a.stride[0] + h * a.stride[1] + d * a.stride[2]);
      double y = load_as_double(b.data, b.dtype, bi * b.stride[0] + h * b.stride[1] + d * b.stride[2]);
      amax = fmax(amax, fabs(x));
      bmax = fmax(bmax, fabs(y));
    }
    amax = wave_max(amax);
    bmax = wave_max(bmax);
    double as = amax > eps ? amax : eps;
    double bs = bmax > eps ? bmax : eps;
    double na = 0.0, nb = 0.0;
    for (int64_t d = lane; d < D; d += 64) {
      double x = load_as_double(a.data, a.dtype, i * a.stride[0] + h * a.stride[1] + d * a.stride[2]) / as;
      double y = load_as_double(b.data, b.dtype, bi * b.stride[0] + h * b.stride[1] + d * b.stride[2]) / bs;
      na += x * x;
      nb += y * y;
    }
    na = sqrt(wave_sum(na));
    nb = sqrt(wave_sum(nb));
    double da = na > tiny ? na : tiny;
    double db = nb > tiny ? nb : tiny;
    double dot = 0.0;
    for (int64_t d = lane; d < D; d += 64) {
      double x = load_as_double(a.data, a.dtype, i * a.stride[0] + h * a.stride[1] + d * a.stride[2]) / as / da;
      double y = load_as_double(b.data, b.dtype, bi * b.stride[0] + h * b.stride[1] + d * b.stride[2]) / bs / db;
      dot += x * y;
    }
    dot = wave_sum(dot);
    dot = dot < -1.0 ? -1.0 : (dot > 1.0 ? 1.0 : dot);
    total += dot;
  }
  if (lane == 0) out[i] = total / static_cast<double>(H);
}

// WCAState.initialize masks (wca.py:161-171): candidate = reused & (err > 0);
// counts[0] = #reused, counts[1] = #candidates; flag 32 when a token is neither
// reused nor mandatory.  Single workgroup.
__global__ void __launch_bounds__(kSelThreads) wca_init_masks_kernel(
    const double* err, const uint8_t* reused, const uint8_t* mandatory, int64_t n,
    uint8_t* candidate, int64_t* counts, int32_t* flags) {
  __shared__ int scan_tmp[kSelThreads];
  int nr = 0, nc = 0, bad = 0;
  for (int64_t t = threadIdx.x; t < n; t += kSelThreads) {
    bool r = reused[t] != 0;
    bool c = r && err[t] > 0.0;
    candidate[t] = c ? 1 : 0;
    nr += r;
    nc += c;
    if (!r && !mandatory[t]) bad = 1;
  }
  int ex;
  int tr = block_exclusive_scan(nr, scan_tmp, ex);
  int tc = block_exclusive_scan(nc, scan_tmp, ex);
  int tb = block_exclusive_scan(bad, scan_tmp, ex);
  if (threadIdx.x == 0) {
    counts[0] = tr;
    counts[1] = tc;
    if (tb) atomicOr(flags, 32);
  }
}

// used[i] = 1 if mandatory[rows[i]] else (previous ? alpha[rows[i]] : next[i])
// (wca.py:257-265).
__global__ void wca_used_alpha_kernel(const double* alpha, const double* next, const int64_t* rows,
                                      const uint8_t* mandatory, int64_t a, int32_t previous,
                                      double* used) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= a) return;
  int64_t r = rows[i];
  used[i] = mandatory[r] ? 1.0 : (previous ? alpha[r] : next[i]);
}

// Gate removal (wca.py:277-287): removed = rows[i] with selected[rows[i]] and
// metric < threshold, metric = cosine (paper_cosine_lt) or 1 - cosine
// (distance_lt); ascending (rows are ascending).  Single workgroup.
__global__ void __launch_bounds__(kSelThreads) wca_gate_kernel(
    const double* cosine, const int64_t* rows, const uint8_t* selected, int64_t a,
    int32_t distance, double threshold, int64_t* removed, int64_t* count) {
  __shared__ int scan_tmp[kSelThreads];
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < a; c0 += kSelThreads) {
    int64_t i = c0 + threadIdx.x;
    int f = 0;
    if (i < a) {
      double metric = distance ? 1.0 - cosine[i] : cosine[i];
      f = selected[rows[i]] && metric < threshold;
    }
    int ex;
    int tot = block_exclusive_scan(f, scan_tmp, ex);
    if (f) removed[base + ex] = rows[i];
    base += tot;
  }
  if (threadIdx.x == 0) *count = base;
}

// Commit (wca.py:289-293): alpha[rows[i]] = next[i]; removed tokens leave the
// selection and the candidates and are marked removed.
__global__ void wca_commit_kernel(double* alpha, const double* next, const int64_t* rows, int64_t a,
                                  const int64_t* removed, int64_t nrem, uint8_t* selected,
                                  uint8_t* candidate, uint8_t* removed_mask) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < a) alpha[rows[i]] = next[i];
  if (i < nrem) {
    int64_t t = removed[i];
    selected[t] = 0;
    candidate[t] = 0;
    removed_mask[t] = 1;
  }
}

int grid_for(int64_t total, int threads) {
  int64_t g = ceil_div(total, threads);
  if (g > 65535 * 16) g = 65535 * 16;
  return static_cast<int>(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace cs

extern "C" int cs_wca_init_masks(const double* err, const uint8_t* reused, const uint8_t* mandatory,
                                 int64_t n, uint8_t* candidate, int64_t* counts, int32_t* flags,
                                 void* stream) {
  CS_REQUIRE(err && reused && mandatory && candidate && counts && flags, "null arguments");
  hipLaunchKernelGGL(cs::wca_init_masks_kernel, dim3(1), dim3(cs::kSelThreads), 0,
                     cs::as_stream(stream), err, reused, mandatory, n, candidate, counts, flags);
  CS_LAUNCH_CHECK("wca_init_masks");
  return CS_OK;
}

extern "C" int cs_wca_used_alpha(const double* alpha, const double* next, const int64_t* rows,
                                 const uint8_t* mandatory, int64_t a, int32_t previous_layer,
                                 double* used, void* stream) {
  if (a == 0) return CS_OK;
  CS_REQUIRE(alpha && next && rows && mandatory && used, "null arguments");
  hipLaunchKernelGGL(cs::wca_used_alpha_kernel, dim3(cs::ceil_div(a, 256)), dim3(256), 0,
                     cs::as_stream(stream), alpha, next, rows, mandatory, a, previous_layer, used);
  CS_LAUNCH_CHECK("wca_used_alpha");
  return CS_OK;
}

extern "C" int cs_wca_gate(const double* cosine, const int64_t* rows, const uint8_t* selected,
                           int64_t a, int32_t distance_mode, double threshold, int64_t* removed,
                           int64_t* count, void* stream) {
  CS_REQUIRE(rows && selected && removed && count && (a == 0 || cosine), "null arguments");
  hipLaunchKernelGGL(cs::wca_gate_kernel, dim3(1), dim3(cs::kSelThreads), 0, cs::as_stream(stream),
                     cosine, rows, selected, a, distance_mode, threshold, removed, count);
  CS_LAUNCH_CHECK("wca_gate");
  return CS_OK;
}

extern "C" int cs_wca_commit(double* alpha, const double* next, const int64_t* rows, int64_t a,
                             const int64_t* removed, int64_t nrem, uint8_t* selected,
                             uint8_t* candidate, uint8_t* removed_mask, void* stream) {
  int64_t n = a > nrem ? a : nrem;
  if (n == 0) return CS_OK;
  CS_REQUIRE(alpha && selected && candidate && removed_mask, "null arguments");
  hipLaunchKernelGGL(cs::wca_commit_kernel, dim3(cs::ceil_div(n, 256)), dim3(256), 0,
                     cs::as_stream(stream), alpha, next, rows, a, removed, nrem, selected,
                     candidate, removed_mask);
  CS_LAUNCH_CHECK("wca_commit");
  return CS_OK;
}

using namespace cs;

extern "C" int cs_wca_score(const cs_view* old_rows_src, const int64_t* old_rows,
                            const cs_view* fresh, double* err, double* norm, int32_t* flags,
                            void* stream) {
  CS_REQUIRE(old_rows_src && fresh && err && norm && flags && old_rows_src->ndim == 3 &&
                 fresh->ndim == 3,
             "old/new must be 3-d views");
  CS_REQUIRE(old_rows_src->shape[1] == fresh->shape[1] && old_rows_src->shape[2] == fresh->shape[2],
             "old/new head shapes differ");
  int64_t n = fresh->shape[0];
  if (n == 0) return CS_OK;
  hipLaunchKernelGGL(wca_score_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0,
                     as_stream(stream), to_dview(old_rows_src), old_rows, to_dview(fresh), err,
                     norm, flags);
  CS_LAUNCH_CHECK("wca_score");
  return CS_OK;
}

extern "C" int cs_wca_alpha(const double* err, const double* norm, int64_t n, double eps,
                            int32_t clamp, double* alpha, int32_t* flags, void* stream) {
  if (n == 0) return CS_OK;
  CS_REQUIRE(err && norm && alpha && flags, "null arguments");
  hipLaunchKernelGGL(wca_alpha_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, as_stream(stream),
                     err, norm, n, eps, clamp, alpha, flags);
  CS_LAUNCH_CHECK("wca_alpha");
  return CS_OK;
}

extern "C" int cs_wca_promote(const double* key, const uint8_t* candidate, const uint8_t* removed,
                              uint8_t* selected, int64_t n, int64_t budget, int64_t* scratch,
                              int64_t* promoted, int64_t* count_out, void* stream) {
  CS_REQUIRE(key && candidate && removed && selected && scratch && promoted && count_out,
             "null arguments");
  CS_REQUIRE(n >= 0 && n <= (1ll << 24), "at most 2^24 tokens");
  hipLaunchKernelGGL(wca_promote_kernel, dim3(1), dim3(kSelThreads), 0, as_stream(stream), key,
                     candidate, removed, selected, n, budget, scratch, promoted, count_out);
  CS_LAUNCH_CHECK("wca_promote");
  return CS_OK;
}

extern "C" int cs_mask_nonzero(const uint8_t* a, const uint8_t* b, int64_t n, int64_t* out,
                               int64_t* count, void* stream) {
  CS_REQUIRE(a && out && count, "null arguments");
  hipLaunchKernelGGL(mask_nonzero_kernel, dim3(1), dim3(kSelThreads), 0, as_stream(stream), a, b,
                     n, out, count);
  CS_LAUNCH_CHECK("mask_nonzero");
  return CS_OK;
}

extern "C" int cs_wca_blend(const cs_view* old_k, const cs_view* old_v, const int64_t* rows,
                            const cs_view* new_k, const cs_view* new_v, const double* weight,
                            const uint8_t* mandatory, cs_view* fused_k, cs_view* fused_v,
                            int32_t* flags, void* stream) {
  CS_REQUIRE(old_k && old_v && new_k && new_v && fused_k && fused_v && weight && flags,
             "null arguments");
  CS_REQUIRE(new_k->ndim == 3 && new_v->ndim == 3 && fused_k->ndim == 3 && fused_v->ndim == 3 &&
                 old_k->ndim == 3 && old_v->ndim == 3,
             "3-d views required");
  int64_t total = new_k->shape[0] * new_k->shape[1] * new_k->shape[2];
  if (total == 0) return CS_OK;
  hipLaunchKernelGGL(wca_blend_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                     as_stream(stream), to_dview(old_k), to_dview(old_v), rows, to_dview(new_k),
                     to_dview(new_v), weight, mandatory, to_dview(fused_k), to_dview(fused_v),
                     flags);
  CS_LAUNCH_CHECK("wca_blend");
  return CS_OK;
}

extern "C" int cs_wca_head_cosine(const cs_view* a, const cs_view* b, const int64_t* b_rows,
                                  double eps, double* out, void* stream) {
  CS_REQUIRE(a && b && out && a->ndim == 3 && b->ndim == 3, "3-d views required");
  int64_t n = a->shape[0];
  if (n == 0) return CS_OK;
  hipLaunchKernelGGL(wca_cosine_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0,
                     as_stream(stream), to_dview(a), to_dview(b), b_rows, eps, out);
  CS_LAUNCH_CHECK("wca_head_cosine");
  return CS_OK;
}
