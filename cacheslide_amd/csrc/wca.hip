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

struct score_acc {
  dd e{0.0, 0.0}, n{0.0, 0.0};
  int bad = 0;
  __device__ void add(double o, double f) {
    if (!isfinite(o) || !isfinite(f)) bad = 1;
    const double diff = f - o;
    const double sq = diff * diff;
    const double osq = o * o;
    e = dd_add_double(e, sq);
    n = dd_add_double(n, osq);
  }
  // Wave reduction; lane 0 stores err[i], norm[i] and the flags.
  __device__ void finish(int lane, int64_t i, double* err, double* norm, int32_t* flags) {
    e = dd_wave_sum(e);
    n = dd_wave_sum(n);
    const int any_bad = __any(bad);
    if (lane == 0) {
      double ev = dd_round(e), nv = dd_round(n);
      // an infinite term makes hi infinite and lo NaN; report it as overflow
      if (!isfinite(e.hi)) ev = e.hi != e.hi ? e.hi : INFINITY;
      if (!isfinite(n.hi)) nv = n.hi != n.hi ? n.hi : INFINITY;
      err[i] = ev;
      norm[i] = nv;
      int f = 0;
      if (any_bad) f |= 1;
      if (!isfinite(ev)) f |= 2;
      if (!isfinite(nv)) f |= 16;
      if (f) atomicOr(flags, f);
    }
  }
};

// One wavefront per token, any dtype and strides.
__global__ void __launch_bounds__(64 * kWaves) wca_score_kernel(dview old_src,
                                                                const int64_t* old_rows,
                                                                dview fresh, double* err,
                                                                double* norm, int32_t* flags) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  const int64_t n = fresh.shape[0], H = fresh.shape[1], D = fresh.shape[2];
  if (i >= n) return;
  const int64_t row = old_rows ? old_rows[i] : i;
  score_acc acc;
  const int64_t HD = H * D;
  for (int64_t x = lane; x < HD; x += 64) {
    int64_t h = x / D, d = x % D;
    acc.add(load_as_double(old_src.data, old_src.dtype,
                           row * old_src.stride[0] + h * old_src.stride[1] + d * old_src.stride[2]),
            load_as_double(fresh.data, fresh.dtype,
                           i * fresh.stride[0] + h * fresh.stride[1] + d * fresh.stride[2]));
  }
  acc.finish(lane, i, err, norm, flags);
}

// bf16 rows whose [H, D] block is contiguous and 16-byte aligned: one
// wavefront per token, 8 elements per 16-byte load.  The per-token sums are
// exact, so the result matches the generic kernel's.
__global__ void __launch_bounds__(64 * kWaves) wca_score_bf16_kernel(
    const uint16_t* old_base, int64_t old_stride, const int64_t* old_rows,
    const uint16_t* new_base, int64_t new_stride, int64_t n, int64_t words, double* err,
    double* norm, int32_t* flags, int32_t old_bit, int32_t new_bit) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (i >= n) return;
  const int64_t row = old_rows ? old_rows[i] : i;
  const uint4* o = reinterpret_cast<const uint4*>(old_base + row * old_stride);
  const uint4* f = reinterpret_cast<const uint4*>(new_base + i * new_stride);
  score_acc acc;
  // with old_bit / new_bit set, the finite checks of both row sets ride on
  // these loads (cs_check_finite's bits, for callers that read every row)
  bool bad_o = false, bad_f = false;
  for (int64_t w = lane; w < words; w += 64) {
    const uint4 ov = o[w], fv = f[w];
    if (old_bit) bad_o |= word_nonfinite<0>(ov);
    if (new_bit) bad_f |= word_nonfinite<0>(fv);
    const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w}, fw[4] = {fv.x, fv.y, fv.z, fv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc.add(bf16_to_float(static_cast<uint16_t>(ow[q])), bf16_to_float(static_cast<uint16_t>(fw[q])));
      acc.add(bf16_to_float(static_cast<uint16_t>(ow[q] >> 16)),
              bf16_to_float(static_cast<uint16_t>(fw[q] >> 16)));
    }
  }
  const int32_t bits = (__any(bad_o) ? old_bit : 0) | (__any(bad_f) ? new_bit : 0);
  if (lane == 0 && bits) atomicOr(flags, bits);
  acc.finish(lane, i, err, norm, flags);
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

// ------------------------------------------------------------ selection
// Selection kernels run as one workgroup of 1024 threads.  Each thread owns a
// run of kRun consecutive tokens per chunk of kChunk tokens, so one block scan
// per chunk orders a whole 16384-token request.
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kRun = 16;
constexpr int64_t kChunk = static_cast<int64_t>(kSelThreads) * kRun;

__device__ inline uint64_t key_bits(double k) {
  uint64_t u = __double_as_longlong(k);
  // err >= 0, so the IEEE pattern is monotone; map -0.0 to +0.0.
  return (u >> 63) ? 0ull : u;
}

// Block-wide exclusive scan of one int per thread; returns the total.  Wave
// scans by lane shifts, then one pass over the 16 wave totals.
__device__ inline int block_scan(int v, int* wave_tot, int& excl) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
  }
  if (lane == 63) wave_tot[w] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    const int t = wave_tot[i];
    before += i < w ? t : 0;
    total += t;
  }
  __syncthreads();
  excl = before + incl - v;
  return total;
}

// block_scan over int64 (several counts packed in fields of one word).
__device__ inline int64_t block_scan64(int64_t v, int64_t* wave_tot, int64_t& excl) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
  }
  if (lane == 63) wave_tot[w] = incl;
  __syncthreads();
  int64_t before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    const int64_t t = wave_tot[i];
    before += i < w ? t : 0;
    total += t;
  }
  __syncthreads();
  excl = before + incl - v;
  return total;
}

// Bit j set when p[start + j] != 0 (j < kRun, start + j < n).
__device__ inline uint32_t run_mask(const uint8_t* p, int64_t start, int64_t n) {
  uint32_t m = 0;
  if (start + kRun <= n && (reinterpret_cast<uintptr_t>(p + start) & 15) == 0) {
    const uint4 v = *reinterpret_cast<const uint4*>(p + start);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        if ((w[q] >> (8 * b)) & 0xffu) m |= 1u << (4 * q + b);
  } else {
    for (int j = 0; j < kRun; ++j)
      if (start + j < n && p[start + j]) m |= 1u << j;
  }
  return m;
}

// key_bits of key[start + j], j < kRun: one batch of 16-byte loads when the
// run is whole (start is a multiple of kRun, so 128-byte aligned for an
// aligned base), clamped scalar loads for the last partial run.
__device__ inline void load_key_run(const double* key, int64_t start, int64_t n, uint64_t kb[kRun]) {
  if (start + kRun <= n && (reinterpret_cast<uintptr_t>(key + start) & 15) == 0) {
    const uint4* p = reinterpret_cast<const uint4*>(key + start);
    uint4 v[kRun / 2];
#pragma unroll
    for (int q = 0; q < kRun / 2; ++q) v[q] = p[q];
#pragma unroll
    for (int q = 0; q < kRun / 2; ++q) {
      kb[2 * q] = key_bits(__longlong_as_double((static_cast<uint64_t>(v[q].y) << 32) | v[q].x));
      kb[2 * q + 1] = key_bits(__longlong_as_double((static_cast<uint64_t>(v[q].w) << 32) | v[q].z));
    }
  } else {
    const int64_t last = n - 1;
#pragma unroll
    for (int j = 0; j < kRun; ++j) kb[j] = key_bits(key[start + j < n ? start + j : last]);
  }
}

// Add one to hist[bin] for every lane with bin >= 0.  Lanes that share the
// first lane's bin are counted with one atomic (up to four rounds), which
// removes the serialisation of many equal bins; the rest add individually.
__device__ inline void hist_add(int* hist, int bin) {
  const int lane = threadIdx.x & 63;
  bool pending = bin >= 0;
#pragma unroll
  for (int round = 0; round < 4; ++round) {
    const uint64_t live = __ballot(pending);
    if (live == 0) return;
    const int leader = __ffsll(static_cast<unsigned long long>(live)) - 1;
    const int lb = __shfl(bin, leader, 64);
    const uint64_t same = __ballot(pending && bin == lb);
    if (lane == leader) atomicAdd(&hist[lb], __popcll(same));
    if (pending && bin == lb) pending = false;
  }
  if (pending) atomicAdd(&hist[bin], 1);
}

// One pass of the radix select (8-bit digit at bit `shift`) over keys held
// in registers: histogram of the available keys under the current prefix
// (one private copy per wavefront, so waves never contend for a bin, then
// summed), then the bin where the count from the top reaches the number
// still needed.
__device__ inline void radix_pass_regs(const uint64_t kb[kRun], uint32_t av, int shift, int* hist,
                                       uint64_t& s_prefix, uint64_t& s_mask, int64_t& s_remaining,
                                       int& s_done) {
  __shared__ int hw[kSelWaves * 256];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int i = tid; i < kSelWaves * 256; i += kSelThreads) hw[i] = 0;
  __syncthreads();
  const uint64_t prefix = s_prefix, mask = s_mask;
  int* mine_hist = hw + (tid >> 6) * 256;
#pragma unroll
  for (int j = 0; j < kRun; ++j) {
    const bool in = ((av >> j) & 1u) && (kb[j] & mask) == prefix;
    if (in) atomicAdd(&mine_hist[static_cast<int>((kb[j] >> shift) & 255)], 1);
  }
  __syncthreads();
  for (int i = tid; i < 256; i += kSelThreads) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) t += hw[w * 256 + i];
    hist[i] = t;
  }
  __syncthreads();
  if (tid < 64) {
    // Bins 4*lane .. 4*lane+3; find the bin where the count from the top reaches need.
    int hb[4], mine = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      hb[q] = hist[4 * lane + q];
      mine += hb[q];
    }
    int above = mine;  // inclusive suffix sum over lanes >= lane
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_down(above, d, 64);
      if (lane + d < 64) above += t;
    }
    above -= mine;  // lanes strictly above
    const int64_t need = s_remaining;
    if (above < need && above + mine >= need) {
      int64_t cum = above;
      for (int q = 3; q >= 0; --q) {
        if (cum + hb[q] >= need) {
          const int bin = 4 * lane + q;
          s_remaining = need - cum;
          s_prefix = prefix | (static_cast<uint64_t>(bin) << shift);
          s_mask = mask | (255ull << shift);
          s_done = (need - cum) == hb[q];
          break;
        }
        cum += hb[q];
      }
    }
  }
  __syncthreads();
}

// Radix select of the k-th largest key over keys held in registers (one
// chunk: kb[j] of the tokens with bit j of av set), with s_prefix = s_mask
// = 0, s_remaining = k and s_done set by the caller and visible.  The bits
// above the highest bit in which the available keys differ are common to
// all of them: they enter the prefix at once (one min/max reduction), and
// the 8-bit passes start below them; the last pass takes bits 0..7.  The
// result -- threshold under the final mask and the number of keys equal to
// it still to take -- is the byte-aligned passes' result.
__device__ inline void radix_select_regs(const uint64_t kb[kRun], uint32_t av, int* hist, uint64_t* wred,
                                         uint64_t& s_prefix, uint64_t& s_mask, int64_t& s_remaining,
                                         int& s_done, int& s_start) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (s_done) return;
  uint64_t lo = ~0ull, hi = 0;
#pragma unroll
  for (int j = 0; j < kRun; ++j) {
    if ((av >> j) & 1u) {
      lo = kb[j] < lo ? kb[j] : lo;
      hi = kb[j] > hi ? kb[j] : hi;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t l2 = __shfl_xor(lo, off, 64), h2 = __shfl_xor(hi, off, 64);
    lo = l2 < lo ? l2 : lo;
    hi = h2 > hi ? h2 : hi;
  }
  if (lane == 0) {
    wred[w] = lo;
    wred[kSelWaves + w] = hi;
  }
  __syncthreads();
  if (tid == 0) {
    uint64_t a = ~0ull, b = 0;
    for (int i = 0; i < kSelWaves; ++i) {
      a = wred[i] < a ? wred[i] : a;
      b = wred[kSelWaves + i] > b ? wred[kSelWaves + i] : b;
    }
    const uint64_t diff = a ^ b;
    if (diff == 0) {  // every available key is equal: take the lowest-index k
      s_prefix = b;
      s_mask = ~0ull;
      s_done = 1;
      s_start = 0;
    } else {
      const int top = 63 - __clzll(static_cast<long long>(diff));
      const uint64_t common = top == 63 ? 0ull : ~0ull << (top + 1);
      s_prefix = b & common;
      s_mask = common;
      s_start = top - 7;
    }
  }
  __syncthreads();
  for (int shift = s_start; !s_done; shift -= 8) {
    const int sh = shift > 0 ? shift : 0;
    radix_pass_regs(kb, av, sh, hist, s_prefix, s_mask, s_remaining, s_done);
    if (sh == 0) break;
  }
}

// WCAState._promote, first half: radix select of the k-th largest available
// key (8-bit digits, most significant first, stopping once the chosen digit's
// bucket is taken whole), then one pass that marks the taken tokens selected
// and compacts them in index order into scratch[0..k), their key bits into
// scratch[n..n+k).  Skips everything
// (count 0) when abort_flags has a bit of abort_mask set, so a failed update
// leaves the selection unchanged.
__device__ void promote_block(
    const double* key, const uint8_t* candidate, const uint8_t* removed, uint8_t* selected,
    int64_t n, int64_t budget, int64_t* scratch, int64_t* count_out,
    const int32_t* abort_flags, int32_t abort_mask) {
  __shared__ int hist[256];
  __shared__ int wave_tot[kSelWaves];
  __shared__ uint64_t wred[2 * kSelWaves];
  __shared__ uint64_t s_prefix, s_mask;
  __shared__ int64_t s_remaining;
  __shared__ int s_done, s_start;
  const int tid = threadIdx.x, lane = tid & 63;
  if (abort_flags && (*abort_flags & abort_mask)) {
    if (tid == 0) *count_out = 0;
    return;
  }

  // slots = max(0, budget - #selected); available = candidate & ~selected & ~removed
  int cnt_sel = 0, cnt_av = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kChunk) {
    const int64_t s = c0 + static_cast<int64_t>(tid) * kRun;
    const uint32_t sel = run_mask(selected, s, n);
    const uint32_t av = run_mask(candidate, s, n) & ~sel & ~run_mask(removed, s, n);
    cnt_sel += __popc(sel);
    cnt_av += __popc(av);
  }
  int ex;
  const int total_sel = block_scan(cnt_sel, wave_tot, ex);
  const int total_av = block_scan(cnt_av, wave_tot, ex);
  int64_t slots = budget - total_sel;
  if (slots < 0) slots = 0;
  const int64_t k = slots < total_av ? slots : total_av;
  if (tid == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_remaining = k;
    s_done = k == total_av;  // every available token is taken
    *count_out = k;
  }
  __syncthreads();
  if (k == 0) return;

  // A request of at most one chunk keeps its keys and availability in registers.
  const bool single = n <= kChunk;
  uint64_t kb[kRun] = {};
  uint32_t av = 0;
  if (single) {
    const int64_t s = static_cast<int64_t>(tid) * kRun;
    av = run_mask(candidate, s, n) & ~run_mask(selected, s, n) & ~run_mask(removed, s, n);
    if (s < n) load_key_run(key, s, n, kb);
    radix_select_regs(kb, av, hist, wred, s_prefix, s_mask, s_remaining, s_done, s_start);
  }
  for (int pass = 0; pass < 8 && !single && !s_done; ++pass) {
    const int shift = 56 - 8 * pass;
    for (int i = tid; i < 256; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    const uint64_t prefix = s_prefix, mask = s_mask;
    for (int64_t c0 = 0; c0 < n; c0 += kChunk) {
      const int64_t s = c0 + static_cast<int64_t>(tid) * kRun;
      if (!single) {
        av = run_mask(candidate, s, n) & ~run_mask(selected, s, n) & ~run_mask(removed, s, n);
        if (s < n) load_key_run(key, s, n, kb);
      }
#pragma unroll
      for (int j = 0; j < kRun; ++j) {
        const bool in = ((av >> j) & 1u) && (kb[j] & mask) == prefix;
        hist_add(hist, in ? static_cast<int>((kb[j] >> shift) & 255) : -1);
      }
    }
    __syncthreads();
    if (tid < 64) {
      // Bins 4*lane .. 4*lane+3; find the bin where the count from the top reaches need.
      int hb[4], mine = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        hb[q] = hist[4 * lane + q];
        mine += hb[q];
      }
      int above = mine;  // inclusive suffix sum over lanes >= lane
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_down(above, d, 64);
        if (lane + d < 64) above += t;
      }
      above -= mine;  // lanes strictly above
      const int64_t need = s_remaining;
      if (above < need && above + mine >= need) {
        int64_t cum = above;
        for (int q = 3; q >= 0; --q) {
          if (cum + hb[q] >= need) {
            const int bin = 4 * lane + q;
            s_remaining = need - cum;
            s_prefix = prefix | (static_cast<uint64_t>(bin) << shift);
            s_mask = mask | (255ull << shift);
            s_done = (need - cum) == hb[q];
            break;
          }
          cum += hb[q];
        }
      }
    }
    __syncthreads();
  }
  const uint64_t thr = s_prefix, mask = s_mask;
  const int64_t need_eq = s_remaining;  // keys equal to thr (under mask) taken, lowest index first

  // Mark and compact: all keys above thr, plus the need_eq lowest-index keys equal to it.
  int64_t eq_seen = 0, base = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kChunk) {
    const int64_t s = c0 + static_cast<int64_t>(tid) * kRun;
    if (!single) {
      av = run_mask(candidate, s, n) & ~run_mask(selected, s, n) & ~run_mask(removed, s, n);
      if (s < n) load_key_run(key, s, n, kb);
    }
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const uint64_t km = kb[j] & mask;
      if (((av >> j) & 1u) && km > thr) gt |= 1u << j;
      if (((av >> j) & 1u) && km == thr) eq |= 1u << j;
    }
    int eq_rank;
    const int eq_tot = block_scan(__popc(eq), wave_tot, eq_rank);
    uint32_t take = gt;
    for (uint32_t m = eq; m; m &= m - 1) {
      if (eq_seen + eq_rank < need_eq) take |= m & (~m + 1);
      ++eq_rank;
    }
    int pos;
    const int tot = block_scan(__popc(take), wave_tot, pos);
    for (uint32_t m = take; m; m &= m - 1) {
      const int j = __ffs(m) - 1;
      scratch[base + pos] = s + j;
      scratch[n + base + pos] = static_cast<int64_t>(kb[j]);
      ++pos;
      selected[s + j] = 1;
    }
    eq_seen += eq_tot;
    base += tot;
  }
}

__global__ void __launch_bounds__(kSelThreads) wca_promote_kernel(
    const double* key, const uint8_t* candidate, const uint8_t* removed, uint8_t* selected,
    int64_t n, int64_t budget, int64_t* scratch, int64_t* count_out,
    const int32_t* abort_flags, int32_t abort_mask) {
  promote_block(key, candidate, removed, selected, n, budget, scratch, count_out, abort_flags,
                abort_mask);
}

// Second half of the promotion: orders the k = *count promoted tokens
// (scratch[0..k) in index order, their key bits at scratch[n..n+k)) by (key
// descending, index ascending): rank_i = #{j: key_j > key_i} + #{j < i:
// key_j == key_i}.  A workgroup ranks 64 entries (one per lane); each of its
// 16 wavefronts counts over a sixteenth of the keys, read as wave-uniform
// scalar loads, and the partial counts are summed through LDS.
constexpr int kOrderSlices = 16;

__global__ void __launch_bounds__(64 * kOrderSlices) wca_promote_order_kernel(
    const int64_t* scratch, int64_t n, const int64_t* count, int64_t* promoted, int64_t done_upto) {
  __shared__ int partial[kOrderSlices][64];
  const int64_t k = *count;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * 64;
  if (e0 >= k || k <= done_upto) return;  // done_upto: promotions already ordered
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint64_t* keys = reinterpret_cast<const uint64_t*>(scratch + n);
  const int64_t i = e0 + lane;
  const bool mine = i < k;
  const uint64_t ki = keys[mine ? i : e0];
  const int64_t per = (k + kOrderSlices - 1) / kOrderSlices;
  const int64_t j0 = w * per < k ? w * per : k;
  const int64_t j1 = j0 + per < k ? j0 + per : k;
  int rank = 0;
  int64_t j = j0;
  for (; j + 8 <= j1; j += 8) {
    uint64_t kj[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) kj[u] = keys[j + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) rank += (kj[u] > ki) || (kj[u] == ki && j + u < i);
  }
  for (; j < j1; ++j) {
    const uint64_t kj = keys[j];
    rank += (kj > ki) || (kj == ki && j < i);
  }
  partial[w][lane] = rank;
  __syncthreads();
  if (w == 0 && mine) {
    int r = 0;
#pragma unroll
    for (int q = 0; q < kOrderSlices; ++q) r += partial[q][lane];
    promoted[r] = scratch[i];
  }
}

// Ascending indices of (a[t] | b[t]) (b may be null).
__device__ void nonzero_block(const uint8_t* a, const uint8_t* b, int64_t n, int64_t* out,
                              int64_t* count) {
  __shared__ int wave_tot[kSelWaves];
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kChunk) {
    const int64_t s = c0 + static_cast<int64_t>(threadIdx.x) * kRun;
    uint32_t m = run_mask(a, s, n);
    if (b) m |= run_mask(b, s, n);
    int pos;
    const int tot = block_scan(__popc(m), wave_tot, pos);
    for (; m; m &= m - 1) out[base + pos++] = s + (__ffs(m) - 1);
    base += tot;
  }
  if (threadIdx.x == 0) *count = base;
}

__global__ void __launch_bounds__(kSelThreads) mask_nonzero_kernel(const uint8_t* a,
                                                                   const uint8_t* b, int64_t n,
                                                                   int64_t* out, int64_t* count) {
  nonzero_block(a, b, n, out, count);
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

// bf16 fast path of the blend: rows with contiguous 16-byte aligned [H, D]
// blocks, one thread per 8 elements of K and of V, same fp64 arithmetic.
__device__ inline uint32_t blend_pair(uint32_t o, uint32_t nw, double w, double one_minus, int& bad) {
  uint32_t out = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const double od = bf16_to_float(static_cast<uint16_t>(o >> (16 * h)));
    const double nd = bf16_to_float(static_cast<uint16_t>(nw >> (16 * h)));
    const double t1 = w * nd;
    const double t2 = one_minus * od;
    const uint16_t r = double_to_bf16(t1 + t2);
    if ((r & 0x7f80u) == 0x7f80u) bad = 1;
    out |= static_cast<uint32_t>(r) << (16 * h);
  }
  return out;
}

__global__ void wca_blend_bf16_kernel(const uint16_t* old_k, int64_t ok_s, const uint16_t* old_v,
                                      int64_t ov_s, const int64_t* rows, const uint16_t* new_k,
                                      int64_t nk_s, const uint16_t* new_v, int64_t nv_s,
                                      const double* weight, const uint8_t* mandatory,
                                      uint16_t* fused_k, int64_t fk_s, uint16_t* fused_v,
                                      int64_t fv_s, int64_t a, int64_t words, int32_t* flags) {
  int bad = 0;
  const int64_t total = a * words;
  for (int64_t x = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; x < total;
       x += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = x / words, w = x % words;
    const int64_t row = rows ? rows[i] : i;
    const double wt = (mandatory && mandatory[i]) ? 1.0 : weight[i];
    const double one_minus = 1.0 - wt;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const uint4 o = reinterpret_cast<const uint4*>((kv ? old_v : old_k) + row * (kv ? ov_s : ok_s))[w];
      const uint4 nw = reinterpret_cast<const uint4*>((kv ? new_v : new_k) + i * (kv ? nv_s : nk_s))[w];
      uint4 r;
      r.x = blend_pair(o.x, nw.x, wt, one_minus, bad);
      r.y = blend_pair(o.y, nw.y, wt, one_minus, bad);
      r.z = blend_pair(o.z, nw.z, wt, one_minus, bad);
      r.w = blend_pair(o.w, nw.w, wt, one_minus, bad);
      reinterpret_cast<uint4*>((kv ? fused_v : fused_k) + i * (kv ? fv_s : fk_s))[w] = r;
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

// mean_head_cosine of one bf16 row pair (a_row, b_row: [H, D] contiguous),
// returned on every lane of the wavefront.
__device__ inline double cosine_bf16_row(const uint16_t* a_row, const uint16_t* b_row, int H, int D,
                                         double eps, int lane) {
  const int L = D / 16, per = 64 / L;
  const double tiny = 2.2250738585072014e-308;
  double total = 0.0;
  for (int h0 = 0; h0 < H; h0 += per) {
    const int h = h0 + lane / L;
    const int hc = h < H ? h : H - 1;  // lanes past the last head load it and are ignored
    const int64_t off = static_cast<int64_t>(hc) * D + (lane % L) * 16;
    const uint4* pa = reinterpret_cast<const uint4*>(a_row + off);
    const uint4* pb = reinterpret_cast<const uint4*>(b_row + off);
    const uint4 va[2] = {pa[0], pa[1]}, vb[2] = {pb[0], pb[1]};
    double x[16], y[16];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t wa[4] = {va[q].x, va[q].y, va[q].z, va[q].w};
      const uint32_t wb[4] = {vb[q].x, vb[q].y, vb[q].z, vb[q].w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[8 * q + 2 * r] = bf16_to_float(static_cast<uint16_t>(wa[r]));
        x[8 * q + 2 * r + 1] = bf16_to_float(static_cast<uint16_t>(wa[r] >> 16));
        y[8 * q + 2 * r] = bf16_to_float(static_cast<uint16_t>(wb[r]));
        y[8 * q + 2 * r + 1] = bf16_to_float(static_cast<uint16_t>(wb[r] >> 16));
      }
    }
    double amax = 0.0, bmax = 0.0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      amax = fmax(amax, fabs(x[e]));
      bmax = fmax(bmax, fabs(y[e]));
    }
    for (int o = 1; o < L; o <<= 1) {
      amax = fmax(amax, __shfl_xor(amax, o, 64));
      bmax = fmax(bmax, __shfl_xor(bmax, o, 64));
    }
    const double as = amax > eps ? amax : eps;
    const double bs = bmax > eps ? bmax : eps;
    double na = 0.0, nb = 0.0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const double xs = x[e] / as, ys = y[e] / bs;
      na += xs * xs;
      nb += ys * ys;
    }
    for (int o = 1; o < L; o <<= 1) {
      na += __shfl_xor(na, o, 64);
      nb += __shfl_xor(nb, o, 64);
    }
    na = sqrt(na);
    nb = sqrt(nb);
    const double da = na > tiny ? na : tiny;
    const double db = nb > tiny ? nb : tiny;
    double dot = 0.0;
#pragma unroll
    for (int e = 0; e < 16; ++e) dot += (x[e] / as / da) * (y[e] / bs / db);
    for (int o = 1; o < L; o <<= 1) dot += __shfl_xor(dot, o, 64);
    dot = dot < -1.0 ? -1.0 : (dot > 1.0 ? 1.0 : dot);
    for (int g = 0; g < per; ++g) {
      const double v = __shfl(dot, g * L, 64);
      if (h0 + g < H) total += v;
    }
  }
  return total / static_cast<double>(H);
}

// bf16 fast path of mean_head_cosine: rows with contiguous 16-byte aligned
// [H, D] blocks and D / 16 a power of two.  One wavefront per token; each head
// is held by D / 16 lanes of 16 elements, reduced within those lanes; heads
// are summed in ascending order as in the generic kernel.
__global__ void __launch_bounds__(64 * kWaves) wca_cosine_bf16_kernel(
    const uint16_t* a, int64_t a_s, const uint16_t* b, int64_t b_s, const int64_t* b_rows,
    int64_t n, int H, int D, double eps, double* out) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (i >= n) return;
  const int64_t bi = b_rows ? b_rows[i] : i;
  const double c = cosine_bf16_row(a + i * a_s, b + bi * b_s, H, D, eps, lane);
  if (lane == 0) out[i] = c;
}

// WCAState.initialize masks (wca.py:161-171): candidate = reused & (err > 0);
// counts[0] = #reused, counts[1] = #candidates; flag 32 when a token is neither
// reused nor mandatory.  Single workgroup.
__global__ void __launch_bounds__(kSelThreads) wca_init_masks_kernel(
    const double* err, const uint8_t* reused, const uint8_t* mandatory, int64_t n,
    uint8_t* candidate, int64_t* counts, int32_t* flags) {
  __shared__ int wave_tot[kSelWaves];
  int nr = 0, nc = 0, bad = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kChunk) {
    const int64_t s = c0 + static_cast<int64_t>(threadIdx.x) * kRun;
    if (s >= n) continue;
    const uint32_t r = run_mask(reused, s, n);
    const uint32_t mand = run_mask(mandatory, s, n);
    const uint32_t live = s + kRun <= n ? 0xffffu : (1u << (n - s)) - 1u;
    uint64_t kb[kRun];
    load_key_run(err, s, n, kb);  // err >= 0 or NaN: key_bits > 0 exactly when err > 0
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const double e = __longlong_as_double(kb[j]);
      if (((r >> j) & 1u) && e > 0.0) c |= 1u << j;
    }
    c &= live;
    if (s + kRun <= n && (reinterpret_cast<uintptr_t>(candidate + s) & 15) == 0) {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[q] = ((c >> (4 * q)) & 1u) | (((c >> (4 * q + 1)) & 1u) << 8) |
               (((c >> (4 * q + 2)) & 1u) << 16) | (((c >> (4 * q + 3)) & 1u) << 24);
      *reinterpret_cast<uint4*>(candidate + s) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      for (int j = 0; j < kRun && s + j < n; ++j) candidate[s + j] = (c >> j) & 1u;
    }
    nr += __popc(r);
    nc += __popc(c);
    if (~(r | mand) & live) bad = 1;
  }
  int ex;
  const int tr = block_scan(nr, wave_tot, ex);
  const int tc = block_scan(nc, wave_tot, ex);
  const int tb = block_scan(bad, wave_tot, ex);
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
__device__ void gate_block(
    const double* cosine, const int64_t* rows, const uint8_t* selected, int64_t a,
    int32_t distance, double threshold, int64_t* removed, int64_t* count) {
  __shared__ int wave_tot[kSelWaves];
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < a; c0 += kChunk) {
    const int64_t s = c0 + static_cast<int64_t>(threadIdx.x) * kRun;
    uint32_t f = 0;
    for (int j = 0; j < kRun && s + j < a; ++j) {
      const double metric = distance ? 1.0 - cosine[s + j] : cosine[s + j];
      if (selected[rows[s + j]] && metric < threshold) f |= 1u << j;
    }
    int pos;
    const int tot = block_scan(__popc(f), wave_tot, pos);
    for (; f; f &= f - 1) {
      const int64_t i = s + (__ffs(f) - 1);
      removed[base + pos++] = rows[i];
    }
    base += tot;
  }
  if (threadIdx.x == 0) *count = base;
}

__global__ void __launch_bounds__(kSelThreads) wca_gate_kernel(
    const double* cosine, const int64_t* rows, const uint8_t* selected, int64_t a,
    int32_t distance, double threshold, int64_t* removed, int64_t* count) {
  gate_block(cosine, rows, selected, a, distance, threshold, removed, count);
}

// Commit (wca.py:289-293): alpha[rows[i]] = next[i]; the nrem[0] removed
// tokens (nrem may be null: none) leave the selection and the candidates and
// are marked removed.  Nothing is written when abort_flags has a bit of
// abort_mask set (the update failed a check), which keeps the state unchanged.
__global__ void wca_commit_kernel(double* alpha, const double* next, const int64_t* rows, int64_t a,
                                  const int64_t* removed, const int64_t* nrem, uint8_t* selected,
                                  uint8_t* candidate, uint8_t* removed_mask,
                                  const int32_t* abort_flags, int32_t abort_mask) {
  if (abort_flags && (*abort_flags & abort_mask)) return;
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < a) alpha[rows[i]] = next[i];
  const int64_t r = nrem ? *nrem : 0;
  if (i < r) {
    const int64_t t = removed[i];
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
                             const int64_t* removed, const int64_t* nrem, uint8_t* selected,
                             uint8_t* candidate, uint8_t* removed_mask, const int32_t* abort_flags,
                             int32_t abort_mask, void* stream) {
  if (a == 0) return CS_OK;  // removed tokens are a subset of the active rows
  CS_REQUIRE(alpha && next && rows && selected && candidate && removed_mask, "null arguments");
  CS_REQUIRE(!nrem || removed, "removed list missing");
  hipLaunchKernelGGL(cs::wca_commit_kernel, dim3(cs::ceil_div(a, 256)), dim3(256), 0,
                     cs::as_stream(stream), alpha, next, rows, a, removed, nrem, selected,
                     candidate, removed_mask, abort_flags, abort_mask);
  CS_LAUNCH_CHECK("wca_commit");
  return CS_OK;
}

using namespace cs;

// True when v is a bf16 [n, H, D] view whose [H, D] rows are contiguous with
// 16-byte aligned starts (row stride a multiple of 8 elements).
static bool bf16_rows16(const cs_view* v) {
  return v->dtype == CS_BF16 && v->stride[2] == 1 && v->stride[1] == v->shape[2] &&
         (v->shape[1] * v->shape[2]) % 8 == 0 && v->stride[0] % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(v->data) & 15) == 0;
}

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
  if (bf16_rows16(old_rows_src) && bf16_rows16(fresh)) {
    hipLaunchKernelGGL(wca_score_bf16_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0,
                       as_stream(stream), static_cast<const uint16_t*>(old_rows_src->data),
                       old_rows_src->stride[0], old_rows, static_cast<const uint16_t*>(fresh->data),
                       fresh->stride[0], n, fresh->shape[1] * fresh->shape[2] / 8, err, norm, flags, 0, 0);
  } else {
    hipLaunchKernelGGL(wca_score_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0,
                       as_stream(stream), to_dview(old_rows_src), old_rows, to_dview(fresh), err,
                       norm, flags);
  }
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
                              int64_t* promoted, int64_t* count_out, const int32_t* abort_flags,
                              int32_t abort_mask, void* stream) {
  CS_REQUIRE(key && candidate && removed && selected && scratch && promoted && count_out,
             "null arguments");
  CS_REQUIRE(n >= 0 && n <= (1ll << 24), "at most 2^24 tokens");
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(wca_promote_kernel, dim3(1), dim3(kSelThreads), 0, s, key, candidate, removed,
                     selected, n, budget, scratch, count_out, abort_flags, abort_mask);
  const int64_t kmax = budget < n ? (budget > 0 ? budget : 0) : n;  // bound on the device count
  if (kmax > 0)
    hipLaunchKernelGGL(wca_promote_order_kernel, dim3(ceil_div(kmax, 64)), dim3(64 * kOrderSlices),
                       0, s, scratch, n, count_out, promoted, int64_t(0));
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

namespace cs {
namespace {
// ORs bit into *flags when a[i] != b[i] for some i < n.
__global__ void same_rows_kernel(const int64_t* a, const int64_t* b, int64_t n, int32_t bit, int32_t* flags) {
  bool diff = false;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    diff |= a[i] != b[i];
  if (__any(diff) && (threadIdx.x & 63) == 0) atomicOr(flags, bit);
}
}  // namespace
}  // namespace cs

extern "C" int cs_wca_same_rows(const int64_t* a, const int64_t* b, int64_t n, int32_t bit,
                                int32_t* flags, void* stream) {
  CS_REQUIRE(flags && n >= 0 && (n == 0 || (a && b)), "null arguments");
  if (n == 0) return CS_OK;
  const int64_t blocks = ceil_div(n, 256);
  hipLaunchKernelGGL(same_rows_kernel, dim3(static_cast<unsigned>(blocks < 1024 ? blocks : 1024)), dim3(256), 0,
                     as_stream(stream), a, b, n, bit, flags);
  CS_LAUNCH_CHECK("same_rows");
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
  const bool same_rows = old_k->shape[1] == new_k->shape[1] && old_k->shape[2] == new_k->shape[2] &&
                         old_v->shape[1] == new_k->shape[1] && old_v->shape[2] == new_k->shape[2] &&
                         new_v->shape[1] == new_k->shape[1] && new_v->shape[2] == new_k->shape[2] &&
                         fused_k->shape[1] == new_k->shape[1] && fused_k->shape[2] == new_k->shape[2] &&
                         fused_v->shape[1] == new_k->shape[1] && fused_v->shape[2] == new_k->shape[2];
  if (same_rows && bf16_rows16(old_k) && bf16_rows16(old_v) && bf16_rows16(new_k) &&
      bf16_rows16(new_v) && bf16_rows16(fused_k) && bf16_rows16(fused_v)) {
    const int64_t words = new_k->shape[1] * new_k->shape[2] / 8;
    const int64_t a = new_k->shape[0];
    hipLaunchKernelGGL(wca_blend_bf16_kernel, dim3(grid_for(a * words, 256)), dim3(256), 0,
                       as_stream(stream), static_cast<const uint16_t*>(old_k->data),
                       old_k->stride[0], static_cast<const uint16_t*>(old_v->data),
                       old_v->stride[0], rows, static_cast<const uint16_t*>(new_k->data),
                       new_k->stride[0], static_cast<const uint16_t*>(new_v->data),
                       new_v->stride[0], weight, mandatory, static_cast<uint16_t*>(fused_k->data),
                       fused_k->stride[0], static_cast<uint16_t*>(fused_v->data), fused_v->stride[0],
                       a, words, flags);
    CS_LAUNCH_CHECK("wca_blend");
    return CS_OK;
  }
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
  const int64_t H = a->shape[1], D = a->shape[2];
  const int64_t L = D / 16;
  if (bf16_rows16(a) && bf16_rows16(b) && b->shape[1] == H && b->shape[2] == D && D % 16 == 0 &&
      L >= 1 && L <= 64 && (L & (L - 1)) == 0 && H <= (1 << 20)) {
    hipLaunchKernelGGL(wca_cosine_bf16_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0,
                       as_stream(stream), static_cast<const uint16_t*>(a->data), a->stride[0],
                       static_cast<const uint16_t*>(b->data), b->stride[0], b_rows, n,
                       static_cast<int>(H), static_cast<int>(D), eps, out);
  } else {
    hipLaunchKernelGGL(wca_cosine_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0,
                       as_stream(stream), to_dview(a), to_dview(b), b_rows, eps, out);
  }
  CS_LAUNCH_CHECK("wca_head_cosine");
  return CS_OK;
}

namespace cs {
namespace {
// The checks that open an update, in one launch: the finite checks of four
// contiguous, 16-byte aligned tensors (segments 0..3) and the row-list
// equality (segment 4).  Each workgroup serves one segment; the flag bits are
// those of the separate launches.
struct update_checks {
  const uint4* p[4];
  int64_t words[4];
  int32_t kind[4];
  int32_t bit[4];
  int64_t first[6];  // first workgroup of each segment; first[5] = grid
  const int64_t* ra;
  const int64_t* rb;
  int64_t rn;
};

template <int KIND>
__device__ inline bool words_nonfinite(const uint4* p, int64_t words, int64_t i, int64_t step) {
  bool bad = false;
  for (; i + 3 * step < words; i += 4 * step) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = p[i + u * step];
#pragma unroll
    for (int u = 0; u < 4; ++u) bad |= word_nonfinite<KIND>(v[u]);
  }
  for (; i < words; i += step) bad |= word_nonfinite<KIND>(p[i]);
  return bad;
}

__device__ inline void run_checks(const update_checks& c, int64_t b, int32_t* flags) {
  int seg = 0;
  while (seg < 5 && b >= c.first[seg + 1]) ++seg;
  const int64_t step = (c.first[seg + 1] - c.first[seg]) * 256;
  const int64_t i = (b - c.first[seg]) * 256 + threadIdx.x;
  bool bad = false;
  int32_t bit = 64;
  if (seg < 4) {
    bit = c.bit[seg];
    switch (c.kind[seg]) {
      case 0: bad = words_nonfinite<0>(c.p[seg], c.words[seg], i, step); break;
      case 1: bad = words_nonfinite<1>(c.p[seg], c.words[seg], i, step); break;
      case 2: bad = words_nonfinite<2>(c.p[seg], c.words[seg], i, step); break;
      default: bad = words_nonfinite<3>(c.p[seg], c.words[seg], i, step); break;
    }
  } else {
    for (int64_t j = i; j < c.rn; j += step) bad |= c.ra[j] != c.rb[j];
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flags, bit);
}

__global__ void __launch_bounds__(256) update_checks_kernel(update_checks c, int32_t* flags) {
  run_checks(c, blockIdx.x, flags);
}

// The per-row work of a fused update (bf16 rows, contiguous [H, D] blocks):
// one wavefront per active row i computes what the separate launches compute
// -- the finite checks of recomputed row i, the exact squared deviation and
// norm, the weight, the weight used, the blend of K and V, and on gate layers
// the head cosine -- with the same arithmetic in the same order, so every
// value and flag bit is theirs.
struct update_rows {
  const uint16_t* old_k;
  int64_t ok_s;
  const uint16_t* old_v;
  int64_t ov_s;
  const uint16_t* new_k;
  int64_t nk_s;
  const uint16_t* new_v;
  int64_t nv_s;
  uint16_t* fused_k;
  int64_t fk_s;
  uint16_t* fused_v;
  int64_t fv_s;
  const int64_t* rows;
  int64_t a, words;
  int32_t H, D;
  const double* alpha;
  const uint8_t* mandatory;
  double eps;
  int32_t clamp, previous, gate;
  double *err, *norm, *next, *used, *cosine;
};

__device__ inline void update_row(const update_rows& r, int64_t i, int lane, int32_t* flags) {
  const int64_t row = r.rows[i];
  const uint4* ok = reinterpret_cast<const uint4*>(r.old_k + row * r.ok_s);
  const uint4* nk = reinterpret_cast<const uint4*>(r.new_k + i * r.nk_s);
  // squared deviation and norm (wca_score_bf16_kernel's order), on every lane;
  // the finite checks of the recomputed rows ride on the loads of this pass
  // and of the V blend (the rows are exactly the recomputed tensors' rows)
  score_acc acc;
  bool bad_nk = false, bad_nv = false;
  for (int64_t w = lane; w < r.words; w += 64) {
    const uint4 ov = ok[w], fv = nk[w];
    bad_nk |= word_nonfinite<0>(fv);
    const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w}, fw[4] = {fv.x, fv.y, fv.z, fv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc.add(bf16_to_float(static_cast<uint16_t>(ow[q])), bf16_to_float(static_cast<uint16_t>(fw[q])));
      acc.add(bf16_to_float(static_cast<uint16_t>(ow[q] >> 16)),
              bf16_to_float(static_cast<uint16_t>(fw[q] >> 16)));
    }
  }
  const dd e = dd_wave_sum(acc.e), nn = dd_wave_sum(acc.n);
  const int any_bad = __any(acc.bad);
  double ev = dd_round(e), nv = dd_round(nn);
  if (!isfinite(e.hi)) ev = e.hi != e.hi ? e.hi : INFINITY;
  if (!isfinite(nn.hi)) nv = nn.hi != nn.hi ? nn.hi : INFINITY;
  int f = 0;
  if (any_bad) f |= 1;
  if (!isfinite(ev)) f |= 2;
  if (!isfinite(nv)) f |= 16;
  // weight (wca_alpha_kernel) and the weight used (wca_used_alpha_kernel)
  const double num = ev, den = nv + r.eps;
  if (!isfinite(num) || !isfinite(den)) f |= 2;
  double nxt = num / den;
  if (!isfinite(nxt)) f |= 4;
  if (r.clamp) nxt = nxt < 0.0 ? 0.0 : (nxt > 1.0 ? 1.0 : nxt);
  const double wt = r.mandatory[row] ? 1.0 : (r.previous ? r.alpha[row] : nxt);
  if (lane == 0) {
    r.err[i] = ev;
    r.norm[i] = nv;
    r.next[i] = nxt;
    r.used[i] = wt;
  }
  // blend of K and V (wca_blend_bf16_kernel's arithmetic)
  const double one_minus = 1.0 - wt;
  int bad = 0;
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    const uint4* o = kv ? reinterpret_cast<const uint4*>(r.old_v + row * r.ov_s) : ok;
    const uint4* nw = kv ? reinterpret_cast<const uint4*>(r.new_v + i * r.nv_s) : nk;
    uint4* out = reinterpret_cast<uint4*>(kv ? r.fused_v + i * r.fv_s : r.fused_k + i * r.fk_s);
    for (int64_t w = lane; w < r.words; w += 64) {
      const uint4 ov = o[w], fv = nw[w];
      if (kv) bad_nv |= word_nonfinite<0>(fv);
      uint4 res;
      res.x = blend_pair(ov.x, fv.x, wt, one_minus, bad);
      res.y = blend_pair(ov.y, fv.y, wt, one_minus, bad);
      res.z = blend_pair(ov.z, fv.z, wt, one_minus, bad);
      res.w = blend_pair(ov.w, fv.w, wt, one_minus, bad);
      out[w] = res;
    }
  }
  if (__any(bad)) f |= 8;
  if (__any(bad_nk)) f |= 1 << 21;
  if (__any(bad_nv)) f |= 1 << 23;
  if (r.gate) {
    const double c = cosine_bf16_row(r.new_k + i * r.nk_s, r.old_k + row * r.ok_s, r.H, r.D, r.eps, lane);
    if (lane == 0) r.cosine[i] = c;
  }
  if (lane == 0 && f) atomicOr(flags, f);
}

// Opening checks and the row pass in one launch: the first workgroups serve
// four active rows each (their chains of dependent loads and reductions start
// first), the remaining first[5] workgroups stream the checks behind them.
__global__ void __launch_bounds__(256) update_fused_kernel(update_checks c, update_rows r, int32_t* flags) {
  const int64_t row_blocks = (r.a + 3) / 4;
  const int64_t b = blockIdx.x;
  if (b >= row_blocks) {
    run_checks(c, b - row_blocks, flags);
    return;
  }
  const int64_t i = b * 4 + (threadIdx.x >> 6);
  if (i < r.a) update_row(r, i, threadIdx.x & 63, flags);
}

// The rest of a fused update in one workgroup: the gate's removed rows, the
// commit (skipped when a registered check fired), the promotion's selection
// and the next active rows -- the bodies of the separate launches, in their
// order.
// The status of an update for the host: the flags word and the three counts,
// written by the thread that wrote the counts (after them, in its program
// order), as plain stores into host-visible memory.  With clear set the same
// thread then zeroes the status block for the next call (every other write
// to it in this call is ordered before: the flags' atomics by the kernel
// boundary, the counts by the thread's own program order).
__device__ inline void write_report(int64_t* report, int32_t* flags, int64_t* counts, bool clear) {
  report[0] = static_cast<int64_t>(static_cast<uint32_t>(*flags));
  report[1] = counts[0];
  report[2] = counts[1];
  report[3] = counts[2];
  if (clear) {
    *flags = 0;
    counts[0] = 0;
    counts[1] = 0;
    counts[2] = 0;
  }
}

__global__ void status_clear_kernel(int32_t* flags, int64_t* counts) {
  if (threadIdx.x == 0) *flags = 0;
  if (threadIdx.x < 3) counts[threadIdx.x] = 0;
}

__global__ void status_report_kernel(int64_t* report, int32_t* flags, int64_t* counts, int32_t clear) {
  if (threadIdx.x == 0) write_report(report, flags, counts, clear != 0);
}

// The status of a one-call initialize: the flags word and five counts.
__global__ void init_status_clear_kernel(int32_t* flags, int64_t* counts) {
  if (threadIdx.x == 0) *flags = 0;
  if (threadIdx.x < 5) counts[threadIdx.x] = 0;
}

// ... written into the caller's report word, after which the block is
// zeroed for the next call (every other write to it is ordered before).
__global__ void init_status_report_kernel(int64_t* report, int32_t* flags, int64_t* counts) {
  if (threadIdx.x == 0) {
    report[0] = static_cast<int64_t>(static_cast<uint32_t>(*flags));
    for (int i = 0; i < 5; ++i) report[1 + i] = counts[i];
    *flags = 0;
    for (int i = 0; i < 5; ++i) counts[i] = 0;
  }
}

// The promotion of WCAState.initialize with its budget taken on the device
// from the mask counts (wca.py:177-180): min(ceil(fraction * reused),
// candidates), written to counts[2]; the promoted count goes to counts[3].
__global__ void __launch_bounds__(kSelThreads) wca_initial_promote_kernel(
    const double* key, const uint8_t* candidate, const uint8_t* removed, uint8_t* selected, int64_t n,
    int64_t* counts, double fraction, int64_t* scratch, const int32_t* abort_flags, int32_t abort_mask) {
  int64_t budget = static_cast<int64_t>(ceil(fraction * static_cast<double>(counts[0])));
  if (budget > counts[1]) budget = counts[1];
  if (threadIdx.x == 0) counts[2] = budget;
  promote_block(key, candidate, removed, selected, n, budget, scratch, counts + 3, abort_flags, abort_mask);
}

struct update_final {
  double* alpha;
  const double* next;
  const int64_t* rows;
  int64_t a;
  const double* cosine;
  uint8_t *selected, *candidate, *removed_mask;
  const uint8_t* mandatory;
  const double* deviation;
  int64_t n, budget;
  int64_t* scratch;
  int64_t *removed, *active, *counts;
  int64_t* promoted;  // the small finish orders promotions of up to kRankMax tokens here
  int64_t* report;    // NULL, or host-visible {flags word, counts[0..2]}
  int32_t gate, distance;
  double threshold;
  int32_t* flags;
  int32_t abort_mask;
  int32_t clear_after;  // zero the status block once the report is written
};

__global__ void __launch_bounds__(kSelThreads) update_finalize_kernel(update_final f) {
  const int tid = threadIdx.x;
  if (f.gate)
    gate_block(f.cosine, f.rows, f.selected, f.a, f.distance, f.threshold, f.removed, f.counts);
  else if (tid == 0)
    f.counts[0] = 0;
  __syncthreads();
  if (!(*f.flags & f.abort_mask)) {
    for (int64_t i = tid; i < f.a; i += kSelThreads) f.alpha[f.rows[i]] = f.next[i];
    const int64_t nrem = f.gate ? f.counts[0] : 0;
    for (int64_t i = tid; i < nrem; i += kSelThreads) {
      const int64_t t = f.removed[i];
      f.selected[t] = 0;
      f.candidate[t] = 0;
      f.removed_mask[t] = 1;
    }
  }
  __syncthreads();
  promote_block(f.deviation, f.candidate, f.removed_mask, f.selected, f.n, f.budget, f.scratch,
                f.counts + 1, f.flags, f.abort_mask);
  __syncthreads();
  nonzero_block(f.selected, f.mandatory, f.n, f.active, f.counts + 2);
  if (threadIdx.x == 0 && f.report) write_report(f.report, f.flags, f.counts, f.clear_after != 0);
}

// Stores the 16 bits of a run as bytes 0 / 1 (run_mask's inverse).
__device__ inline void store_run_mask(uint8_t* p, int64_t start, int64_t n, uint32_t m) {
  if (start + kRun <= n && (reinterpret_cast<uintptr_t>(p + start) & 15) == 0) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t x = (m >> (4 * q)) & 0xFu;
      w[q] = (x & 1u) | ((x & 2u) << 7) | ((x & 4u) << 14) | ((x & 8u) << 21);
    }
    *reinterpret_cast<uint4*>(p + start) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    for (int j = 0; j < kRun; ++j)
      if (start + j < n) p[start + j] = static_cast<uint8_t>((m >> j) & 1u);
  }
}

constexpr int kRankMax = 4096;  // promotions the small finish orders itself

// update_finalize_kernel for a request of at most one chunk (n <= kChunk
// tokens).  Thread t owns tokens [16 t, 16 t + 16) and holds their selected,
// candidate, removed and mandatory bits in registers, loaded once at the
// start with the flags; the gate reads the selected bits from LDS, removals
// reach the owning thread through LDS, and the promotion's radix select runs
// on keys held in registers.  The phases, their order and every result are
// those of update_finalize_kernel (gate_block, commit, promote_block,
// nonzero_block); the three masks are stored once at the end.
__global__ void __launch_bounds__(kSelThreads) update_finalize_small_kernel(update_final f) {
  __shared__ uint32_t sel_run[kSelThreads];
  __shared__ uint32_t rm_run[kSelThreads];
  __shared__ int wave_tot[kSelWaves];
  __shared__ int64_t wave_tot64[kSelWaves];
  __shared__ int hist[256];
  __shared__ uint64_t wred[2 * kSelWaves];
  __shared__ uint64_t s_prefix, s_mask;
  __shared__ int64_t s_remaining;
  __shared__ int s_done, s_start;
  __shared__ uint64_t p_key[kRankMax];  // promoted tokens in index order and their key bits
  __shared__ int32_t p_tok[kRankMax];
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t n = f.n, a = f.a;
  const int64_t s = static_cast<int64_t>(tid) * kRun;
  uint32_t sel = run_mask(f.selected, s, n);
  uint32_t cand = run_mask(f.candidate, s, n);
  uint32_t remm = run_mask(f.removed_mask, s, n);
  const uint32_t mand = f.mandatory ? run_mask(f.mandatory, s, n) : 0u;
  const bool abort = (*f.flags & f.abort_mask) != 0;
  // commit of the next weights (nothing below reads alpha): the first
  // 4 * kSelThreads entries are loaded with the masks and stored before the
  // gate on gate layers, else after the counting scan, so that without a
  // gate or a promotion no barrier waits for their stores; entries past
  // them are committed here
  int64_t r4[4];
  double n4[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = u * kSelThreads + tid;
    r4[u] = i < a ? f.rows[i] : -1;
    n4[u] = i < a ? f.next[i] : 0.0;
  }
  for (int64_t i0 = 4 * kSelThreads; i0 < a; i0 += 4 * kSelThreads) {
    int64_t rr[4];
    double nr[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = i0 + u * kSelThreads + tid;
      rr[u] = i < a ? f.rows[i] : -1;
      nr[u] = i < a ? f.next[i] : 0.0;
    }
    if (!abort) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (rr[u] >= 0) f.alpha[rr[u]] = nr[u];
    }
  }

  // gate (gate_block): the selected rows whose metric is below the threshold
  int64_t nrem = 0;
  if (f.gate) {
    if (!abort) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (r4[u] >= 0) f.alpha[r4[u]] = n4[u];
    }
    sel_run[tid] = sel;
    rm_run[tid] = 0;
    __syncthreads();
    for (int64_t c0 = 0; c0 < a; c0 += kChunk) {
      const int64_t s2 = c0 + s;
      uint32_t fl = 0;
#pragma unroll
      for (int j = 0; j < kRun; ++j) {
        if (s2 + j < a) {
          const int64_t t = f.rows[s2 + j];
          const double metric = f.distance ? 1.0 - f.cosine[s2 + j] : f.cosine[s2 + j];
          if (((sel_run[t >> 4] >> (t & 15)) & 1u) && metric < f.threshold) fl |= 1u << j;
        }
      }
      int pos;
      const int tot = block_scan(__popc(fl), wave_tot, pos);
      for (; fl; fl &= fl - 1) {
        const int64_t t = f.rows[s2 + (__ffs(fl) - 1)];
        f.removed[nrem + pos++] = t;
        if (!abort) atomicOr(&rm_run[t >> 4], 1u << (t & 15));
      }
      nrem += tot;
    }
    __syncthreads();
    if (!abort) {
      const uint32_t r = rm_run[tid];
      sel &= ~r;
      cand &= ~r;
      remm |= r;
    }
  }
  if (tid == 0) f.counts[0] = nrem;

  // promotion (promote_block, one chunk): slots = max(0, budget - #selected),
  // available = candidate & ~selected & ~removed, the k largest keys taken
  // one scan for three counts in 16-bit fields (each total is at most
  // kChunk = 2^14): selected, available, and selected | mandatory -- the
  // next active rows' positions when nothing gets promoted
  const uint32_t av = cand & ~sel & ~remm;
  int64_t ex;
  const int64_t packed = block_scan64(static_cast<int64_t>(__popc(sel)) |
                                          (static_cast<int64_t>(__popc(av)) << 16) |
                                          (static_cast<int64_t>(__popc(sel | mand)) << 32),
                                      wave_tot64, ex);
  const int total_sel = static_cast<int>(packed & 0xffff);
  const int total_av = static_cast<int>((packed >> 16) & 0xffff);
  int64_t slots = f.budget - total_sel;
  if (slots < 0) slots = 0;
  // the same on every lane (at most kChunk); read from one lane so the
  // branches below are uniform and their values do not stay live across
  // each other
  const int64_t k = __builtin_amdgcn_readfirstlane(
      static_cast<int>(abort ? 0 : (slots < total_av ? slots : total_av)));
  if (tid == 0) f.counts[1] = k;
  if (!abort && !f.gate) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (r4[u] >= 0) f.alpha[r4[u]] = n4[u];
  }
  int nz_pos, nz_tot;  // positions of the next active rows
  if (k > 0) {
    if (tid == 0) {
      s_prefix = 0;
      s_mask = 0;
      s_remaining = k;
      s_done = k == total_av;
    }
    __syncthreads();
    uint64_t kb[kRun] = {};
    if (s < n) load_key_run(f.deviation, s, n, kb);
    radix_select_regs(kb, av, hist, wred, s_prefix, s_mask, s_remaining, s_done, s_start);
    const uint64_t thr = s_prefix, mask = s_mask;
    const int64_t need_eq = s_remaining;
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const uint64_t km = kb[j] & mask;
      if (((av >> j) & 1u) && km > thr) gt |= 1u << j;
      if (((av >> j) & 1u) && km == thr) eq |= 1u << j;
    }
    int eq_rank;
    block_scan(__popc(eq), wave_tot, eq_rank);
    uint32_t take = gt;
    for (uint32_t m = eq; m; m &= m - 1) {
      if (eq_rank < need_eq) take |= m & (~m + 1);
      ++eq_rank;
    }
    int pos;
    block_scan(__popc(take), wave_tot, pos);
    for (uint32_t m = take; m; m &= m - 1) {
      const int j = __ffs(m) - 1;
      f.scratch[pos] = s + j;
      f.scratch[n + pos] = static_cast<int64_t>(kb[j]);
      if (pos < kRankMax) {
        p_tok[pos] = static_cast<int32_t>(s + j);
        p_key[pos] = kb[j];
      }
      ++pos;
    }
    sel |= take;
    // order of the promotions (wca_promote_order_kernel's rank: key
    // descending, index ascending) when they fit the LDS lists
    __syncthreads();
    if (k <= kRankMax) {
      for (int e = tid; e < k; e += kSelThreads) {
        const uint64_t ke = p_key[e];
        int rank = 0;
        for (int j = 0; j < k; ++j) {
          const uint64_t kj = p_key[j];
          rank += (kj > ke) || (kj == ke && j < e);
        }
        f.promoted[rank] = p_tok[e];
      }
    }
    nz_tot = block_scan(__popc(sel | mand), wave_tot, nz_pos);
  } else {
    nz_pos = static_cast<int>(ex >> 32);
    nz_tot = static_cast<int>(packed >> 32);
  }

  // next active rows (nonzero_block): ascending tokens of selected | mandatory
  {
    int pos = nz_pos;
    for (uint32_t m = sel | mand; m; m &= m - 1) f.active[pos++] = s + (__ffs(m) - 1);
    if (tid == 0) f.counts[2] = nz_tot;
  }
  if (s < n) {
    store_run_mask(f.selected, s, n, sel);
    store_run_mask(f.candidate, s, n, cand);
    store_run_mask(f.removed_mask, s, n, remm);
  }
  if (tid == 0 && f.report) write_report(f.report, f.flags, f.counts, f.clear_after != 0);
}

// Fills one check segment when v is contiguous, 16-byte aligned and floating;
// false leaves the separate launch to the caller.  An absent or empty view
// takes no workgroups.
bool check_segment(const cs_view* v, int32_t bit, update_checks& c, int seg, int64_t& blocks) {
  c.p[seg] = nullptr;
  c.words[seg] = 0;
  c.bit[seg] = bit;
  c.kind[seg] = 0;
  c.first[seg] = blocks;
  if (!v->data) return true;
  int64_t numel = 1, expect = 1;
  bool contiguous = true;
  for (int d = 0; d < v->ndim; ++d) numel *= v->shape[d];
  for (int d = v->ndim - 1; d >= 0; --d) {
    if (v->shape[d] != 1 && v->stride[d] != expect) contiguous = false;
    expect *= v->shape[d];
  }
  if (numel == 0) return true;
  const int64_t bytes = numel * dtype_size(v->dtype);
  if (!is_float_dtype(v->dtype) || !contiguous || (reinterpret_cast<uintptr_t>(v->data) & 15) || bytes % 16)
    return false;
  c.p[seg] = static_cast<const uint4*>(v->data);
  c.words[seg] = bytes / 16;
  c.kind[seg] = v->dtype == CS_BF16 ? 0 : v->dtype == CS_F16 ? 1 : v->dtype == CS_F32 ? 2 : 3;
  blocks += std::min<int64_t>(ceil_div(c.words[seg], 256 * 8), 4096);
  return true;
}
}  // namespace
}  // namespace cs

namespace cs {
namespace {
// The fused update applies to bf16 K/V with contiguous, 16-byte aligned
// [H, D] rows (D a multiple of 16 with D / 16 a power of two) whose finite
// checks fit the single opening launch.
bool fused_update_ok(const cs_wca_update_args* u) {
  const cs_view* v[6] = {&u->cached_k, &u->cached_v, &u->recomputed_k, &u->recomputed_v, &u->fused_k,
                         &u->fused_v};
  for (const cs_view* x : v) {
    if (!x->data || x->ndim != 3 || !bf16_rows16(x)) return false;
    if (x->shape[1] != u->cached_k.shape[1] || x->shape[2] != u->cached_k.shape[2]) return false;
  }
  const int64_t D = u->cached_k.shape[2], L = D / 16;
  return u->rows && u->a > 0 && u->recomputed_k.shape[0] == u->a && D % 16 == 0 && L >= 1 && L <= 64 &&
         (L & (L - 1)) == 0 && u->cached_k.shape[1] <= (1 << 20) && u->n <= (1ll << 24);
}
}  // namespace
}  // namespace cs

extern "C" int cs_wca_update(const cs_wca_update_args* u, void* stream) {
  CS_REQUIRE(u && u->flags && u->counts, "null arguments");
  CS_REQUIRE(u->a >= 0 && (!u->computed || u->a == 0 || u->rows), "null arguments");
  CS_REQUIRE(!(u->clear_status & 2) || u->report, "clearing the status at the end needs a report");
  int32_t* f = u->flags;
  int st;
  if (u->clear_status & 1) {
    hipLaunchKernelGGL(status_clear_kernel, dim3(1), dim3(64), 0, as_stream(stream), f, u->counts);
    CS_LAUNCH_CHECK("wca_update status");
  }
#define CS_STEP(expr) \
  do {                \
    st = (expr);      \
    if (st != CS_OK) return st; \
  } while (0)
  update_checks c{};
  int64_t blocks = 0;
  const bool rows_fused = fused_update_ok(u);
  bool fused = check_segment(&u->cached_k, 1 << 20, c, 0, blocks) &&
               check_segment(&u->cached_v, 1 << 22, c, 1, blocks);
  if (fused && rows_fused) {
    // the row pass checks the recomputed rows as it reads them (update_row)
    const cs_view none{};
    check_segment(&none, 1 << 21, c, 2, blocks);
    check_segment(&none, 1 << 23, c, 3, blocks);
  } else {
    fused = fused && check_segment(&u->recomputed_k, 1 << 21, c, 2, blocks) &&
            check_segment(&u->recomputed_v, 1 << 23, c, 3, blocks);
  }
  if (fused) {
    c.first[4] = blocks;
    if (u->computed && u->a > 0) {
      c.ra = u->computed;
      c.rb = u->rows;
      c.rn = u->a;
      blocks += std::min<int64_t>(ceil_div(u->a, 256), 1024);
    }
    c.first[5] = blocks;
  }
  if (fused && rows_fused) {
    // three launches: checks + rows, the one-workgroup finish, the promotion order
    update_rows r{};
    r.old_k = static_cast<const uint16_t*>(u->cached_k.data);
    r.ok_s = u->cached_k.stride[0];
    r.old_v = static_cast<const uint16_t*>(u->cached_v.data);
    r.ov_s = u->cached_v.stride[0];
    r.new_k = static_cast<const uint16_t*>(u->recomputed_k.data);
    r.nk_s = u->recomputed_k.stride[0];
    r.new_v = static_cast<const uint16_t*>(u->recomputed_v.data);
    r.nv_s = u->recomputed_v.stride[0];
    r.fused_k = static_cast<uint16_t*>(u->fused_k.data);
    r.fk_s = u->fused_k.stride[0];
    r.fused_v = static_cast<uint16_t*>(u->fused_v.data);
    r.fv_s = u->fused_v.stride[0];
    r.rows = u->rows;
    r.a = u->a;
    r.H = static_cast<int32_t>(u->cached_k.shape[1]);
    r.D = static_cast<int32_t>(u->cached_k.shape[2]);
    r.words = static_cast<int64_t>(r.H) * r.D / 8;
    r.alpha = u->alpha;
    r.mandatory = u->mandatory;
    r.eps = u->epsilon;
    r.clamp = u->clamp;
    r.previous = u->previous_layer;
    r.gate = u->gate;
    r.err = u->err;
    r.norm = u->norm;
    r.next = u->next_alpha;
    r.used = u->used;
    r.cosine = u->cosine;
    const int64_t grid = blocks + ceil_div(u->a, 4);
    CS_REQUIRE(grid < (1ll << 31), "grid too large");
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(update_fused_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, c, r, f);
    update_final fin{};
    fin.alpha = u->alpha;
    fin.next = u->next_alpha;
    fin.rows = u->rows;
    fin.a = u->a;
    fin.cosine = u->cosine;
    fin.selected = u->selected;
    fin.candidate = u->candidate;
    fin.removed_mask = u->removed_mask;
    fin.mandatory = u->mandatory;
    fin.deviation = u->deviation;
    fin.n = u->n;
    fin.budget = u->budget;
    fin.scratch = u->scratch;
    fin.removed = u->removed;
    fin.active = u->active;
    fin.counts = u->counts;
    fin.gate = u->gate;
    fin.distance = u->distance_mode;
    fin.threshold = u->threshold;
    fin.flags = f;
    fin.abort_mask = u->abort_mask;
    fin.promoted = u->promoted;
    fin.report = u->report;
    const bool small = u->n <= kChunk;
    // promotions beyond what the small finish orders get their own launch
    // (kmax bounds the device count); it reads counts[1], so the status is
    // then cleared by a launch of its own behind it
    const int64_t kmax = u->budget < u->n ? (u->budget > 0 ? u->budget : 0) : u->n;
    const int64_t done = small ? kRankMax : 0;
    const bool order = kmax > done;
    fin.clear_after = (u->clear_status & 2) && !order;
    if (small)
      hipLaunchKernelGGL(update_finalize_small_kernel, dim3(1), dim3(kSelThreads), 0, s, fin);
    else
      hipLaunchKernelGGL(update_finalize_kernel, dim3(1), dim3(kSelThreads), 0, s, fin);
    if (order) {
      hipLaunchKernelGGL(wca_promote_order_kernel, dim3(ceil_div(kmax, 64)), dim3(64 * kOrderSlices), 0,
                         s, u->scratch, u->n, u->counts + 1, u->promoted, done);
      if (u->clear_status & 2) hipLaunchKernelGGL(status_clear_kernel, dim3(1), dim3(64), 0, s, f, u->counts);
    }
    CS_LAUNCH_CHECK("wca_update");
    return CS_OK;
  }
  if (fused) {
    if (blocks > 0) {
      hipLaunchKernelGGL(update_checks_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                         as_stream(stream), c, f);
      CS_LAUNCH_CHECK("update_checks");
    }
  } else {
    CS_STEP(cs_check_finite(&u->cached_k, 1 << 20, f, stream));
    CS_STEP(cs_check_finite(&u->cached_v, 1 << 22, f, stream));
    if (u->computed) CS_STEP(cs_wca_same_rows(u->computed, u->rows, u->a, 64, f, stream));
    CS_STEP(cs_check_finite(&u->recomputed_k, 1 << 21, f, stream));
    CS_STEP(cs_check_finite(&u->recomputed_v, 1 << 23, f, stream));
  }
  CS_STEP(cs_wca_score(&u->cached_k, u->rows, &u->recomputed_k, u->err, u->norm, f, stream));
  CS_STEP(cs_wca_alpha(u->err, u->norm, u->a, u->epsilon, u->clamp, u->next_alpha, f, stream));
  CS_STEP(cs_wca_used_alpha(u->alpha, u->next_alpha, u->rows, u->mandatory, u->a, u->previous_layer,
                            u->used, stream));
  cs_view fk = u->fused_k, fv = u->fused_v;
  CS_STEP(cs_wca_blend(&u->cached_k, &u->cached_v, u->rows, &u->recomputed_k, &u->recomputed_v, u->used,
                       nullptr, &fk, &fv, f, stream));
  if (u->gate) {
    CS_STEP(cs_wca_head_cosine(&u->recomputed_k, &u->cached_k, u->rows, u->epsilon, u->cosine, stream));
    CS_STEP(cs_wca_gate(u->cosine, u->rows, u->selected, u->a, u->distance_mode, u->threshold, u->removed,
                        u->counts, stream));
  }
  CS_STEP(cs_wca_commit(u->alpha, u->next_alpha, u->rows, u->a, u->gate ? u->removed : nullptr,
                        u->gate ? u->counts : nullptr, u->selected, u->candidate, u->removed_mask, f,
                        u->abort_mask, stream));
  CS_STEP(cs_wca_promote(u->deviation, u->candidate, u->removed_mask, u->selected, u->n, u->budget,
                         u->scratch, u->promoted, u->counts + 1, f, u->abort_mask, stream));
  CS_STEP(cs_mask_nonzero(u->selected, u->mandatory, u->n, u->active, u->counts + 2, stream));
#undef CS_STEP
  if (u->report) {
    hipLaunchKernelGGL(status_report_kernel, dim3(1), dim3(64), 0, as_stream(stream), u->report, f, u->counts,
                       u->clear_status & 2);
    CS_LAUNCH_CHECK("wca_update report");
  }
  return CS_OK;
}

extern "C" int cs_wca_initialize(const cs_wca_initialize_args* a, void* stream) {
  CS_REQUIRE(a && a->flags && a->counts && a->report, "null arguments");
  const int64_t n = a->n;
  CS_REQUIRE(n >= 0 && n <= (1ll << 24), "at most 2^24 tokens");
  CS_REQUIRE(n == 0 || (a->reused && a->mandatory && a->err && a->norm && a->alpha && a->candidate &&
                        a->selected && a->removed && a->scratch && a->promoted && a->active),
             "null arguments");
  CS_REQUIRE(a->cached_k.ndim == 3 && a->recomputed_k.ndim == 3 && a->cached_k.shape[0] == n &&
                 a->recomputed_k.shape[0] == n,
             "K views must be [n, H, D]");
  hipStream_t s = as_stream(stream);
  int32_t* f = a->flags;
  int st;
  if (a->clear_status & 1) {
    hipLaunchKernelGGL(init_status_clear_kernel, dim3(1), dim3(64), 0, s, f, a->counts);
    CS_LAUNCH_CHECK("wca_initialize status");
  }
#define CS_STEP(expr) \
  do {                \
    st = (expr);      \
    if (st != CS_OK) return st; \
  } while (0)
  const cs_view& ck = a->cached_k;
  const cs_view& rk = a->recomputed_k;
  if (bf16_rows16(&ck) && bf16_rows16(&rk) && ck.shape[1] == rk.shape[1] && ck.shape[2] == rk.shape[2]) {
    // the score reads every row of both: the finite checks ride on its loads
    if (n > 0) {
      hipLaunchKernelGGL(wca_score_bf16_kernel, dim3(ceil_div(n, kWaves)), dim3(64 * kWaves), 0, s,
                         static_cast<const uint16_t*>(ck.data), ck.stride[0], nullptr,
                         static_cast<const uint16_t*>(rk.data), rk.stride[0], n, rk.shape[1] * rk.shape[2] / 8,
                         a->err, a->norm, f, 1 << 20, 1 << 21);
      CS_LAUNCH_CHECK("wca_initialize score");
    }
  } else {
    CS_STEP(cs_check_finite(&ck, 1 << 20, f, stream));
    CS_STEP(cs_check_finite(&rk, 1 << 21, f, stream));
    CS_STEP(cs_wca_score(&ck, nullptr, &rk, a->err, a->norm, f, stream));
  }
  CS_STEP(cs_wca_init_masks(a->err, a->reused, a->mandatory, n, a->candidate, a->counts, f, stream));
  CS_STEP(cs_wca_alpha(a->err, a->norm, n, a->epsilon, a->clamp, a->alpha, f, stream));
  if (n > 0) {
    const int32_t abort = (1 << 20) | (1 << 21) | 2 | 4 | 16 | 32;
    hipLaunchKernelGGL(wca_initial_promote_kernel, dim3(1), dim3(kSelThreads), 0, s, a->err, a->candidate,
                       a->removed, a->selected, n, a->counts, a->fraction, a->scratch, f, abort);
    // the budget is on the device: n bounds the promoted count
    hipLaunchKernelGGL(wca_promote_order_kernel, dim3(ceil_div(n, 64)), dim3(64 * kOrderSlices), 0, s, a->scratch,
                       n, a->counts + 3, a->promoted, int64_t(0));
    CS_LAUNCH_CHECK("wca_initialize promote");
  }
  CS_STEP(cs_mask_nonzero(a->selected, a->mandatory, n, a->active, a->counts + 4, stream));
#undef CS_STEP
  hipLaunchKernelGGL(init_status_report_kernel, dim3(1), dim3(64), 0, s, a->report, f, a->counts);
  CS_LAUNCH_CHECK("wca_initialize report");
  return CS_OK;
}
