// CCPE (contextual position encoding) attention with the full reference
// semantics, for any float dtype and head size, plus the input checks and the
// stand-alone position/validation kernels.
//
// Reference: src/cacheslide_vllm/position.py
//   _logits            :157-164   logits = (q . k) / sqrt(D), accumulation dtype
//   _allowed           :167-193   causal key_pos <= query_pos AND attention_mask
//   contextual_positions :295-307 gates = sigmoid(masked logits); reverse cumsum
//                                 over all keys; clamp(0, P-1)
//   positional_bias    :309-344   lerp of (q . E)[floor p] and [min(floor p+1, P-1)]
//   cope_attention     :404-560   bias added to logits, visibility after gates,
//                                 masked softmax, rows with no visible key -> 0
//   validate_contextual_path :28-114 structural path checks
// and src/cacheslide_vllm/attention.py:18-72 (the two policies, lowered to data).
//
// One wavefront owns one (query row, query head) pair and walks the keys in
// 64-key tiles from the last causal key leftwards, so the reverse cumulative
// gate sum is a carried suffix plus an in-tile suffix scan.  The scan and the
// carry are accumulated in fp64 and each position is rounded once to the
// position dtype, which is what torch's CPU cumsum does for fp32 inputs.

#include "common.h"
#include "ccpe_path.h"

namespace cs {
namespace {

constexpr int kGenWaves = 2;
constexpr int kMaxDvChunks = 8;  // Dv <= 512

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct mask3 {  // uint8 [Hm, nq, nk] (head stride 0 when broadcast)
  const uint8_t* data;
  int64_t sh, sq, sk;
  __device__ bool get(int64_t h, int64_t r, int64_t j) const {
    return data == nullptr || data[h * sh + r * sq + j * sk] != 0;
  }
};

struct gen_params {
  const void* q;
  int64_t q_s0, q_s1, q_s2;
  const void* k;
  int64_t k_s0, k_s1, k_s2;
  const void* v;
  int64_t v_s0, v_s1, v_s2;
  const void* e;
  int32_t e_dtype;
  int64_t e_s0, e_s1;
  int64_t nq, nk, hq, hkv, d, dv, npos;
  const int64_t* qpos;
  const int64_t* kpos;
  mask3 amask, vmask;
  const uint8_t* sel_rows;
  const uint8_t* fixed_keys;
  const void* fixed;
  int32_t fixed_dtype;
  int64_t f_s0, f_s1, f_s2;
  const void* canon;
  int32_t canon_dtype;
  int64_t c_s0, c_s1, c_s2;
  const int64_t* q_ord;
  const int64_t* k_ord;
  int32_t strict;
  int32_t chunk_rows;
  int32_t* chunk_flags;
  void* out;
  int64_t o_s0, o_s1, o_s2;
  void* pos_out;
  int32_t pos_dtype;
  int64_t p_s0, p_s1, p_s2;
  int32_t* flags;
  int64_t wave_bytes;  // LDS bytes per wave
  int64_t p_pad;
};

template <typename Acc>
__device__ inline Acc sigmoid_of(Acc x) {
  return Acc(1) / (Acc(1) + exp(-x));
}

// bias = low + frac * (high - low) with frac = p - floor(p) (position.py:339-344).
template <typename Acc>
__device__ inline Acc lerp_bias(const Acc* qe, double p, int64_t npos, bool* bad) {
  if (!(p >= 0.0) || !(p <= static_cast<double>(npos - 1))) {  // also NaN
    *bad = true;
    p = p >= 0.0 ? (p <= static_cast<double>(npos - 1) ? p : static_cast<double>(npos - 1)) : 0.0;
  }
  double fl = floor(p);
  int64_t lo = static_cast<int64_t>(fl);
  int64_t hi = lo + 1 < npos - 1 ? lo + 1 : npos - 1;
  Acc frac = static_cast<Acc>(p - fl);
  Acc low = qe[lo];
  Acc high = qe[hi];
  Acc delta = high - low;
  Acc scaled = frac * delta;
  return low + scaled;
}

template <typename T>
__global__ void __launch_bounds__(64 * kGenWaves) ccpe_generic_kernel(gen_params g) {
  using E = elem<T>;
  using Acc = typename E::acc;
  using S = typename E::storage;
  using TP = Acc;  // contextual positions live in the accumulation dtype
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * kGenWaves + wave;
  if (pair >= g.nq * g.hq) return;  // wave-uniform; no workgroup barriers below
  const int64_t row = pair / g.hq;
  const int64_t h = pair % g.hq;
  const int64_t kvh = h / (g.hq / g.hkv);
  Acc* qs = reinterpret_cast<Acc*>(smem_raw + wave * g.wave_bytes);
  Acc* qe = qs + g.d;
  Acc* pr = qe + g.p_pad;

  const S* q = static_cast<const S*>(g.q);
  const S* kk = static_cast<const S*>(g.k);
  const S* vv = static_cast<const S*>(g.v);
  int local_flags = 0;

  for (int64_t d = lane; d < g.d; d += 64) qs[d] = E::load(q, row * g.q_s0 + h * g.q_s1 + d * g.q_s2);
  wave_sync();
  for (int64_t pp = lane; pp < g.npos; pp += 64) {
    Acc acc = 0;
    for (int64_t d = 0; d < g.d; ++d)
      acc += qs[d] * static_cast<Acc>(load_as_double(g.e, g.e_dtype, d * g.e_s0 + pp * g.e_s1));
    qe[pp] = acc;
  }
  wave_sync();

  const int64_t qp = g.qpos[row];
  // Number of causal keys: key positions are strictly increasing (checked
  // separately), so the causal keys form a prefix.
  int64_t lo = 0, hi = g.nk;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (g.kpos[mid] <= qp) lo = mid + 1; else hi = mid;
  }
  const int64_t kend = lo;

  const bool contextual = g.fixed == nullptr;
  const int64_t qo = (g.canon && g.q_ord) ? g.q_ord[row] : -1;
  const bool sel_row = g.sel_rows ? g.sel_rows[row] != 0 : false;
  const Acc inv_sqrt = Acc(1);
  const Acc sqrt_d = static_cast<Acc>(sqrt(static_cast<double>(g.d)));
  (void)inv_sqrt;
  const TP atol = static_cast<TP>(1e-6);

  double carry = 0.0;
  Acc m = -INFINITY, l = 0;
  Acc o[kMaxDvChunks];
#pragma unroll
  for (int i = 0; i < kMaxDvChunks; ++i) o[i] = 0;
  const int ndv = static_cast<int>((g.dv + 63) / 64);

  TP prev_p = 0;
  bool prev_valid = false;
  int64_t prev_kp = 0;
  int path_bits = 0;
  bool bad_pos = false;

  const int64_t ntiles = (kend + 63) / 64;
  for (int64_t t = ntiles - 1; t >= 0; --t) {
    const int64_t j = t * 64 + lane;
    const bool causal = j < kend;
    const int64_t kp = causal ? g.kpos[j] : 0;
    const bool allowed = causal && g.amask.get(h, row, j);
    Acc logit = 0;
    if (causal) {
      Acc dot = 0;
      const int64_t kb = j * g.k_s0 + kvh * g.k_s1;
      for (int64_t d = 0; d < g.d; ++d) dot += qs[d] * E::load(kk, kb + d * g.k_s2);
      logit = dot / sqrt_d;
      if (!isfinite(logit)) local_flags |= CS_FLAG_LOGIT_NONFINITE;
    }
    double gate = allowed ? static_cast<double>(sigmoid_of<Acc>(logit)) : 0.0;
    // inclusive suffix scan across lanes (right to left)
    double s = gate;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      double nb = __shfl_down(s, off, 64);
      if (lane + off < 64) s += nb;
    }
    const double tile_total = __shfl(s, 0, 64);
    double p;
    if (contextual) {
      TP pc = static_cast<TP>(carry + s);
      if (pc < TP(0)) pc = TP(0);
      if (pc > static_cast<TP>(g.npos - 1)) pc = static_cast<TP>(g.npos - 1);
      p = static_cast<double>(pc);
      if (qo >= 0 && causal) {
        int64_t ko = g.k_ord[j];
        if (ko >= 0)
          p = static_cast<double>(static_cast<TP>(
              load_as_double(g.canon, g.canon_dtype, h * g.c_s0 + qo * g.c_s1 + ko * g.c_s2)));
      }
    } else {
      p = causal ? load_as_double(g.fixed, g.fixed_dtype, h * g.f_s0 + row * g.f_s1 + j * g.f_s2)
                 : 0.0;
    }
    carry += tile_total;

    if (g.strict) {
      TP pt = static_cast<TP>(p);
      TP right = static_cast<TP>(__shfl_down(static_cast<double>(pt), 1, 64));
      bool right_valid = __shfl_down(causal ? 1 : 0, 1, 64) != 0;
      int64_t right_kp = __shfl_down(kp, 1, 64);
      if (lane == 63) {
        right = prev_p;
        right_valid = prev_valid;
        right_kp = prev_kp;
      }
      path_bits |= path_violations<TP>(pt, causal, right, causal && right_valid, qp, kp,
                                       right_kp, atol);
      prev_p = static_cast<TP>(__shfl(static_cast<double>(pt), 0, 64));
      prev_valid = __shfl(causal ? 1 : 0, 0, 64) != 0;
      prev_kp = __shfl(kp, 0, 64);
    }

    Acc score = -INFINITY;
    bool vis = false;
    if (causal) {
      Acc b = lerp_bias<Acc>(qe, p, g.npos, &bad_pos);
      score = logit + b;
      if (!isfinite(score)) local_flags |= CS_FLAG_SCORE_NONFINITE;
      vis = allowed && g.vmask.get(h, row, j);
      if (vis && g.sel_rows) vis = !sel_row || !g.fixed_keys[j] || qp == kp;
    }
    if (g.pos_out && causal)
      store_from_double(g.pos_out, g.pos_dtype, h * g.p_s0 + row * g.p_s1 + j * g.p_s2, p);

    if (g.out) {
      Acc sv = vis ? score : static_cast<Acc>(-INFINITY);
      Acc tmax = wave_max(sv);
      if (tmax > static_cast<Acc>(-INFINITY)) {
        Acc mnew = m > tmax ? m : tmax;
        Acc corr = exp(m - mnew);
        Acc pj = vis ? exp(score - mnew) : Acc(0);
        l = l * corr + wave_sum(pj);
        pr[lane] = pj;
        wave_sync();
#pragma unroll
        for (int i = 0; i < kMaxDvChunks; ++i) o[i] *= corr;
        const int64_t tile_keys = (kend - t * 64) < 64 ? (kend - t * 64) : 64;
        for (int64_t jj = 0; jj < tile_keys; ++jj) {
          Acc w = pr[jj];
          if (w != Acc(0)) {
            const int64_t vb = (t * 64 + jj) * g.v_s0 + kvh * g.v_s1;
#pragma unroll
            for (int i = 0; i < kMaxDvChunks; ++i) {
              int64_t dvi = lane + 64 * i;
              if (i < ndv && dvi < g.dv) o[i] += w * E::load(vv, vb + dvi * g.v_s2);
            }
          }
        }
        m = mnew;
        wave_sync();
      }
    }
  }

  // Non-causal keys: the contextual position is 0 (no allowed gate to the
  // right), unless a canonical or fixed value replaces it; those values are
  // bounds-checked like every other bias position.
  if (g.pos_out || g.canon || !contextual) {
    for (int64_t j = kend + lane; j < g.nk; j += 64) {
      double p = 0.0;
      if (contextual) {
        if (qo >= 0) {
          int64_t ko = g.k_ord[j];
          if (ko >= 0)
            p = static_cast<double>(static_cast<TP>(
                load_as_double(g.canon, g.canon_dtype, h * g.c_s0 + qo * g.c_s1 + ko * g.c_s2)));
        }
      } else {
        p = load_as_double(g.fixed, g.fixed_dtype, h * g.f_s0 + row * g.f_s1 + j * g.f_s2);
      }
      if (!(p >= 0.0) || !(p <= static_cast<double>(g.npos - 1))) bad_pos = true;
      if (g.pos_out) store_from_double(g.pos_out, g.pos_dtype, h * g.p_s0 + row * g.p_s1 + j * g.p_s2, p);
    }
  }

  if (g.out) {
    S* out = static_cast<S*>(g.out);
    const int64_t ob = row * g.o_s0 + h * g.o_s1;
#pragma unroll
    for (int i = 0; i < kMaxDvChunks; ++i) {
      int64_t dvi = lane + 64 * i;
      if (i < ndv && dvi < g.dv) {
        Acc val = l > Acc(0) ? o[i] / l : Acc(0);
        E::store(out, ob + dvi * g.o_s2, val);
      }
    }
  }
  // With canonical substitution the contextual cells are clamped into range,
  // so an out-of-range position is a canonical cell: the reference rejects it
  // in the transform's bounds check of its chunk (position.py:500-515), in
  // chunk order with the policy's other errors.
  const bool canon_oob = bad_pos && g.canon && contextual;
  if (bad_pos && !canon_oob) local_flags |= CS_FLAG_POS_INVALID;
  // one atomic per wave
  int all_flags = local_flags;
  for (int off = 32; off > 0; off >>= 1) all_flags |= __shfl_xor(all_flags, off, 64);
  int all_path = path_bits | (canon_oob ? kChunkCanonOutOfRange : 0);
  for (int off = 32; off > 0; off >>= 1) all_path |= __shfl_xor(all_path, off, 64);
  if (lane == 0) {
    if (all_flags) atomicOr(g.flags, all_flags);
    // q_ord == -2 marks a fixed row whose ordinal the profile does not cover:
    // no substitution, but the chunk still counts as holding a fixed row.
    const bool fixed_row = g.canon && g.q_ord && g.q_ord[row] != -1;
    const bool unknown_row = g.canon && g.q_ord && g.q_ord[row] == -2;
    if (g.chunk_flags && (all_path || fixed_row))
      atomicOr(&g.chunk_flags[row / g.chunk_rows], all_path | (fixed_row ? kChunkHasFixedRow : 0) |
                                                        (unknown_row ? kChunkUnknownRow : 0));
  }
}

// ------------------------------------------------------------ input checks
__device__ inline int64_t view_offset(const dview& v, int64_t linear) {
  int64_t off = 0;
  for (int dim = v.ndim - 1; dim >= 0; --dim) {
    int64_t sz = v.shape[dim];
    int64_t idx = linear % sz;
    linear /= sz;
    off += idx * v.stride[dim];
  }
  return off;
}

__global__ void check_finite_kernel(dview v, int64_t numel, int32_t bit, int32_t* flags) {
  int found = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < numel;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    double x = load_as_double(v.data, v.dtype, view_offset(v, i));
    if (!isfinite(x)) found = 1;
  }
  if (__any(found) && (threadIdx.x & 63) == 0) atomicOr(flags, bit);
}

// Contiguous, 16-byte aligned tensors: test the exponent fields of 16-byte
// words (all-ones exponent = inf or NaN), four words in flight per thread.
// KIND: 0 bf16, 1 f16, 2 f32, 3 f64.
template <int KIND>
__global__ void __launch_bounds__(256) check_finite_vec_kernel(const uint4* p, int64_t words,
                                                               int32_t bit, int32_t* flags) {
  bool bad = false;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  for (; i + 3 * step < words; i += 4 * step) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = p[i + u * step];
#pragma unroll
    for (int u = 0; u < 4; ++u) bad |= word_nonfinite<KIND>(v[u]);
  }
  for (; i < words; i += step) bad |= word_nonfinite<KIND>(p[i]);
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flags, bit);
}

constexpr int32_t kQposUnsortedInternal = 1 << 24;

__global__ void check_positions_kernel(const int64_t* pos, int64_t n, int32_t neg_bit,
                                       int32_t unsorted_bit, int32_t* flags) {
  int bits = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t p = pos[i];
    if (p < 0) bits |= neg_bit;
    if (i > 0 && p <= pos[i - 1]) bits |= unsorted_bit;
  }
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off, 64);
  if (bits && (threadIdx.x & 63) == 0) atomicOr(flags, bits);
}

// Quadratic duplicate scan, skipped unless the order check found a descent.
__global__ void check_duplicates_kernel(const int64_t* pos, int64_t n, int32_t unsorted_bit,
                                        int32_t dup_bit, int32_t* flags) {
  if ((*flags & unsorted_bit) == 0) return;
  int found = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t p = pos[i];
    for (int64_t jdx = i + 1; jdx < n; ++jdx)
      if (pos[jdx] == p) { found = 1; break; }
  }
  if (__any(found) && (threadIdx.x & 63) == 0) atomicOr(flags, dup_bit);
}

__global__ void check_bias_positions_kernel(dview v, int64_t numel, double top, int32_t* flags) {
  int bits = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < numel;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    double x = load_as_double(v.data, v.dtype, view_offset(v, i));
    if (!isfinite(x)) bits |= CS_FLAG_POS_INVALID | CS_FLAG_POS_NONFINITE;
    else if (x < 0.0 || x > top) bits |= CS_FLAG_POS_INVALID;
  }
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off, 64);
  if (bits && (threadIdx.x & 63) == 0) atomicOr(flags, bits);
}

// validate_contextual_path on an explicit positions tensor [H, q, k].
template <typename TP>
__global__ void validate_path_kernel(dview pos, const int64_t* qpos, const int64_t* kpos,
                                     mask3 am, TP atol, int32_t* flags) {
  const int64_t H = pos.shape[0], Q = pos.shape[1], K = pos.shape[2];
  const int64_t total = H * Q * K;
  int bits = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t j = i % K;
    int64_t r = (i / K) % Q;
    int64_t h = i / (K * Q);
    int64_t qp = qpos[r], kp = kpos[j];
    bool valid = kp <= qp && am.get(h, r, j);
    if (!valid) continue;
    TP p = static_cast<TP>(load_as_double(pos.data, pos.dtype, h * pos.stride[0] + r * pos.stride[1] + j * pos.stride[2]));
    bool pair = false;
    TP pr = 0;
    int64_t kpr = 0;
    if (j + 1 < K) {
      kpr = kpos[j + 1];
      pair = kpr <= qp && am.get(h, r, j + 1);
      if (pair)
        pr = static_cast<TP>(load_as_double(pos.data, pos.dtype,
                                            h * pos.stride[0] + r * pos.stride[1] + (j + 1) * pos.stride[2]));
    }
    bits |= path_violations<TP>(p, true, pr, pair, qp, kp, kpr, atol);
  }
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off, 64);
  if (bits && (threadIdx.x & 63) == 0) atomicOr(flags, bits);
}

// CoPE.positional_bias for a full positions tensor: one wave per (row, head).
template <typename T>
__global__ void __launch_bounds__(64 * kGenWaves) positional_bias_kernel(
    dview q, dview e, dview pos, dview out, int64_t npos, int64_t wave_bytes, int32_t* flags) {
  using E = elem<T>;
  using Acc = typename E::acc;
  using S = typename E::storage;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t nq = q.shape[0], hq = q.shape[1], d = q.shape[2], nk = pos.shape[2];
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * kGenWaves + wave;
  if (pair >= nq * hq) return;
  const int64_t row = pair / hq, h = pair % hq;
  Acc* qs = reinterpret_cast<Acc*>(smem_raw + wave * wave_bytes);
  Acc* qe = qs + d;
  const S* qd = static_cast<const S*>(q.data);
  for (int64_t i = lane; i < d; i += 64) qs[i] = E::load(qd, row * q.stride[0] + h * q.stride[1] + i * q.stride[2]);
  wave_sync();
  for (int64_t pp = lane; pp < npos; pp += 64) {
    Acc acc = 0;
    for (int64_t i = 0; i < d; ++i)
      acc += qs[i] * static_cast<Acc>(load_as_double(e.data, e.dtype, i * e.stride[0] + pp * e.stride[1]));
    qe[pp] = acc;
  }
  wave_sync();
  bool bad = false;
  for (int64_t j = lane; j < nk; j += 64) {
    double p = load_as_double(pos.data, pos.dtype, h * pos.stride[0] + row * pos.stride[1] + j * pos.stride[2]);
    Acc b = lerp_bias<Acc>(qe, p, npos, &bad);
    store_from_double(out.data, out.dtype, h * out.stride[0] + row * out.stride[1] + j * out.stride[2],
                      static_cast<double>(b));
  }
  if (__any(bad) && lane == 0) atomicOr(flags, CS_FLAG_POS_INVALID);
}

// Membership by binary search: `set` is sorted ascending.
__global__ void isin_kernel(const int64_t* values, int64_t n, const int64_t* set, int64_t m,
                            uint8_t* out) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= n) return;
  const int64_t x = values[i];
  int64_t lo = 0, hi = m;  // first element >= x
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (set[mid] < x) lo = mid + 1; else hi = mid;
  }
  out[i] = (lo < m && set[lo] == x) ? 1 : 0;
}

__global__ void selected_visibility_kernel(const int64_t* queries, int64_t nq,
                                           const int64_t* keys, int64_t nk,
                                           const uint8_t* qsel, const uint8_t* kfix,
                                           uint8_t* out) {
  int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= nq * nk) return;
  int64_t r = i / nk, j = i % nk;
  out[i] = (!qsel[r] || !kfix[j] || queries[r] == keys[j]) ? 1 : 0;
}

__global__ void canonical_substitute_kernel(dview res, dview canon, const int64_t* rows,
                                            const int64_t* row_ord, int64_t nrows,
                                            const int64_t* cols, const int64_t* col_ord,
                                            int64_t ncols) {
  const int64_t H = res.shape[0];
  const int64_t total = H * nrows * ncols;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t c = i % ncols;
    int64_t r = (i / ncols) % nrows;
    int64_t h = i / (ncols * nrows);
    double v = load_as_double(canon.data, canon.dtype,
                              h * canon.stride[0] + row_ord[r] * canon.stride[1] + col_ord[c] * canon.stride[2]);
    store_from_double(res.data, res.dtype, h * res.stride[0] + rows[r] * res.stride[1] + cols[c] * res.stride[2], v);
  }
}

// contextual_positions on given logits (position.py:295-307): one wave per
// (head, query) row, right-to-left tiles, fp64 suffix sums rounded once.
__global__ void __launch_bounds__(64 * kGenWaves) contextual_positions_kernel(
    dview lg, mask3 allowed, int64_t npos, dview out, int32_t* flags) {
  const int lane = threadIdx.x & 63;
  const int64_t H = lg.shape[0], Q = lg.shape[1], K = lg.shape[2];
  const int64_t rowid = static_cast<int64_t>(blockIdx.x) * kGenWaves + (threadIdx.x >> 6);
  if (rowid >= H * Q) return;
  const int64_t h = rowid / Q, r = rowid % Q;
  const bool dbl = lg.dtype == CS_F64;
  double carry = 0.0;
  int bad = 0;
  for (int64_t t = (K + 63) / 64 - 1; t >= 0; --t) {
    const int64_t j = t * 64 + lane;
    double gate = 0.0;
    if (j < K && allowed.get(h, r, j)) {
      double x = load_as_double(lg.data, lg.dtype, h * lg.stride[0] + r * lg.stride[1] + j * lg.stride[2]);
      if (!isfinite(x)) bad = 1;
      if (dbl) {
        gate = 1.0 / (1.0 + exp(-x));
      } else {
        float xf = static_cast<float>(x);
        float gf = 1.f / (1.f + expf(-xf));
        // the gate is rounded to the logits dtype before the cumulative sum
        double tmp = static_cast<double>(gf);
        if (lg.dtype == CS_BF16) tmp = static_cast<double>(bf16_to_float(float_to_bf16(gf)));
        if (lg.dtype == CS_F16) tmp = static_cast<double>(f16_to_float(float_to_f16(gf)));
        gate = tmp;
      }
    }
    double s = gate;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      double nb = __shfl_down(s, off, 64);
      if (lane + off < 64) s += nb;
    }
    const double total = __shfl(s, 0, 64);
    if (j < K) {
      double p = carry + s;
      // round once to the output dtype, then clamp in that dtype
      int64_t off = h * out.stride[0] + r * out.stride[1] + j * out.stride[2];
      store_from_double(out.data, out.dtype, off, p);
      double pr = load_as_double(out.data, out.dtype, off);
      double topv = static_cast<double>(npos - 1);
      if (pr < 0.0) pr = 0.0;
      if (pr > topv) pr = topv;
      store_from_double(out.data, out.dtype, off, pr);
    }
    carry += total;
  }
  if (__any(bad) && lane == 0) atomicOr(flags, CS_FLAG_LOGIT_NONFINITE);
}

// Full logits matrix (position.py:157-164): out[h, r, j] = (q[r,h] . k[j,kvh]) / sqrt(D).
template <typename T>
__global__ void logits_kernel(dview q, dview k, dview out, int32_t* flags) {
  using E = elem<T>;
  using Acc = typename E::acc;
  using S = typename E::storage;
  const int64_t Q = q.shape[0], H = q.shape[1], D = q.shape[2], K = k.shape[0], HKV = k.shape[1];
  const int64_t total = H * Q * K;
  const Acc sqrt_d = static_cast<Acc>(sqrt(static_cast<double>(D)));
  int bad = 0;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t j = i % K, r = (i / K) % Q, h = i / (K * Q);
    int64_t kvh = h / (H / HKV);
    const S* qd = static_cast<const S*>(q.data);
    const S* kd = static_cast<const S*>(k.data);
    Acc dot = 0;
    for (int64_t d = 0; d < D; ++d)
      dot += E::load(qd, r * q.stride[0] + h * q.stride[1] + d * q.stride[2]) *
             E::load(kd, j * k.stride[0] + kvh * k.stride[1] + d * k.stride[2]);
    Acc l = dot / sqrt_d;
    if (!isfinite(l)) bad = 1;
    store_from_double(out.data, out.dtype, h * out.stride[0] + r * out.stride[1] + j * out.stride[2],
                      static_cast<double>(l));
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flags, CS_FLAG_LOGIT_NONFINITE);
}

int grid_for(int64_t total, int threads) {
  int64_t g = ceil_div(total, threads);
  if (g > 65535 * 16) g = 65535 * 16;
  return static_cast<int>(g < 1 ? 1 : g);
}

mask3 to_mask3(const cs_view* m, int64_t hq) {
  mask3 r{};
  if (!present(m)) return r;
  r.data = static_cast<const uint8_t*>(m->data);
  if (m->ndim == 2) {
    r.sh = 0; r.sq = m->stride[0]; r.sk = m->stride[1];
  } else {
    r.sh = m->shape[0] == 1 ? 0 : m->stride[0];
    r.sq = m->stride[1];
    r.sk = m->stride[2];
  }
  (void)hq;
  return r;
}

}  // namespace
}  // namespace cs

using namespace cs;

extern "C" int cs_ccpe_attention(const cs_ccpe_args* a, void* stream) {
  CS_REQUIRE(a != nullptr, "null arguments");
  const cs_view &q = a->q, &k = a->k, &v = a->v, &e = a->e;
  CS_REQUIRE(q.ndim == 3 && k.ndim == 3 && v.ndim == 3 && e.ndim == 2, "q/k/v must be 3-d, e 2-d");
  // zero query tokens is a valid call with an empty result (position.py:117-150
  // asks for one key, not one query); empty tensors carry no data pointer
  const bool no_queries = q.shape[0] == 0;
  CS_REQUIRE((q.data || no_queries) && k.data && v.data && e.data, "q, k, v and e are required");
  CS_REQUIRE(q.dtype == k.dtype && k.dtype == v.dtype && is_float_dtype(q.dtype),
             "q, k, v must share a float dtype");
  const int64_t nq = q.shape[0], hq = q.shape[1], d = q.shape[2];
  const int64_t nk = k.shape[0], hkv = k.shape[1], dv = v.shape[2];
  CS_REQUIRE(k.shape[2] == d && v.shape[0] == nk && v.shape[1] == hkv && hkv > 0 && hq % hkv == 0,
             "inconsistent q/k/v shapes");
  CS_REQUIRE(e.shape[0] == d && e.shape[1] >= 2 && is_float_dtype(e.dtype), "e must be [D, P]");
  CS_REQUIRE((a->qpos || no_queries) && a->kpos && a->flags, "positions and flags are required");
  CS_REQUIRE(dv <= 64 * kMaxDvChunks, "value head dim %lld exceeds %d", (long long)dv,
             64 * kMaxDvChunks);
  const int64_t npos = e.shape[1];
  const bool dbl = q.dtype == CS_F64;
  const int64_t acc_bytes = dbl ? 8 : 4;
  const int64_t p_pad = (npos + 3) & ~int64_t(3);
  int64_t wave_bytes = (d + p_pad + 64) * acc_bytes;
  wave_bytes = (wave_bytes + 15) & ~int64_t(15);
  const int64_t smem = wave_bytes * kGenWaves;
  if (smem > 64 * 1024) {
    set_error("head dim %lld and max_positions %lld exceed the generic kernel's LDS budget",
              (long long)d, (long long)npos);
    return CS_EUNSUPPORTED;
  }
  if (nq == 0 || hq == 0) return CS_OK;
  gen_params g{};
  g.q = q.data; g.q_s0 = q.stride[0]; g.q_s1 = q.stride[1]; g.q_s2 = q.stride[2];
  g.k = k.data; g.k_s0 = k.stride[0]; g.k_s1 = k.stride[1]; g.k_s2 = k.stride[2];
  g.v = v.data; g.v_s0 = v.stride[0]; g.v_s1 = v.stride[1]; g.v_s2 = v.stride[2];
  g.e = e.data; g.e_dtype = e.dtype; g.e_s0 = e.stride[0]; g.e_s1 = e.stride[1];
  g.nq = nq; g.nk = nk; g.hq = hq; g.hkv = hkv; g.d = d; g.dv = dv; g.npos = npos;
  g.qpos = a->qpos; g.kpos = a->kpos;
  g.amask = to_mask3(&a->attn_mask, hq);
  g.vmask = to_mask3(&a->vis_mask, hq);
  g.sel_rows = a->sel_rows;
  g.fixed_keys = a->fixed_keys;
  CS_REQUIRE((g.sel_rows == nullptr) == (g.fixed_keys == nullptr),
             "sel_rows and fixed_keys go together");
  if (present(&a->fixed_pos)) {
    const cs_view& f = a->fixed_pos;
    CS_REQUIRE(f.ndim == 3 && f.shape[0] == hq && f.shape[1] == nq && f.shape[2] == nk &&
                   is_float_dtype(f.dtype),
               "fixed positions must be [Hq, nq, nk]");
    g.fixed = f.data; g.fixed_dtype = f.dtype;
    g.f_s0 = f.stride[0]; g.f_s1 = f.stride[1]; g.f_s2 = f.stride[2];
  }
  if (present(&a->canonical)) {
    const cs_view& c = a->canonical;
    CS_REQUIRE(g.fixed == nullptr, "canonical substitution and fixed positions are exclusive");
    CS_REQUIRE(c.ndim == 3 && c.shape[0] == hq && a->q_ord && a->k_ord && is_float_dtype(c.dtype),
               "canonical must be [Hq, F, F] with ordinal maps");
    g.canon = c.data; g.canon_dtype = c.dtype;
    g.c_s0 = c.stride[0]; g.c_s1 = c.stride[1]; g.c_s2 = c.stride[2];
    g.q_ord = a->q_ord; g.k_ord = a->k_ord;
  }
  g.strict = a->strict;
  g.chunk_rows = a->chunk_rows > 0 ? a->chunk_rows : 1;
  g.chunk_flags = a->chunk_flags;
  CS_REQUIRE(!g.strict || g.chunk_flags, "strict validation needs chunk flags");
  if (present(&a->out)) {
    const cs_view& o = a->out;
    CS_REQUIRE(o.ndim == 3 && o.shape[0] == nq && o.shape[1] == hq && o.shape[2] == dv &&
                   o.dtype == v.dtype,
               "out must be [nq, Hq, Dv] in the value dtype");
    g.out = o.data; g.o_s0 = o.stride[0]; g.o_s1 = o.stride[1]; g.o_s2 = o.stride[2];
  }
  if (present(&a->pos_out)) {
    const cs_view& p = a->pos_out;
    CS_REQUIRE(p.ndim == 3 && p.shape[0] == hq && p.shape[1] == nq && p.shape[2] == nk &&
                   is_float_dtype(p.dtype),
               "pos_out must be [Hq, nq, nk]");
    g.pos_out = p.data; g.pos_dtype = p.dtype;
    g.p_s0 = p.stride[0]; g.p_s1 = p.stride[1]; g.p_s2 = p.stride[2];
  }
  g.flags = a->flags;
  g.wave_bytes = wave_bytes;
  g.p_pad = p_pad;
  const int64_t pairs = nq * hq;
  dim3 grid(static_cast<unsigned>(ceil_div(pairs, kGenWaves)));
  dim3 block(64 * kGenWaves);
  hipStream_t s = as_stream(stream);
  switch (q.dtype) {
    case CS_F32: hipLaunchKernelGGL(ccpe_generic_kernel<float>, grid, block, smem, s, g); break;
    case CS_F64: hipLaunchKernelGGL(ccpe_generic_kernel<double>, grid, block, smem, s, g); break;
    case CS_BF16: hipLaunchKernelGGL(ccpe_generic_kernel<bf16_t>, grid, block, smem, s, g); break;
    case CS_F16: hipLaunchKernelGGL(ccpe_generic_kernel<f16_t>, grid, block, smem, s, g); break;
  }
  CS_LAUNCH_CHECK("ccpe_generic");
  return CS_OK;
}

extern "C" int cs_check_finite(const cs_view* x, int32_t bit, int32_t* flags, void* stream) {
  CS_REQUIRE(x && flags, "null arguments");
  if (!x->data || !is_float_dtype(x->dtype)) return CS_OK;
  int64_t numel = 1;
  for (int i = 0; i < x->ndim; ++i) numel *= x->shape[i];
  if (numel == 0) return CS_OK;
  bool contiguous = true;
  int64_t expect = 1;
  for (int i = x->ndim - 1; i >= 0; --i) {
    if (x->shape[i] != 1 && x->stride[i] != expect) contiguous = false;
    expect *= x->shape[i];
  }
  const int esize = dtype_size(x->dtype);
  const int64_t bytes = numel * esize;
  if (contiguous && (reinterpret_cast<uintptr_t>(x->data) & 15) == 0 && bytes % 16 == 0) {
    const int64_t words = bytes / 16;
    const int grid = static_cast<int>(std::min<int64_t>(ceil_div(words, 256 * 4), 4096));
    const uint4* p = static_cast<const uint4*>(x->data);
    hipStream_t s = as_stream(stream);
    switch (x->dtype) {
      case CS_BF16: hipLaunchKernelGGL((check_finite_vec_kernel<0>), dim3(grid), dim3(256), 0, s, p, words, bit, flags); break;
      case CS_F16: hipLaunchKernelGGL((check_finite_vec_kernel<1>), dim3(grid), dim3(256), 0, s, p, words, bit, flags); break;
      case CS_F32: hipLaunchKernelGGL((check_finite_vec_kernel<2>), dim3(grid), dim3(256), 0, s, p, words, bit, flags); break;
      default: hipLaunchKernelGGL((check_finite_vec_kernel<3>), dim3(grid), dim3(256), 0, s, p, words, bit, flags); break;
    }
    CS_LAUNCH_CHECK("check_finite");
    return CS_OK;
  }
  dview v = to_dview(x);
  hipLaunchKernelGGL(check_finite_kernel, dim3(grid_for(numel, 256)), dim3(256), 0,
                     as_stream(stream), v, numel, bit, flags);
  CS_LAUNCH_CHECK("check_finite");
  return CS_OK;
}

extern "C" int cs_check_positions(const int64_t* pos, int64_t n, int32_t is_key, int32_t* flags,
                                  void* stream) {
  CS_REQUIRE(flags, "null flags");
  if (n == 0) return CS_OK;
  CS_REQUIRE(pos, "null positions");
  int32_t neg = is_key ? CS_FLAG_KPOS_NEGATIVE : CS_FLAG_QPOS_NEGATIVE;
  int32_t uns = is_key ? CS_FLAG_KPOS_UNSORTED : kQposUnsortedInternal;
  int32_t dup = is_key ? CS_FLAG_KPOS_DUPLICATE : CS_FLAG_QPOS_DUPLICATE;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(check_positions_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, pos, n, neg,
                     uns, flags);
  hipLaunchKernelGGL(check_duplicates_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, pos, n, uns,
                     dup, flags);
  CS_LAUNCH_CHECK("check_positions");
  return CS_OK;
}

extern "C" int cs_check_bias_positions(const cs_view* positions, int64_t max_positions,
                                       int32_t* flags, void* stream) {
  CS_REQUIRE(positions && flags, "null arguments");
  if (!positions->data) return CS_OK;
  int64_t numel = 1;
  for (int i = 0; i < positions->ndim; ++i) numel *= positions->shape[i];
  if (numel == 0) return CS_OK;
  if (!is_float_dtype(positions->dtype)) {
    set_error("positions must be floating");
    return CS_EINVAL;
  }
  hipLaunchKernelGGL(check_bias_positions_kernel, dim3(grid_for(numel, 256)), dim3(256), 0,
                     as_stream(stream), to_dview(positions), numel,
                     static_cast<double>(max_positions - 1), flags);
  CS_LAUNCH_CHECK("check_bias_positions");
  return CS_OK;
}

extern "C" int cs_validate_contextual_path(const cs_view* positions, const int64_t* qpos,
                                           const int64_t* kpos, const cs_view* attn_mask,
                                           double atol, int32_t* flags, void* stream) {
  CS_REQUIRE(positions && positions->data && positions->ndim == 3 && qpos && kpos && flags,
             "positions [H,q,k], coordinates and flags are required");
  CS_REQUIRE(is_float_dtype(positions->dtype), "positions must be floating");
  int64_t total = positions->shape[0] * positions->shape[1] * positions->shape[2];
  if (total == 0) return CS_OK;
  mask3 am = to_mask3(attn_mask, positions->shape[0]);
  hipStream_t s = as_stream(stream);
  dview p = to_dview(positions);
  if (positions->dtype == CS_F64)
    hipLaunchKernelGGL(validate_path_kernel<double>, dim3(grid_for(total, 256)), dim3(256), 0, s,
                       p, qpos, kpos, am, atol, flags);
  else
    hipLaunchKernelGGL(validate_path_kernel<float>, dim3(grid_for(total, 256)), dim3(256), 0, s,
                       p, qpos, kpos, am, static_cast<float>(atol), flags);
  CS_LAUNCH_CHECK("validate_contextual_path");
  return CS_OK;
}

extern "C" int cs_cope_positional_bias(const cs_view* q, const cs_view* e,
                                       const cs_view* positions, cs_view* out, int32_t* flags,
                                       void* stream) {
  CS_REQUIRE(q && e && positions && out && flags && q->data && e->data && positions->data &&
                 out->data,
             "null arguments");
  CS_REQUIRE(q->ndim == 3 && e->ndim == 2 && positions->ndim == 3 && out->ndim == 3,
             "bad ranks");
  const int64_t nq = q->shape[0], hq = q->shape[1], d = q->shape[2], npos = e->shape[1];
  CS_REQUIRE(e->shape[0] == d && positions->shape[0] == hq && positions->shape[1] == nq,
             "shape mismatch");
  const bool dbl = q->dtype == CS_F64;
  const int64_t acc_bytes = dbl ? 8 : 4;
  int64_t wave_bytes = ((d + ((npos + 3) & ~int64_t(3))) * acc_bytes + 15) & ~int64_t(15);
  int64_t smem = wave_bytes * kGenWaves;
  if (smem > 64 * 1024) {
    set_error("positional bias table exceeds the LDS budget");
    return CS_EUNSUPPORTED;
  }
  if (nq * hq == 0) return CS_OK;
  dim3 grid(static_cast<unsigned>(ceil_div(nq * hq, kGenWaves)));
  dim3 block(64 * kGenWaves);
  hipStream_t s = as_stream(stream);
  dview qd = to_dview(q), ed = to_dview(e), pd = to_dview(positions), od = to_dview(out);
  switch (q->dtype) {
    case CS_F32: hipLaunchKernelGGL(positional_bias_kernel<float>, grid, block, smem, s, qd, ed, pd, od, npos, wave_bytes, flags); break;
    case CS_F64: hipLaunchKernelGGL(positional_bias_kernel<double>, grid, block, smem, s, qd, ed, pd, od, npos, wave_bytes, flags); break;
    case CS_BF16: hipLaunchKernelGGL(positional_bias_kernel<bf16_t>, grid, block, smem, s, qd, ed, pd, od, npos, wave_bytes, flags); break;
    case CS_F16: hipLaunchKernelGGL(positional_bias_kernel<f16_t>, grid, block, smem, s, qd, ed, pd, od, npos, wave_bytes, flags); break;
    default: set_error("unsupported dtype"); return CS_EINVAL;
  }
  CS_LAUNCH_CHECK("positional_bias");
  return CS_OK;
}

extern "C" int cs_selected_visibility(const int64_t* queries, int64_t nq, const int64_t* keys,
                                      int64_t nk, const int64_t* fixed, int64_t nfixed,
                                      const int64_t* selected, int64_t nselected, uint8_t* out,
                                      void* stream) {
  // The boolean row/column flags live at the front of `out`'s tail-free
  // scratch: callers pass out with nq*nk + nq + nk bytes.
  if (nq == 0 || nk == 0) return CS_OK;
  CS_REQUIRE(queries && keys && out, "null arguments");
  uint8_t* qsel = out + nq * nk;
  uint8_t* kfix = qsel + nq;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(isin_kernel, dim3(ceil_div(nq, 256)), dim3(256), 0, s, queries, nq,
                     selected, nselected, qsel);
  hipLaunchKernelGGL(isin_kernel, dim3(ceil_div(nk, 256)), dim3(256), 0, s, keys, nk, fixed,
                     nfixed, kfix);
  hipLaunchKernelGGL(selected_visibility_kernel, dim3(ceil_div(nq * nk, 256)), dim3(256), 0, s,
                     queries, nq, keys, nk, qsel, kfix, out);
  CS_LAUNCH_CHECK("selected_visibility");
  return CS_OK;
}

extern "C" int cs_isin(const int64_t* values, int64_t n, const int64_t* set, int64_t m,
                       uint8_t* out, void* stream) {
  if (n == 0) return CS_OK;
  CS_REQUIRE(values && out && (m == 0 || set), "null arguments");
  hipLaunchKernelGGL(isin_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, as_stream(stream), values,
                     n, set, m, out);
  CS_LAUNCH_CHECK("isin");
  return CS_OK;
}

extern "C" int cs_canonical_substitute(cs_view* result, const cs_view* canonical,
                                       const int64_t* rows, const int64_t* row_ordinals,
                                       int64_t nrows, const int64_t* cols,
                                       const int64_t* col_ordinals, int64_t ncols, void* stream) {
  CS_REQUIRE(result && canonical && result->ndim == 3 && canonical->ndim == 3, "bad views");
  int64_t total = result->shape[0] * nrows * ncols;
  if (total == 0) return CS_OK;
  hipLaunchKernelGGL(canonical_substitute_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                     as_stream(stream), to_dview(result), to_dview(canonical), rows, row_ordinals,
                     nrows, cols, col_ordinals, ncols);
  CS_LAUNCH_CHECK("canonical_substitute");
  return CS_OK;
}

extern "C" int cs_contextual_positions(const cs_view* logits, const cs_view* allowed,
                                       int64_t max_positions, cs_view* out, int32_t* flags,
                                       void* stream) {
  CS_REQUIRE(logits && allowed && out && flags && logits->ndim == 3 && out->ndim == 3,
             "logits/out must be [H, q, k]");
  CS_REQUIRE(present(allowed), "allowed mask required");
  int64_t rows = logits->shape[0] * logits->shape[1];
  if (rows == 0 || logits->shape[2] == 0) return CS_OK;
  mask3 am = to_mask3(allowed, logits->shape[0]);
  hipLaunchKernelGGL(contextual_positions_kernel, dim3(ceil_div(rows, kGenWaves)),
                     dim3(64 * kGenWaves), 0, as_stream(stream), to_dview(logits), am,
                     max_positions, to_dview(out), flags);
  CS_LAUNCH_CHECK("contextual_positions");
  return CS_OK;
}

extern "C" int cs_ccpe_logits(const cs_view* q, const cs_view* k, cs_view* out, int32_t* flags,
                              void* stream) {
  CS_REQUIRE(q && k && out && flags && q->ndim == 3 && k->ndim == 3 && out->ndim == 3,
             "q, k, out must be 3-d");
  CS_REQUIRE(q->dtype == k->dtype && k->shape[1] > 0 && q->shape[1] % k->shape[1] == 0,
             "q/k mismatch");
  int64_t total = q->shape[0] * q->shape[1] * k->shape[0];
  if (total == 0) return CS_OK;
  dim3 grid(grid_for(total, 256));
  hipStream_t s = as_stream(stream);
  dview qd = to_dview(q), kd = to_dview(k), od = to_dview(out);
  switch (q->dtype) {
    case CS_F32: hipLaunchKernelGGL(logits_kernel<float>, grid, dim3(256), 0, s, qd, kd, od, flags); break;
    case CS_F64: hipLaunchKernelGGL(logits_kernel<double>, grid, dim3(256), 0, s, qd, kd, od, flags); break;
    case CS_BF16: hipLaunchKernelGGL(logits_kernel<bf16_t>, grid, dim3(256), 0, s, qd, kd, od, flags); break;
    case CS_F16: hipLaunchKernelGGL(logits_kernel<f16_t>, grid, dim3(256), 0, s, qd, kd, od, flags); break;
    default: set_error("unsupported dtype"); return CS_EINVAL;
  }
  CS_LAUNCH_CHECK("ccpe_logits");
  return CS_OK;
}
