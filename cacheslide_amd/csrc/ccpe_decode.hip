// CCPE decode attention: one new query row per request at position nk-1 over
// keys 0..nk-1 (position.py:404-560 with q = 1, as called from
// runtime.py:489-508), bf16, head dim 128, K/V from the paged cache.
//
// Split-K with speculative saturation.  The keys of a request are cut into
// splits aligned to the last key (split r covers [nk-(r+1)S, nk-rS)), so the
// right-most split always holds S keys.  Split 0 is computed exactly (carry 0).
// Every other split assumes that the gate mass of the keys to its right is
// already >= P-1, which makes every position in it P-1 and the bias the row
// constant QE[P-1]; it records its own gate total.  A fixup launch then forms
// each split's true carry (sum of the totals to its right) and recomputes
// exactly only the splits whose carry is below P-1.  A combine launch merges
// the per-split (max, sum, accumulator) triples.
//
// Inside a split, each of the 4 wavefronts owns a contiguous quarter of the
// keys.  Speculative splits stream K and V once with an online softmax
// (decode_spec_kernel).  Exact splits (decode_split_kernel): pass 1 streams K
// (16 lanes x 16 B per key row) and leaves the logits of the whole GQA group in
// LDS; pass 2 turns them into scores with an exact right-to-left wave scan from
// the carry; pass 3 streams V and accumulates P.V.

#include "common.h"

namespace cs {
namespace {

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxGroup = 8;
constexpr int kMaxPos = 256;
constexpr int kMaxSplit = 1024;

struct kv_addr {
  const uint16_t* cache;
  int64_t s_block, s_head, s_offset;
  int32_t block_size, bs_shift;  // bs_shift >= 0 when block_size is a power of two
  int64_t num_blocks;
  const int32_t* block_table;
  int64_t bt_stride, bt_cols;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;
};

struct decode_params {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  int32_t batch, hq, hkv, group;
  const int32_t* nk;
  kv_addr kv;
  const float* e;
  int32_t npos;
  int32_t split, smax;
  double* tot;   // [B, hq, smax] gate totals
  float* mx;     // [B, hq, smax] running max (log2 domain)
  float* sm;     // [B, hq, smax] sum of exp2
  float* acc;    // [B, hq, smax, 128]
  uint16_t* out;
  int32_t* flags;
};

__device__ inline const uint16_t* kv_row(const kv_addr& a, int b, int kvh, int64_t j, bool is_v,
                                         bool* bad) {
  if (a.block_table) {
    const int64_t bi = a.bs_shift >= 0 ? (j >> a.bs_shift) : j / a.block_size;
    if (bi >= a.bt_cols) {
      *bad = true;
      return nullptr;
    }
    const int32_t blk = a.block_table[b * a.bt_stride + bi];
    if (blk < 0 || blk >= a.num_blocks) {
      *bad = true;
      return nullptr;
    }
    const int64_t off = a.bs_shift >= 0 ? (j & ((int64_t(1) << a.bs_shift) - 1)) : j % a.block_size;
    return a.cache + blk * a.s_block + kvh * a.s_head + off * a.s_offset + (is_v ? kD : 0);
  }
  return is_v ? a.v + b * a.v_sb + j * a.v_st + kvh * a.v_sh
              : a.k + b * a.k_sb + j * a.k_st + kvh * a.k_sh;
}

__device__ inline void unpack8(uint4 u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ inline int64_t ws_index(const decode_params& p, int b, int h, int r) {
  return (static_cast<int64_t>(b) * p.hq + h) * p.smax + r;
}

// Speculative split r >= 1: every position is assumed saturated (p = P-1), so
// the bias is the per-head constant QE[P-1] and the split is one streaming pass
// of plain attention.  Each 16-lane group owns one key at a time (lane x holds
// dims 8x..8x+7 of its K and V rows) and keeps an online-softmax state per
// head over the keys it has seen; the 4 lane groups and 4 waves are merged at
// the end.  The split's gate total is recorded for the fixup pass.
constexpr int kSpecUnroll = 4;

template <int GT>
__global__ void __launch_bounds__(kThreads) decode_spec_kernel(decode_params p) {
  constexpr int kMaxGroup = GT;  // registers sized for this group, not the maximum
  __shared__ float wave_m[kWaves][kMaxGroup];
  __shared__ float wave_l[kWaves][kMaxGroup];
  __shared__ double wave_tot[kWaves][kMaxGroup];
  __shared__ float wave_o[kWaves][kMaxGroup][kD];

  const int r = blockIdx.x + 1, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int a4 = lane >> 4, x = lane & 15;
  constexpr int G = GT;
  const int nk = p.nk[b];
  int splits = (nk + p.split - 1) / p.split;
  if (splits > p.smax) splits = p.smax;
  if (r >= splits) return;
  const int64_t hi = static_cast<int64_t>(nk) - static_cast<int64_t>(r) * p.split;
  const int64_t lo = hi - p.split > 0 ? hi - p.split : 0;
  const int h0 = kvh * G;
  const float kLog2e = 1.4426950408889634f;
  const float c_scale = 0.08838834764831845f * kLog2e;  // log2(e) / sqrt(128)

  // q slice of every head in registers; QE[P-1] by a 16-lane reduction
  float qr[kMaxGroup][8];
  float bias2[kMaxGroup];  // QE[P-1] * log2(e)
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg) {
    if (gg < G) {
      uint4 u = *reinterpret_cast<const uint4*>(p.q + b * p.q_sb + (h0 + gg) * p.q_sh + 8 * x);
      unpack8(u, qr[gg]);
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) part += qr[gg][i] * p.e[(8 * x + i) * p.npos + (p.npos - 1)];
      part += __shfl_xor(part, 8, 64);
      part += __shfl_xor(part, 4, 64);
      part += __shfl_xor(part, 2, 64);
      part += __shfl_xor(part, 1, 64);
      bias2[gg] = part * kLog2e;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) qr[gg][i] = 0.f;
      bias2[gg] = 0.f;
    }
  }

  float m[kMaxGroup], l[kMaxGroup], o[kMaxGroup][8];
  double tsum[kMaxGroup];
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg) {
    m[gg] = -INFINITY;
    l[gg] = 0.f;
    tsum[gg] = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[gg][i] = 0.f;
  }

  const int kw = p.split / kWaves;
  int64_t wlo = lo + static_cast<int64_t>(wave) * kw;
  int64_t whi = wlo + kw;
  if (wlo > hi) wlo = hi;
  if (whi > hi) whi = hi;
  bool bad = false;
  for (int64_t base = wlo; base < whi; base += 4 * kSpecUnroll) {
    uint4 kb[kSpecUnroll], vb[kSpecUnroll];
#pragma unroll
    for (int u = 0; u < kSpecUnroll; ++u) {
      const int64_t j = base + 4 * u + a4;
      kb[u] = make_uint4(0, 0, 0, 0);
      vb[u] = make_uint4(0, 0, 0, 0);
      if (j < whi) {
        const uint16_t* kr = kv_row(p.kv, b, kvh, j, false, &bad);
        if (kr) {
          kb[u] = *reinterpret_cast<const uint4*>(kr + 8 * x);
          vb[u] = *reinterpret_cast<const uint4*>(kr + kD + 8 * x);
        }
      }
    }
    float s[kSpecUnroll][kMaxGroup];
#pragma unroll
    for (int u = 0; u < kSpecUnroll; ++u) {
      float kf[8];
      unpack8(kb[u], kf);
#pragma unroll
      for (int gg = 0; gg < kMaxGroup; ++gg) {
        float d = 0.f;
        if (gg < G) {
#pragma unroll
          for (int i = 0; i < 8; ++i) d += qr[gg][i] * kf[i];
          d += __shfl_xor(d, 8, 64);
          d += __shfl_xor(d, 4, 64);
          d += __shfl_xor(d, 2, 64);
          d += __shfl_xor(d, 1, 64);
        }
        s[u][gg] = d;
      }
    }
#pragma unroll
    for (int gg = 0; gg < kMaxGroup; ++gg) {
      if (gg >= G) continue;
      float xs[kSpecUnroll];
      float mx = m[gg];
#pragma unroll
      for (int u = 0; u < kSpecUnroll; ++u) {
        const bool in = base + 4 * u + a4 < whi;
        // natural-log logit for the gate mass, log2-domain score for softmax
        const float logit = s[u][gg] * 0.08838834764831845f;
        if (in && x == 0) tsum[gg] += static_cast<double>(1.f / (1.f + __expf(-logit)));
        xs[u] = in ? s[u][gg] * c_scale + bias2[gg] : -INFINITY;
        mx = fmaxf(mx, xs[u]);
      }
      if (mx == -INFINITY) continue;
      const float corr = __builtin_amdgcn_exp2f(m[gg] - mx);
      l[gg] *= corr;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[gg][i] *= corr;
#pragma unroll
      for (int u = 0; u < kSpecUnroll; ++u) {
        const float pw = __builtin_amdgcn_exp2f(xs[u] - mx);
        l[gg] += pw;
        float vf[8];
        unpack8(vb[u], vf);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[gg][i] += pw * vf[i];
      }
      m[gg] = mx;
    }
  }

  // merge the 4 lane groups of the wave (xor 16, then xor 32)
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int gg = 0; gg < kMaxGroup; ++gg) {
      if (gg >= G) continue;
      const float m2 = __shfl_xor(m[gg], off, 64);
      const float l2 = __shfl_xor(l[gg], off, 64);
      const float M = fmaxf(m[gg], m2);
      const float f1 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[gg] - M);
      const float f2 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - M);
      l[gg] = l[gg] * f1 + l2 * f2;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o2 = __shfl_xor(o[gg][i], off, 64);
        o[gg][i] = o[gg][i] * f1 + o2 * f2;
      }
      m[gg] = M;
      tsum[gg] += __shfl_xor(tsum[gg], off, 64);
    }
  }
  if (a4 == 0) {
#pragma unroll
    for (int gg = 0; gg < kMaxGroup; ++gg)
      if (gg < G)
#pragma unroll
        for (int i = 0; i < 8; ++i) wave_o[wave][gg][8 * x + i] = o[gg][i];
  }
  if (lane == 0) {
#pragma unroll
    for (int gg = 0; gg < kMaxGroup; ++gg)
      if (gg < G) {
        wave_m[wave][gg] = m[gg];
        wave_l[wave][gg] = l[gg];
        wave_tot[wave][gg] = tsum[gg];
      }
  }
  __syncthreads();
  for (int i = tid; i < G * kD; i += kThreads) {
    const int gg = i / kD, d = i % kD;
    float M = -INFINITY;
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, wave_m[ww][gg]);
    float L = 0.f, O = 0.f;
    for (int ww = 0; ww < kWaves; ++ww) {
      const float wm = wave_m[ww][gg];
      if (wm == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f(wm - M);
      L += wave_l[ww][gg] * f;
      O += wave_o[ww][gg][d] * f;
    }
    const int64_t wi = ws_index(p, b, h0 + gg, r);
    p.acc[wi * kD + d] = O;
    if (d == 0) {
      p.mx[wi] = M;
      p.sm[wi] = L;
      double T = 0.0;
      for (int ww = 0; ww < kWaves; ++ww) T += wave_tot[ww][gg];
      p.tot[wi] = T;
    }
  }
  if (bad) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
}

__global__ void __launch_bounds__(kThreads) decode_split_kernel(decode_params p, int fixup) {
  __shared__ float q_lds[kMaxGroup][kD];
  __shared__ float qe_lds[kMaxGroup][kMaxPos];
  __shared__ float sc_lds[kMaxGroup][kMaxSplit];
  __shared__ double wave_tot[kWaves][kMaxGroup];
  __shared__ double carry_lds[kMaxGroup];
  __shared__ float wave_m[kWaves][kMaxGroup];
  __shared__ float wave_l[kWaves][kMaxGroup];
  __shared__ float wave_o[kWaves][kMaxGroup][kD];
  __shared__ int skip_lds;

  const int r = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = p.group;
  const int nk = p.nk[b];
  int splits = (nk + p.split - 1) / p.split;
  if (splits > p.smax) splits = p.smax;  // the workspace holds smax splits
  if (r >= splits) return;
  const int64_t hi = static_cast<int64_t>(nk) - static_cast<int64_t>(r) * p.split;
  const int64_t lo = hi - p.split > 0 ? hi - p.split : 0;
  const int h0 = kvh * G;
  const float top = static_cast<float>(p.npos - 1);

  if (fixup) {
    if (r == 0) return;
    if (tid < G) {
      double c = 0.0;
      for (int rr = 0; rr < r; ++rr) c += p.tot[ws_index(p, b, h0 + tid, rr)];
      carry_lds[tid] = c;
    }
    if (tid == 0) skip_lds = 1;
    __syncthreads();
    if (tid < G && carry_lds[tid] < static_cast<double>(top)) skip_lds = 0;
    __syncthreads();
    if (skip_lds) return;
  } else {
    if (tid < G) carry_lds[tid] = 0.0;
  }
  const bool exact = fixup || r == 0;

  // q rows of the group (float) and the QE table (full when exact).
  for (int i = tid; i < G * kD; i += kThreads) {
    int gg = i / kD, d = i % kD;
    q_lds[gg][d] = bf16_to_float(p.q[b * p.q_sb + (h0 + gg) * p.q_sh + d]);
  }
  __syncthreads();
  for (int i = tid; i < G * p.npos; i += kThreads) {
    int gg = i / p.npos, pp = i % p.npos;
    if (!exact && pp != p.npos - 1) continue;
    float a = 0.f;
    for (int d = 0; d < kD; ++d) a += q_lds[gg][d] * p.e[d * p.npos + pp];
    qe_lds[gg][pp] = a;
  }

  // ---- pass 1: logits for this wave's quarter of the split -------------
  const int kw = p.split / kWaves;
  const int64_t wlo = lo + static_cast<int64_t>(wave) * kw > hi ? hi : lo + static_cast<int64_t>(wave) * kw;
  int64_t whi_ = lo + static_cast<int64_t>(wave + 1) * kw;
  const int64_t whi = whi_ > hi ? hi : whi_;
  const int a4 = lane >> 4, x = lane & 15;
  float qr[kMaxGroup][8];
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg)
#pragma unroll
    for (int i = 0; i < 8; ++i) qr[gg][i] = gg < G ? q_lds[gg][8 * x + i] : 0.f;
  const float logit_scale = 0.08838834764831845f;  // 1/sqrt(128)
  double gsum[kMaxGroup];
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg) gsum[gg] = 0.0;
  bool bad = false;
  constexpr int kUnroll = 4;
  for (int64_t base = wlo; base < whi; base += 4 * kUnroll) {
    uint4 kb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t j = base + 4 * u + a4;
      kb[u] = make_uint4(0, 0, 0, 0);
      if (j < whi) {
        const uint16_t* kr = kv_row(p.kv, b, kvh, j, false, &bad);
        if (kr) kb[u] = *reinterpret_cast<const uint4*>(kr + 8 * x);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t j = base + 4 * u + a4;
      float kf[8];
      unpack8(kb[u], kf);
      float dot[kMaxGroup];
#pragma unroll
      for (int gg = 0; gg < kMaxGroup; ++gg) {
        float s = 0.f;
        if (gg < G) {
#pragma unroll
          for (int i = 0; i < 8; ++i) s += qr[gg][i] * kf[i];
        }
        dot[gg] = s;
      }
#pragma unroll
      for (int gg = 0; gg < kMaxGroup; ++gg) {
        if (gg < G) {
          float s = dot[gg];
          s += __shfl_xor(s, 8, 64);
          s += __shfl_xor(s, 4, 64);
          s += __shfl_xor(s, 2, 64);
          s += __shfl_xor(s, 1, 64);
          dot[gg] = s * logit_scale;
        }
      }
      if (x == 0 && j < whi) {
#pragma unroll
        for (int gg = 0; gg < kMaxGroup; ++gg)
          if (gg < G) {
            sc_lds[gg][j - lo] = dot[gg];
            gsum[gg] += static_cast<double>(1.f / (1.f + __expf(-dot[gg])));
          }
      }
    }
  }
  // wave gate totals
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg) {
    if (gg < G) {
      double s = gsum[gg];
      s += __shfl_xor(s, 16, 64);
      s += __shfl_xor(s, 32, 64);
      if (lane == 0) wave_tot[wave][gg] = s;
    }
  }
  __syncthreads();

  // ---- pass 2: scores, wave max, probabilities --------------------------
  const float kLog2e = 1.4426950408889634f;
  float m_w[kMaxGroup], l_w[kMaxGroup];
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg) {
    m_w[gg] = -INFINITY;
    l_w[gg] = 0.f;
  }
  for (int gg = 0; gg < G; ++gg) {
    float* sc = sc_lds[gg];
    const float* qe = qe_lds[gg];
    if (exact) {
      double carry = carry_lds[gg];
      for (int ww = kWaves - 1; ww > wave; --ww) carry += wave_tot[ww][gg];
      const int64_t n = whi - wlo;
      for (int64_t c0 = ((n + 63) / 64 - 1) * 64; c0 >= 0; c0 -= 64) {
        int64_t j = wlo + c0 + lane;
        bool in = j < whi;
        float lg = in ? sc[j - lo] : 0.f;
        double gate = in ? static_cast<double>(1.f / (1.f + __expf(-lg))) : 0.0;
        double s = gate;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          double nb = __shfl_down(s, off, 64);
          if (lane + off < 64) s += nb;
        }
        double tile_total = __shfl(s, 0, 64);
        float pos = static_cast<float>(carry + s);
        pos = pos < top ? pos : top;
        pos = pos > 0.f ? pos : 0.f;  // also maps NaN to 0: table reads stay in range
        float fl = floorf(pos);
        int lo_i = static_cast<int>(fl);
        int hi_i = lo_i + 1 < p.npos - 1 ? lo_i + 1 : p.npos - 1;
        float bias = qe[lo_i] + (pos - fl) * (qe[hi_i] - qe[lo_i]);
        if (in) sc[j - lo] = (lg + bias) * kLog2e;
        carry += tile_total;
      }
    } else {
      const float bl = qe[p.npos - 1];
      for (int64_t j = wlo + lane; j < whi; j += 64) sc[j - lo] = (sc[j - lo] + bl) * kLog2e;
    }
    float mx = -INFINITY;
    for (int64_t j = wlo + lane; j < whi; j += 64) mx = fmaxf(mx, sc[j - lo]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int64_t j = wlo + lane; j < whi; j += 64) {
      float pv = __builtin_amdgcn_exp2f(sc[j - lo] - mx);
      sc[j - lo] = pv;
      sum += pv;
    }
    sum = wave_sum(sum);
    m_w[gg] = mx;
    l_w[gg] = sum;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

  // ---- pass 3: P.V -------------------------------------------------------
  float o[kMaxGroup][8];
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg)
#pragma unroll
    for (int i = 0; i < 8; ++i) o[gg][i] = 0.f;
  for (int64_t base = wlo; base < whi; base += 4 * kUnroll) {
    uint4 vb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t j = base + 4 * u + a4;
      vb[u] = make_uint4(0, 0, 0, 0);
      if (j < whi) {
        const uint16_t* vr = kv_row(p.kv, b, kvh, j, true, &bad);
        if (vr) vb[u] = *reinterpret_cast<const uint4*>(vr + 8 * x);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t j = base + 4 * u + a4;
      if (j < whi) {
        float vf[8];
        unpack8(vb[u], vf);
#pragma unroll
        for (int gg = 0; gg < kMaxGroup; ++gg) {
          if (gg < G) {
            float pw = sc_lds[gg][j - lo];
#pragma unroll
            for (int i = 0; i < 8; ++i) o[gg][i] += pw * vf[i];
          }
        }
      }
    }
  }
#pragma unroll
  for (int gg = 0; gg < kMaxGroup; ++gg)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (gg < G) {
        float s = o[gg][i];
        s += __shfl_xor(s, 16, 64);
        s += __shfl_xor(s, 32, 64);
        o[gg][i] = s;
      }
    }
  if (a4 == 0) {
#pragma unroll
    for (int gg = 0; gg < kMaxGroup; ++gg)
      if (gg < G)
#pragma unroll
        for (int i = 0; i < 8; ++i) wave_o[wave][gg][8 * x + i] = o[gg][i];
  }
  if (lane == 0) {
#pragma unroll
    for (int gg = 0; gg < kMaxGroup; ++gg)
      if (gg < G) {
        wave_m[wave][gg] = m_w[gg];
        wave_l[wave][gg] = l_w[gg];
      }
  }
  __syncthreads();

  // ---- merge the 4 waves and write the split's partial ------------------
  for (int i = tid; i < G * kD; i += kThreads) {
    int gg = i / kD, d = i % kD;
    float M = -INFINITY;
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, wave_m[ww][gg]);
    float L = 0.f, O = 0.f;
    for (int ww = 0; ww < kWaves; ++ww) {
      float wm = wave_m[ww][gg];
      if (wm == -INFINITY) continue;
      float f = __builtin_amdgcn_exp2f(wm - M);
      L += wave_l[ww][gg] * f;
      O += wave_o[ww][gg][d] * f;
    }
    int64_t wi = ws_index(p, b, h0 + gg, r);
    p.acc[wi * kD + d] = O;
    if (d == 0) {
      p.mx[wi] = M;
      p.sm[wi] = L;
      if (!fixup) {
        double T = 0.0;
        for (int ww = 0; ww < kWaves; ++ww) T += wave_tot[ww][gg];
        p.tot[wi] = T;
      }
    }
  }
  if (bad) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
}

__global__ void decode_combine_kernel(decode_params p) {
  const int bh = blockIdx.x;
  const int b = bh / p.hq, h = bh % p.hq;
  const int d = threadIdx.x;  // 128 threads
  const int nk = p.nk[b];
  int splits = (nk + p.split - 1) / p.split;
  if (splits > p.smax) splits = p.smax;
  float M = -INFINITY;
  for (int r = 0; r < splits; ++r) M = fmaxf(M, p.mx[ws_index(p, b, h, r)]);
  float L = 0.f, O = 0.f;
  for (int r = 0; r < splits; ++r) {
    int64_t wi = ws_index(p, b, h, r);
    float m = p.mx[wi];
    if (m == -INFINITY) continue;
    float f = __builtin_amdgcn_exp2f(m - M);
    L += p.sm[wi] * f;
    O += p.acc[wi * kD + d] * f;
  }
  float val = L > 0.f ? O / L : 0.f;
  p.out[static_cast<int64_t>(b) * p.hq * kD + h * kD + d] = float_to_bf16(val);
}

}  // namespace
}  // namespace cs

using namespace cs;

extern "C" int64_t cs_ccpe_decode_workspace_bytes(int32_t batch, int32_t hq, int32_t max_nk,
                                                  int32_t split) {
  if (batch <= 0 || hq <= 0 || max_nk <= 0 || split <= 0) return 0;
  int64_t smax = (static_cast<int64_t>(max_nk) + split - 1) / split;
  int64_t n = static_cast<int64_t>(batch) * hq * smax;
  return n * (8 + 4 + 4 + 4 * kD);
}

extern "C" int cs_ccpe_decode_bf16(const void* q, int64_t q_s_batch, int64_t q_s_head,
                                   int32_t batch, int32_t hq, int32_t hkv, const int32_t* nk,
                                   int32_t max_nk, const cs_kv_source* kv, const float* e,
                                   int32_t max_positions, int32_t split, void* workspace,
                                   void* out, int32_t* flags, void* stream) {
  CS_REQUIRE(q && nk && kv && e && out && flags && workspace, "null arguments");
  CS_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0 && hq / hkv <= kMaxGroup,
             "GQA group must be at most %d", kMaxGroup);
  CS_REQUIRE(max_positions >= 2 && max_positions <= kMaxPos, "max_positions must be in [2, %d]",
             kMaxPos);
  CS_REQUIRE(split >= 64 && split <= kMaxSplit && split % 64 == 0,
             "split must be a multiple of 64 in [64, %d]", kMaxSplit);
  CS_REQUIRE(max_nk >= 1, "max_nk must be positive");
  CS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) % 16) == 0, "workspace must be aligned");
  decode_params p{};
  p.q = static_cast<const uint16_t*>(q);
  p.q_sb = q_s_batch;
  p.q_sh = q_s_head;
  p.batch = batch;
  p.hq = hq;
  p.hkv = hkv;
  p.group = hq / hkv;
  p.nk = nk;
  if (kv->block_table) {
    CS_REQUIRE(kv->cache && kv->block_size > 0 && (reinterpret_cast<uintptr_t>(kv->cache) % 16) == 0 &&
                   kv->s_block % 8 == 0 && kv->s_head % 8 == 0 && kv->s_offset % 8 == 0,
               "paged cache rows must be 16-byte aligned");
    p.kv.cache = static_cast<const uint16_t*>(kv->cache);
    p.kv.s_block = kv->s_block;
    p.kv.s_head = kv->s_head;
    p.kv.s_offset = kv->s_offset;
    p.kv.block_size = kv->block_size;
    p.kv.num_blocks = kv->num_blocks;
    p.kv.block_table = kv->block_table;
    p.kv.bt_stride = kv->bt_stride;
    p.kv.bt_cols = kv->bt_cols;
    p.kv.bs_shift = -1;
    for (int s = 0; s < 31; ++s)
      if ((1 << s) == kv->block_size) p.kv.bs_shift = s;
    CS_REQUIRE(p.kv.bt_cols > 0, "block table needs at least one column");
  } else {
    CS_REQUIRE(kv->k && kv->v && kv->k_s_tok % 8 == 0 && kv->v_s_tok % 8 == 0 &&
                   kv->k_s_head % 8 == 0 && kv->v_s_head % 8 == 0,
               "dense K/V rows must be 16-byte aligned");
    p.kv.k = static_cast<const uint16_t*>(kv->k);
    p.kv.v = static_cast<const uint16_t*>(kv->v);
    p.kv.k_sb = kv->k_s_batch;
    p.kv.k_st = kv->k_s_tok;
    p.kv.k_sh = kv->k_s_head;
    p.kv.v_sb = kv->v_s_batch;
    p.kv.v_st = kv->v_s_tok;
    p.kv.v_sh = kv->v_s_head;
  }
  p.e = e;
  p.npos = max_positions;
  p.split = split;
  p.smax = static_cast<int32_t>((static_cast<int64_t>(max_nk) + split - 1) / split);
  int64_t n = static_cast<int64_t>(batch) * hq * p.smax;
  char* ws = static_cast<char*>(workspace);
  p.tot = reinterpret_cast<double*>(ws);
  p.acc = reinterpret_cast<float*>(ws + n * 8);
  p.mx = p.acc + n * kD;
  p.sm = p.mx + n;
  p.out = static_cast<uint16_t*>(out);
  p.flags = flags;
  if (batch == 0) return CS_OK;
  hipStream_t s = as_stream(stream);
  // split 0 exactly; splits >= 1 speculatively; then exact fixups where the
  // speculation does not hold; then the merge.
  hipLaunchKernelGGL(decode_split_kernel, dim3(1, hkv, batch), dim3(kThreads), 0, s, p, 0);
  if (p.smax > 1) {
    dim3 g(p.smax - 1, hkv, batch);
    switch (p.group) {
      case 1: hipLaunchKernelGGL(decode_spec_kernel<1>, g, dim3(kThreads), 0, s, p); break;
      case 2: hipLaunchKernelGGL(decode_spec_kernel<2>, g, dim3(kThreads), 0, s, p); break;
      case 3: hipLaunchKernelGGL(decode_spec_kernel<3>, g, dim3(kThreads), 0, s, p); break;
      case 4: hipLaunchKernelGGL(decode_spec_kernel<4>, g, dim3(kThreads), 0, s, p); break;
      case 5: hipLaunchKernelGGL(decode_spec_kernel<5>, g, dim3(kThreads), 0, s, p); break;
      case 6: hipLaunchKernelGGL(decode_spec_kernel<6>, g, dim3(kThreads), 0, s, p); break;
      case 7: hipLaunchKernelGGL(decode_spec_kernel<7>, g, dim3(kThreads), 0, s, p); break;
      default: hipLaunchKernelGGL(decode_spec_kernel<8>, g, dim3(kThreads), 0, s, p); break;
    }
    hipLaunchKernelGGL(decode_split_kernel, dim3(p.smax, hkv, batch), dim3(kThreads), 0, s, p, 1);
  }
  hipLaunchKernelGGL(decode_combine_kernel, dim3(batch * hq), dim3(kD), 0, s, p);
  CS_LAUNCH_CHECK("ccpe_decode");
  return CS_OK;
}
