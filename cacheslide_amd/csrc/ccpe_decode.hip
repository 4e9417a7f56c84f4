// CCPE decode attention: one new query row per request at position nk-1 over
// keys 0..nk-1 (position.py:404-560 with q = 1, as called from
// runtime.py:489-508), bf16, head dim 128, K/V from the paged cache.
//
// Split-K with speculative saturation.  The keys of a request are cut into
// splits aligned to the last key (split r covers [nk-(r+1)S, nk-rS)), so the
// right-most split always holds S keys.  Split 0 is computed exactly (carry 0).
// Every other split assumes that the gate mass of the keys to its right is
// already >= P-1, which makes every position in it P-1 and the bias the row
// constant QE[P-1]; it records its own gate total.  A second launch, one
// workgroup per (request, KV head), forms the splits' true carries (sum of the
// totals to their right) from the right-most split until every head's carry
// reaches P-1 -- carries only grow, so the splits that need it are a prefix --
// recomputes those splits exactly, and merges the per-split (max, sum,
// accumulator) triples into the output rows.  Split 0's workgroups lead the
// first launch's grid.
//
// Inside a split each of the 4 wavefronts owns a contiguous quarter of the
// keys and walks it in tiles of 16 keys from the right.  Per tile:
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (keys on M, the GQA heads on N):
//     A: lane (g, n) holds key n, dims 32t + 8g .. +7 (t = 0..3)
//     B: lane (g, n) holds head n, the same dims (heads >= group are zero)
//     C: lane (g, n) holds head n, keys 4g .. 4g+3 of the tile
//   so lane (g, n) keeps an online softmax for head n over the keys of row g.
//   P.V runs on the VALU with packed v_dot2c_f32_bf16: lane (g, x) holds V of
//   keys 4g .. 4g+3, dims 8x .. 8x+7, and the probabilities of head h reach it
//   from lane (g, h) through a DPP row broadcast.
// The next tile's K/V loads are issued before the current tile is consumed.
// Record offsets of the split's keys are resolved once, into LDS, through the
// block table or the per-token slot map (native slot or sidecar row).

#include "common.h"
#include "ccpe_path.h"

#include <mutex>

namespace cs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxGroup = 8;
constexpr int kMaxPos = 256;
constexpr int kMaxSplit = 1024;
constexpr int kTile = 16;
constexpr float kInvSqrtD = 0.08838834764831845f;  // 1/sqrt(128)
constexpr float kLog2e = 1.4426950408889634f;

// Masked keys and keys of invalid blocks read this zero record, so every load
// is issued unconditionally and the compiler can count outstanding loads
// exactly (a load under a branch makes it wait for all of them).
__device__ __attribute__((aligned(16))) uint32_t g_zero_record[kD] = {};

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
  const int64_t* slots;  // per-token slot map (replaces the block table)
  int64_t slots_stride, slots_cols;
  int64_t native_slots;  // num_blocks * block_size
  const uint16_t* side_k;
  const uint16_t* side_v;
  int64_t side_sr, side_sh, side_rows;
};

struct decode_params {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  int32_t batch, hq, hkv, group;
  const int32_t* nk;
  int32_t max_nk;
  kv_addr kv;
  const float* e;
  int32_t npos;
  int32_t split, smax;
  double* tot;         // [B, hq, smax] gate totals
  double* carry;       // [B, hq, smax] gate mass to the right of each split
  float* mx;           // [B, hq, smax] running max (log2 domain)
  float* sm;           // [B, hq, smax] sum of exp2
  float* acc;          // [B, hq, smax, 128]
  uint16_t* out;
  int32_t* flags;
  // when non-null, the call runs only if *gate != 0 (read by every
  // workgroup): the exact fallback of a shared-chunk decode
  const int32_t* gate;
};

__device__ inline int64_t ws_index(const decode_params& p, int b, int h, int r) {
  return (static_cast<int64_t>(b) * p.hq + h) * p.smax + r;
}

template <int G>
struct smem_t {
  // K and V rows of each key of the split (paged), as element offsets from
  // the cache base (sidecar rows and the zero record included, so that every
  // row load is a global-memory load off one kernel argument); entry
  // kMaxSplit and the entries of invalid keys hold the zero record's
  int64_t krow[kMaxSplit + 1];
  int64_t vrow[kMaxSplit + 1];
  union {
    float sc[G][kMaxSplit];       // exact splits: logits
    float wave_o[kWaves][G][kD];  // end of a split: per-wave accumulators
    float wgt[2][kD];             // group finish: split weights of two heads
  } u;
  float qe[G][kMaxPos];  // exact splits: QE = q . E
  float q[G][kD];
  double wave_tot[kWaves][G];
  double carry[G];
  float wave_m[kWaves][G];
  float wave_l[kWaves][G];
  float red[2][2];
  int fix_end;  // group finish: splits 1 .. fix_end-1 are recomputed
};

struct split_ctx {
  int b, kvh, h0, r;
  int64_t lo, hi;
};

// Keys the call may read for request b: its context length, clamped to
// max_nk.  A longer context is flagged (CS_FLAG_CONTEXT_RANGE) and its output
// row is not valid, but every read stays inside the [B, max_nk] slot map and
// the max_nk keys the caller sized its K/V for.
__device__ inline int keys_of(const decode_params& p, int b) {
  const int nk = p.nk[b];
  return nk < p.max_nk ? nk : p.max_nk;
}

__device__ inline bool make_ctx(const decode_params& p, int b, int kvh, int r, split_ctx& c) {
  const int nk = keys_of(p, b);
  int splits = (nk + p.split - 1) / p.split;
  if (splits > p.smax) splits = p.smax;  // the workspace holds smax splits
  if (r >= splits) return false;
  c.b = b;
  c.kvh = kvh;
  c.h0 = kvh * p.group;
  c.r = r;
  c.hi = static_cast<int64_t>(nk) - static_cast<int64_t>(r) * p.split;
  c.lo = c.hi - p.split > 0 ? c.hi - p.split : 0;
  return true;
}

// gate of a logit: sigmoid (position.py:305)
__device__ inline float gate_of(float logit) { return 1.f / (1.f + __expf(-logit)); }

template <int H>
__device__ inline uint32_t dpp_row_bcast(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x150 + H, 0xF, 0xF, false));
}

// value of lane h of this lane's row of 16
__device__ inline uint32_t row_bcast(uint32_t x, int h) {
  switch (h) {
    case 0: return dpp_row_bcast<0>(x);
    case 1: return dpp_row_bcast<1>(x);
    case 2: return dpp_row_bcast<2>(x);
    case 3: return dpp_row_bcast<3>(x);
    case 4: return dpp_row_bcast<4>(x);
    case 5: return dpp_row_bcast<5>(x);
    case 6: return dpp_row_bcast<6>(x);
    default: return dpp_row_bcast<7>(x);
  }
}

__device__ inline float row_bcast_f(float x, int h) {
  return __uint_as_float(row_bcast(__float_as_uint(x), h));
}

__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b),
                                         c, false);
}

__device__ inline const uint16_t* zero_record() {
  return reinterpret_cast<const uint16_t*>(g_zero_record);
}

__device__ inline uint4 ld16(const uint16_t* ptr) { return *reinterpret_cast<const uint4*>(ptr); }

// Element offset of the record of native slot `slot` (block slot / bs, offset
// slot % bs) for KV head kvh.
__device__ inline int64_t native_record(const kv_addr& kv, int64_t blk, int64_t o, int kvh) {
  return blk * kv.s_block + kvh * kv.s_head + o * kv.s_offset;
}

// Resolve the K and V rows of keys [lo, hi) through the block table or the
// slot map (native slot or sidecar row), as element offsets from the cache
// base; invalid keys read the zero record and set `bad`.
template <int G>
__device__ void load_offsets(const decode_params& p, smem_t<G>& s, const split_ctx& c, bool& bad) {
  const int n = static_cast<int>(c.hi - c.lo);
  const int64_t zk = zero_record() - p.kv.cache;
  if (threadIdx.x == 0) {
    s.krow[kMaxSplit] = zk;
    s.vrow[kMaxSplit] = zk + kD;
  }
  if (p.kv.slots) {
    const int64_t* row = p.kv.slots + c.b * p.kv.slots_stride;
    const int64_t sk = p.kv.side_k ? p.kv.side_k - p.kv.cache : 0;
    const int64_t sv = p.kv.side_v ? p.kv.side_v - p.kv.cache : 0;
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const int64_t slot = c.lo + i < p.kv.slots_cols ? row[c.lo + i] : -1;
      int64_t kr = zk, vr = zk + kD;
      if (slot >= 0 && slot < p.kv.native_slots) {
        const int64_t blk = p.kv.bs_shift >= 0 ? (slot >> p.kv.bs_shift) : slot / p.kv.block_size;
        const int64_t o = slot - blk * p.kv.block_size;
        kr = native_record(p.kv, blk, o, c.kvh);
        vr = kr + kD;
      } else if (slot >= p.kv.native_slots && slot - p.kv.native_slots < p.kv.side_rows) {
        const int64_t so = (slot - p.kv.native_slots) * p.kv.side_sr + c.kvh * p.kv.side_sh;
        kr = sk + so;
        vr = sv + so;
      } else {
        bad = true;
      }
      s.krow[i] = kr;
      s.vrow[i] = vr;
    }
    return;
  }
  if (!p.kv.block_table) return;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const int64_t j = c.lo + i;
    const int64_t bi = p.kv.bs_shift >= 0 ? (j >> p.kv.bs_shift) : j / p.kv.block_size;
    int64_t kr = zk, vr = zk + kD;
    int64_t blk = -1;
    if (bi < p.kv.bt_cols) blk = p.kv.block_table[c.b * p.kv.bt_stride + bi];
    if (blk >= 0 && blk < p.kv.num_blocks) {
      const int64_t o =
          p.kv.bs_shift >= 0 ? (j & ((int64_t(1) << p.kv.bs_shift) - 1)) : j % p.kv.block_size;
      kr = native_record(p.kv, blk, o, c.kvh);
      vr = kr + kD;
    } else {
      bad = true;
    }
    s.krow[i] = kr;
    s.vrow[i] = vr;
  }
}

// K / V row of key j, or the zero record when the key is masked (valid is
// false) or its block is invalid.  Valid keys satisfy lo <= j < hi.
template <int G, bool PAGED>
__device__ inline const uint16_t* k_row(const decode_params& p, const smem_t<G>& s,
                                        const split_ctx& c, int64_t j, bool valid) {
  if constexpr (PAGED) {
    return p.kv.cache + s.krow[valid ? static_cast<int>(j - c.lo) : kMaxSplit];
  } else {
    return valid ? p.kv.k + c.b * p.kv.k_sb + j * p.kv.k_st + c.kvh * p.kv.k_sh : zero_record();
  }
}

template <int G, bool PAGED>
__device__ inline const uint16_t* v_row(const decode_params& p, const smem_t<G>& s,
                                        const split_ctx& c, int64_t j, bool valid) {
  if constexpr (PAGED) {
    return p.kv.cache + s.vrow[valid ? static_cast<int>(j - c.lo) : kMaxSplit];
  } else {
    return valid ? p.kv.v + c.b * p.kv.v_sb + j * p.kv.v_st + c.kvh * p.kv.v_sh : zero_record() + kD;
  }
}

struct ktile {
  bf16x8 a[4];
};
struct vtile {
  uint4 v[4];
};

// K operand of tile t0: lane (g, n) loads key t0 + n, dims 32t + 8g .. +7.
// Keys below wlo (tiles past the wave's range included) read zeros.
template <int G, bool PAGED>
__device__ inline void load_k(ktile& kt, const decode_params& p, const smem_t<G>& s,
                              const split_ctx& c, int64_t t0, int64_t wlo, int lane) {
  const int g = lane >> 4, n = lane & 15;
  const int64_t j = t0 + n;
  const uint16_t* row = k_row<G, PAGED>(p, s, c, j, j >= wlo);
#pragma unroll
  for (int t = 0; t < 4; ++t) kt.a[t] = __builtin_bit_cast(bf16x8, ld16(row + 32 * t + 8 * g));
}

// V of tile t0: lane (g, x) loads keys t0 + 4g + v (v = 0..3), dims 8x .. +7.
template <int G, bool PAGED>
__device__ inline void load_v(vtile& vt, const decode_params& p, const smem_t<G>& s,
                              const split_ctx& c, int64_t t0, int64_t wlo, int lane) {
  const int g = lane >> 4, x = lane & 15;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t j = t0 + 4 * g + v;
    vt.v[v] = ld16(v_row<G, PAGED>(p, s, c, j, j >= wlo) + 8 * x);
  }
}

__device__ inline floatx4 qk_tile(const ktile& kt, const bf16x8* qb) {
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt.a[t], qb[t], acc, 0, 0, 0);
  return acc;
}

template <int G>
struct wstate {
  float m, l;      // lane (g, n): head n over the keys of row g (log2 domain)
  float o[G][8];   // lane (g, x): head h, dims 8x..8x+7 over the keys of row g
  double tsum;     // lane (g, n): gate mass of head n over the keys of row g
};

template <int G>
__device__ inline void init_state(wstate<G>& st) {
  st.m = -INFINITY;
  st.l = 0.f;
  st.tsum = 0.0;
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) st.o[h][i] = 0.f;
}

// Online-softmax update with the 4 scores x[v] (log2 domain, -inf when masked)
// of this lane's head, then P.V for the 4 keys of the row.
template <int G>
__device__ inline void accumulate(wstate<G>& st, const float* x, const vtile& vt) {
  float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  mx = fmaxf(mx, st.m);
  float corr = 1.f, pv[4] = {0.f, 0.f, 0.f, 0.f};
  if (mx != -INFINITY) {
    corr = __builtin_amdgcn_exp2f(st.m - mx);
#pragma unroll
    for (int v = 0; v < 4; ++v) pv[v] = __builtin_amdgcn_exp2f(x[v] - mx);
  }
  st.l = st.l * corr + ((pv[0] + pv[1]) + (pv[2] + pv[3]));
  st.m = mx;
  const uint32_t p01 = pack_bf16x2(pv[0], pv[1]);
  const uint32_t p23 = pack_bf16x2(pv[2], pv[3]);
  // (key 4g, key 4g+1) and (key 4g+2, key 4g+3) pairs of each dim
  uint32_t lo01[4], hi01[4], lo23[4], hi23[4];
  const uint32_t w0[4] = {vt.v[0].x, vt.v[0].y, vt.v[0].z, vt.v[0].w};
  const uint32_t w1[4] = {vt.v[1].x, vt.v[1].y, vt.v[1].z, vt.v[1].w};
  const uint32_t w2[4] = {vt.v[2].x, vt.v[2].y, vt.v[2].z, vt.v[2].w};
  const uint32_t w3[4] = {vt.v[3].x, vt.v[3].y, vt.v[3].z, vt.v[3].w};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    lo01[w] = __builtin_amdgcn_perm(w1[w], w0[w], 0x05040100u);
    hi01[w] = __builtin_amdgcn_perm(w1[w], w0[w], 0x07060302u);
    lo23[w] = __builtin_amdgcn_perm(w3[w], w2[w], 0x05040100u);
    hi23[w] = __builtin_amdgcn_perm(w3[w], w2[w], 0x07060302u);
  }
  if (__any(corr != 1.f)) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float ch = row_bcast_f(corr, h);
#pragma unroll
      for (int i = 0; i < 8; ++i) st.o[h][i] *= ch;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint32_t a = row_bcast(p01, h);
    const uint32_t b = row_bcast(p23, h);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      st.o[h][2 * w] = dot2(a, lo01[w], st.o[h][2 * w]);
      st.o[h][2 * w + 1] = dot2(a, hi01[w], st.o[h][2 * w + 1]);
      st.o[h][2 * w] = dot2(b, lo23[w], st.o[h][2 * w]);
      st.o[h][2 * w + 1] = dot2(b, hi23[w], st.o[h][2 * w + 1]);
    }
  }
}

// Merge the 4 rows of the wave and leave the wave's (m, l, o, gate total) in LDS.
template <int G>
__device__ inline void wave_finish(wstate<G>& st, smem_t<G>& s, int wave, int lane) {
  const int g = lane >> 4, x = lane & 15;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mh = row_bcast_f(st.m, h);
    float lh = row_bcast_f(st.l, h);
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const float m2 = __shfl_xor(mh, off, 64);
      const float l2 = __shfl_xor(lh, off, 64);
      const float M = fmaxf(mh, m2);
      const float f1 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mh - M);
      const float f2 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - M);
      lh = lh * f1 + l2 * f2;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o2 = __shfl_xor(st.o[h][i], off, 64);
        st.o[h][i] = st.o[h][i] * f1 + o2 * f2;
      }
      mh = M;
    }
    if (g == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) s.u.wave_o[wave][h][8 * x + i] = st.o[h][i];
    }
    if (lane == h) {
      s.wave_m[wave][h] = mh;
      s.wave_l[wave][h] = lh;
    }
  }
  double t = st.tsum;
  t += __shfl_xor(t, 16, 64);
  t += __shfl_xor(t, 32, 64);
  if (lane < G) s.wave_tot[wave][lane] = t;
}

// Merge the 4 waves and write the split's partial.
template <int G>
__device__ inline void split_finish(const decode_params& p, smem_t<G>& s, const split_ctx& c,
                                    bool write_tot) {
  __syncthreads();
  for (int i = threadIdx.x; i < G * kD; i += kThreads) {
    const int h = i / kD, d = i % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s.wave_m[w][h]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wm = s.wave_m[w][h];
      if (wm == -INFINITY) continue;
      const float f = __builtin_amdgcn_exp2f(wm - M);
      L += s.wave_l[w][h] * f;
      O += s.u.wave_o[w][h][d] * f;
    }
    const int64_t wi = ws_index(p, c.b, c.h0 + h, c.r);
    p.acc[wi * kD + d] = O;
    if (d == 0) {
      p.mx[wi] = M;
      p.sm[wi] = L;
      if (write_tot) {
        double T = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) T += s.wave_tot[w][h];
        p.tot[wi] = T;
      }
    }
  }
}

// Q operand (lane (g, n): head n, dims 32t + 8g .. +7; zero for n >= G).
template <int G>
__device__ inline void load_q(bf16x8* qb, const decode_params& p, const split_ctx& c, int lane) {
  const int g = lane >> 4, n = lane & 15;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint4 u = make_uint4(0, 0, 0, 0);
    if (n < G) u = *reinterpret_cast<const uint4*>(p.q + c.b * p.q_sb + (c.h0 + n) * p.q_sh + 32 * t + 8 * g);
    qb[t] = __builtin_bit_cast(bf16x8, u);
  }
}

// Speculative split: every position is P-1, the bias the constant QE[P-1].
template <int G, bool PAGED>
__device__ void run_spec(const decode_params& p, smem_t<G>& s, const split_ctx& c, bool& bad) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, n = lane & 15;
  if constexpr (PAGED) load_offsets(p, s, c, bad);
  bf16x8 qb[4];
  load_q<G>(qb, p, c, lane);
  // QE[P-1] of head n: lane (g, n) sums its 32 dims, then the 4 rows are added
  float part = 0.f;
  if (n < G) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint4 u = __builtin_bit_cast(uint4, qb[t]);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * t + 8 * g + 2 * i;
        part += __uint_as_float(w[i] << 16) * p.e[d * p.npos + (p.npos - 1)];
        part += __uint_as_float(w[i] & 0xffff0000u) * p.e[(d + 1) * p.npos + (p.npos - 1)];
      }
    }
  }
  part += __shfl_xor(part, 16, 64);
  part += __shfl_xor(part, 32, 64);
  const float bias2 = part * kLog2e;
  const float c_scale = kInvSqrtD * kLog2e;
  __syncthreads();

  const int kw = p.split / kWaves;
  int64_t wlo = c.lo + static_cast<int64_t>(wave) * kw;
  int64_t whi = wlo + kw;
  if (wlo > c.hi) wlo = c.hi;
  if (whi > c.hi) whi = c.hi;
  const int ntiles = static_cast<int>((whi - wlo + kTile - 1) / kTile);

  wstate<G> st;
  init_state(st);
  auto tile = [&](const ktile& kt, const vtile& vt, int64_t t0) {
    const floatx4 sT = qk_tile(kt, qb);
    float x[4], tg = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool valid = n < G && t0 + 4 * g + v >= wlo;
      const float logit = sT[v] * kInvSqrtD;
      tg += valid ? __builtin_amdgcn_rcpf(1.f + __expf(-logit)) : 0.f;
      x[v] = valid ? sT[v] * c_scale + bias2 : -INFINITY;
    }
    st.tsum += static_cast<double>(tg);
    accumulate(st, x, vt);
  };
  // Three tile buffers where registers allow (two waves per SIMD): the loads
  // of the next two tiles are in flight while the current one is consumed;
  // two buffers otherwise.  Loads past the wave's range read the zero record
  // and are not consumed.
  constexpr bool kTriple = PAGED ? G <= 8 : G <= 6;
  ktile ka, kb, kc;
  vtile va, vb, vc;
  load_k<G, PAGED>(ka, p, s, c, whi - kTile, wlo, lane);
  load_v<G, PAGED>(va, p, s, c, whi - kTile, wlo, lane);
  if constexpr (kTriple) {
    load_k<G, PAGED>(kb, p, s, c, whi - 2 * kTile, wlo, lane);
    load_v<G, PAGED>(vb, p, s, c, whi - 2 * kTile, wlo, lane);
    for (int i = 0; i < ntiles; i += 3) {
      const int64_t t0 = whi - static_cast<int64_t>(i + 1) * kTile;
      load_k<G, PAGED>(kc, p, s, c, t0 - 2 * kTile, wlo, lane);
      load_v<G, PAGED>(vc, p, s, c, t0 - 2 * kTile, wlo, lane);
      tile(ka, va, t0);
      if (i + 1 >= ntiles) break;
      load_k<G, PAGED>(ka, p, s, c, t0 - 3 * kTile, wlo, lane);
      load_v<G, PAGED>(va, p, s, c, t0 - 3 * kTile, wlo, lane);
      tile(kb, vb, t0 - kTile);
      if (i + 2 >= ntiles) break;
      load_k<G, PAGED>(kb, p, s, c, t0 - 4 * kTile, wlo, lane);
      load_v<G, PAGED>(vb, p, s, c, t0 - 4 * kTile, wlo, lane);
      tile(kc, vc, t0 - 2 * kTile);
    }
  } else {
    for (int i = 0; i < ntiles; i += 2) {
      const int64_t t0 = whi - static_cast<int64_t>(i + 1) * kTile;
      load_k<G, PAGED>(kb, p, s, c, t0 - kTile, wlo, lane);
      load_v<G, PAGED>(vb, p, s, c, t0 - kTile, wlo, lane);
      tile(ka, va, t0);
      load_k<G, PAGED>(ka, p, s, c, t0 - 2 * kTile, wlo, lane);
      load_v<G, PAGED>(va, p, s, c, t0 - 2 * kTile, wlo, lane);
      tile(kb, vb, t0 - kTile);
    }
  }
  __syncthreads();
  wave_finish(st, s, wave, lane);
  split_finish(p, s, c, true);
}

// Exact split with the given carry per head (s.carry): positions from the
// gate suffix sums (fp64), bias by interpolation in the QE table.
template <int G, bool PAGED>
__device__ void run_exact(const decode_params& p, smem_t<G>& s, const split_ctx& c, bool write_tot,
                          bool& bad) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, n = lane & 15;
  if constexpr (PAGED) load_offsets(p, s, c, bad);
  bf16x8 qb[4];
  load_q<G>(qb, p, c, lane);
  for (int i = tid; i < G * kD; i += kThreads) {
    const int h = i / kD, d = i % kD;
    s.q[h][d] = bf16_to_float(p.q[c.b * p.q_sb + (c.h0 + h) * p.q_sh + d]);
  }
  __syncthreads();
  for (int i = tid; i < G * p.npos; i += kThreads) {
    const int h = i / p.npos, pp = i % p.npos;
    float a = 0.f;
    for (int d = 0; d < kD; ++d) a += s.q[h][d] * p.e[d * p.npos + pp];
    s.qe[h][pp] = a;
  }

  const int kw = p.split / kWaves;
  int64_t wlo = c.lo + static_cast<int64_t>(wave) * kw;
  int64_t whi = wlo + kw;
  if (wlo > c.hi) wlo = c.hi;
  if (whi > c.hi) whi = c.hi;
  const int ntiles = static_cast<int>((whi - wlo + kTile - 1) / kTile);

  // ---- pass 1: logits into LDS, gate totals per wave -----------------------
  double gsum = 0.0;
  auto ktile_pass = [&](const ktile& kt, int64_t t0) {
    const floatx4 sT = qk_tile(kt, qb);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t j = t0 + 4 * g + v;
      if (n < G && j >= wlo) {
        const float logit = sT[v] * kInvSqrtD;
        s.u.sc[n][j - c.lo] = logit;
        gsum += static_cast<double>(gate_of(logit));
      }
    }
  };
  {
    ktile ka, kb;
    load_k<G, PAGED>(ka, p, s, c, whi - kTile, wlo, lane);
    for (int i = 0; i < ntiles; i += 2) {
      const int64_t t0 = whi - static_cast<int64_t>(i + 1) * kTile;
      load_k<G, PAGED>(kb, p, s, c, t0 - kTile, wlo, lane);
      ktile_pass(ka, t0);
      load_k<G, PAGED>(ka, p, s, c, t0 - 2 * kTile, wlo, lane);
      ktile_pass(kb, t0 - kTile);
    }
  }
  {
    double t = gsum;
    t += __shfl_xor(t, 16, 64);
    t += __shfl_xor(t, 32, 64);
    if (lane < G) s.wave_tot[wave][lane] = t;
  }
  __syncthreads();

  // ---- pass 2: positions, scores, P.V ---------------------------------------
  const float top = static_cast<float>(p.npos - 1);
  double carry = 0.0;
  if (n < G) {
    carry = s.carry[n];
    for (int w = kWaves - 1; w > wave; --w) carry += s.wave_tot[w][n];
  }
  wstate<G> st;
  init_state(st);
  auto vtile_pass = [&](const vtile& vt, int64_t t0) {
    float lg[4];
    double gt[4];
    bool valid[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t j = t0 + 4 * g + v;
      valid[v] = n < G && j >= wlo;
      lg[v] = valid[v] ? s.u.sc[n][j - c.lo] : 0.f;
      gt[v] = valid[v] ? static_cast<double>(gate_of(lg[v])) : 0.0;
    }
    // suffix sums in descending key order: within the row, then over rows
    double sfx[4];
    sfx[3] = gt[3];
    sfx[2] = sfx[3] + gt[2];
    sfx[1] = sfx[2] + gt[1];
    sfx[0] = sfx[1] + gt[0];
    const double r1 = __shfl(sfx[0], lane + 16, 64);
    const double r2 = __shfl(sfx[0], lane + 32, 64);
    const double r3 = __shfl(sfx[0], lane + 48, 64);
    double above = 0.0;
    if (g < 3) above += r1;
    if (g < 2) above += r2;
    if (g < 1) above += r3;
    const double total = __shfl(above + sfx[0], n, 64);  // lane (0, n): whole tile
    float x[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float pos = static_cast<float>(carry + above + sfx[v]);
      pos = pos < top ? pos : top;
      pos = pos > 0.f ? pos : 0.f;  // also maps NaN to 0: table reads stay in range
      const float fl = floorf(pos);
      const int lo_i = static_cast<int>(fl);
      const int hi_i = lo_i + 1 < p.npos - 1 ? lo_i + 1 : p.npos - 1;
      const int hh = n < G ? n : 0;
      const float bias = s.qe[hh][lo_i] + (pos - fl) * (s.qe[hh][hi_i] - s.qe[hh][lo_i]);
      x[v] = valid[v] ? (lg[v] + bias) * kLog2e : -INFINITY;
    }
    carry += total;
    accumulate(st, x, vt);
  };
  {
    vtile va, vb;
    load_v<G, PAGED>(va, p, s, c, whi - kTile, wlo, lane);
    for (int i = 0; i < ntiles; i += 2) {
      const int64_t t0 = whi - static_cast<int64_t>(i + 1) * kTile;
      load_v<G, PAGED>(vb, p, s, c, t0 - kTile, wlo, lane);
      vtile_pass(va, t0);
      load_v<G, PAGED>(va, p, s, c, t0 - 2 * kTile, wlo, lane);
      vtile_pass(vb, t0 - kTile);
    }
  }
  __syncthreads();  // the per-wave accumulators overwrite the logits
  st.tsum = gsum;    // wave_finish publishes the pass-1 gate totals again
  wave_finish(st, s, wave, lane);
  split_finish(p, s, c, write_tot);
}

// ---- finish of one (request, KV head) group ---------------------------------

// Carries of splits 1, 2, ... (sum of the split totals to their right, fp64,
// accumulated from the right-most split) into p.carry, 64 splits at a time
// (wave 0, lane i: the total of split base+i, the carry of split base+i+1),
// up to the first split at which every head's carry has reached P-1;
// s.fix_end is that split (or `splits`).  Gate totals are sums of sigmoids, so
// carries never decrease along the splits and no later split needs
// recomputing.
template <int G>
__device__ void plan_group(const decode_params& p, smem_t<G>& s, int b, int h0, int splits) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  const double top = static_cast<double>(p.npos - 1);
  double carry_in[G];
#pragma unroll
  for (int h = 0; h < G; ++h) carry_in[h] = 0.0;
  int fix_end = splits > 1 ? splits : 1;
  for (int base = 0; base + 1 < splits; base += 64) {
    const int r = base + lane;
    const bool has_next = r + 1 < splits;
    double v[G];
#pragma unroll
    for (int h = 0; h < G; ++h) v[h] = has_next ? p.tot[ws_index(p, b, h0 + h, r)] : 0.0;
    bool below = false;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      double x = v[h];  // inclusive scan over the wave
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const double y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
      }
      const double carry = carry_in[h] + x;
      if (has_next) {
        p.carry[ws_index(p, b, h0 + h, r + 1)] = carry;
        below |= carry < top;  // false for NaN
      }
      carry_in[h] += __shfl(x, 63, 64);
    }
    const unsigned long long done = __ballot(has_next && !below);
    if (done) {
      fix_end = base + __builtin_ctzll(done) + 1;
      break;
    }
  }
  if (lane == 0) s.fix_end = fix_end;
}

// Exact recomputation of splits 1 .. s.fix_end-1, one after another.
template <int G, bool PAGED>
__device__ void fixup_group(const decode_params& p, smem_t<G>& s, int b, int kvh, bool& bad) {
  // read after the barrier that follows plan_group; the same in every lane
  const int fix_end = __builtin_amdgcn_readfirstlane(s.fix_end);
  for (int r = 1; r < fix_end; ++r) {
    split_ctx c;
    make_ctx(p, b, kvh, r, c);
    if (threadIdx.x < G) s.carry[threadIdx.x] = p.carry[ws_index(p, b, c.h0 + threadIdx.x, r)];
    __syncthreads();
    run_exact<G, PAGED>(p, s, c, false, bad);
    __syncthreads();
  }
}

// Merge of the split partials of two query heads, threads 0..127 for head ha
// and 128..255 for head hb (hb < 0: those threads only join the barriers);
// thread d of a half owns output dim d, split weights are formed 128 at a time.
template <int G>
__device__ void combine_pair(const decode_params& p, smem_t<G>& s, int b, int ha, int hb,
                             int splits) {
  const int half = threadIdx.x >> 7, d = threadIdx.x & (kD - 1);
  const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) & 1;
  const int h = half ? hb : ha;
  const bool live = h >= 0;
  const int64_t w0 = ws_index(p, b, live ? h : ha, 0);
  float* wgt = s.u.wgt[half];
  // the first 128 splits' max and sum stay in registers for the weights below
  float m_first = -INFINITY, l_first = 0.f;
  if (live && d < splits) {
    m_first = p.mx[w0 + d];
    l_first = p.sm[w0 + d];
  }
  float M = m_first;
  if (live)
    for (int r = d + kD; r < splits; r += kD) M = fmaxf(M, p.mx[w0 + r]);
  M = wave_max(M);
  if (lane == 0) s.red[half][wave] = M;
  __syncthreads();
  M = fmaxf(s.red[half][0], s.red[half][1]);
  __syncthreads();
  float L = 0.f, O = 0.f;
  for (int base = 0; base < splits; base += kD) {
    const int r = base + d;
    float f = 0.f;
    if (live && r < splits) {
      const float m = base == 0 ? m_first : p.mx[w0 + r];
      const float l = base == 0 ? l_first : p.sm[w0 + r];
      f = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
      L += l * f;
    }
    wgt[d] = f;
    __syncthreads();
    const int n = splits - base < kD ? splits - base : kD;
    if (live) {
      const float* acc = p.acc + (w0 + base) * kD + d;
      int i = 0;
      // 16 partials in flight per thread: the merge is bound by load latency
      for (; i + 16 <= n; i += 16) {
        float a[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) a[j] = acc[(i + j) * kD];
#pragma unroll
        for (int j = 0; j < 16; j += 4)
          O += wgt[i + j] * a[j] + wgt[i + j + 1] * a[j + 1] + wgt[i + j + 2] * a[j + 2] +
               wgt[i + j + 3] * a[j + 3];
      }
      for (; i + 4 <= n; i += 4) {
        const float a0 = acc[(i + 0) * kD], a1 = acc[(i + 1) * kD];
        const float a2 = acc[(i + 2) * kD], a3 = acc[(i + 3) * kD];
        O += wgt[i] * a0 + wgt[i + 1] * a1 + wgt[i + 2] * a2 + wgt[i + 3] * a3;
      }
      for (; i < n; ++i) O += wgt[i] * acc[i * kD];
    }
    __syncthreads();
  }
  L = wave_sum(L);
  if (lane == 0) s.red[half][wave] = L;
  __syncthreads();
  L = s.red[half][0] + s.red[half][1];
  __syncthreads();
  if (live) p.out[static_cast<int64_t>(b) * p.hq * kD + h * kD + d] = float_to_bf16(L > 0.f ? O / L : 0.f);
}

// The finish of a group of at most 16 * NCH splits when no split needs
// recomputing.  Every split partial of the group's heads is loaded before the
// carries are planned, so the whole merge waits for one round of loads, not
// one per head pair and split chunk: thread (half, d) owns output dim d of
// heads half, half + 2, ..., holds the accumulators of all their splits in
// registers (indices past the last split repeat the last one, so every load
// is issued unconditionally; their weights are 0), and lane r of each wave
// holds split r's max and sum, whose weight reaches every lane through
// v_readlane.  Returns false, with the plan in s.fix_end and nothing
// written, when some split must be recomputed first; the value is the same
// in every thread.
template <int G>
constexpr int fast_chunks() { return (G + 1) / 2 > 2 ? 2 : 4; }

template <int G, int NCH>
__device__ bool merge_fast(const decode_params& p, smem_t<G>& s, int b, int h0, int splits) {
  constexpr int NH = (G + 1) / 2;
  constexpr int R = 16 * NCH;
  static_assert(R <= 64 && NH * R <= 128, "partials held per thread");
  const int half = threadIdx.x >> 7, d = threadIdx.x & (kD - 1), lane = threadIdx.x & 63;
  const int last = splits - 1;
  float a[NH][R], mv[NH], lv[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    // a thread without a j-th head reads head 0's partials and drops them
    const int h = half + 2 * j < G ? half + 2 * j : 0;
    const int64_t w0 = ws_index(p, b, h0 + h, 0);
    const float* acc = p.acc + w0 * kD + d;
#pragma unroll
    for (int r = 0; r < R; ++r) a[j][r] = acc[static_cast<int64_t>(r < last ? r : last) * kD];
    const int rl = lane < last ? lane : last;
    mv[j] = p.mx[w0 + rl];
    lv[j] = p.sm[w0 + rl];
  }
  plan_group<G>(p, s, b, h0, splits);
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(s.fix_end) > 1) return false;
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    const int h = half + 2 * j;
    const float m = lane < splits ? mv[j] : -INFINITY;
    const float M = wave_max(m);
    const float f = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    const float L = wave_sum(lane < splits ? lv[j] * f : 0.f);
    const int fb = __float_as_int(f);
    float O = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) O += __int_as_float(__builtin_amdgcn_readlane(fb, r)) * a[j][r];
    if (h < G)
      p.out[static_cast<int64_t>(b) * p.hq * kD + (h0 + h) * kD + d] = float_to_bf16(L > 0.f ? O / L : 0.f);
  }
  return true;
}

template <int G>
__device__ bool merge_fast_any(const decode_params& p, smem_t<G>& s, int b, int h0, int splits) {
  switch ((splits + 15) >> 4) {
    case 1: return merge_fast<G, 1>(p, s, b, h0, splits);
    case 2: return merge_fast<G, 2>(p, s, b, h0, splits);
    case 3: if constexpr (fast_chunks<G>() >= 3) return merge_fast<G, 3>(p, s, b, h0, splits); break;
    case 4: if constexpr (fast_chunks<G>() >= 4) return merge_fast<G, 4>(p, s, b, h0, splits); break;
    default: break;
  }
  // no key, or more splits than the registers hold: plan only
  plan_group<G>(p, s, b, h0, splits);
  __syncthreads();
  return false;
}

// Split 0 of every (request, KV head) exactly, then the speculative splits;
// the grid is ordered split-major so the exact workgroups start first.
template <int G, bool PAGED>
__global__ void __launch_bounds__(kThreads) decode_main_kernel(decode_params p) {
  __shared__ smem_t<G> s;
  if (p.gate != nullptr && __builtin_amdgcn_readfirstlane(*p.gate) == 0) return;  // before any barrier
  const int per_r = p.hkv * p.batch;
  const int id = blockIdx.x;
  const int r = id / per_r, rem = id % per_r;
  const int b = rem / p.hkv, kvh = rem % p.hkv;
  if (r == 0 && kvh == 0 && threadIdx.x == 0) {
    const int nk = p.nk[b];
    if (nk < 1) atomicOr(p.flags, CS_FLAG_NO_KEY);
    if (nk > p.max_nk) atomicOr(p.flags, CS_FLAG_CONTEXT_RANGE);
  }
  split_ctx c;
  if (!make_ctx(p, b, kvh, r, c)) return;
  bool bad = false;
  if (r == 0) {
    if (threadIdx.x < G) s.carry[threadIdx.x] = 0.0;
    run_exact<G, PAGED>(p, s, c, true, bad);
  } else {
    run_spec<G, PAGED>(p, s, c, bad);
  }
  if (bad) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
}

// One workgroup per (request, KV head): carries, recomputation of the splits
// whose carry is below P-1, and the merge into the output rows.
template <int G, bool PAGED>
__global__ void __launch_bounds__(kThreads) decode_finish_kernel(decode_params p) {
  __shared__ smem_t<G> s;
  if (p.gate != nullptr && __builtin_amdgcn_readfirstlane(*p.gate) == 0) return;  // before any barrier
  const int b = blockIdx.x / p.hkv, kvh = blockIdx.x % p.hkv;
  const int h0 = kvh * G;
  int splits = (keys_of(p, b) + p.split - 1) / p.split;
  if (splits > p.smax) splits = p.smax;
  if (splits < 0) splits = 0;  // no key: zero rows (the call is flagged)
  bool bad = false;
  if (merge_fast_any<G>(p, s, b, h0, splits)) return;
  fixup_group<G, PAGED>(p, s, b, kvh, bad);
  for (int h = 0; h < G; h += 2) combine_pair<G>(p, s, b, h0 + h, h + 1 < G ? h0 + h + 1 : -1, splits);
  if (bad) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
}

template <int G, bool PAGED>
void launch_split_kernels(const decode_params& p, hipStream_t s) {
  const int64_t main_grid = static_cast<int64_t>(p.smax) * p.hkv * p.batch;
  hipLaunchKernelGGL((decode_main_kernel<G, PAGED>), dim3(static_cast<uint32_t>(main_grid)),
                     dim3(kThreads), 0, s, p);
  hipLaunchKernelGGL((decode_finish_kernel<G, PAGED>), dim3(static_cast<uint32_t>(p.hkv * p.batch)),
                     dim3(kThreads), 0, s, p);
}

template <int G>
void launch_group(const decode_params& p, hipStream_t s) {
  if (p.kv.block_table || p.kv.slots)
    launch_split_kernels<G, true>(p, s);
  else
    launch_split_kernels<G, false>(p, s);
}

}  // namespace
}  // namespace cs

using namespace cs;

extern "C" int64_t cs_ccpe_decode_workspace_bytes(int32_t batch, int32_t hq, int32_t max_nk,
                                                  int32_t split) {
  if (batch <= 0 || hq <= 0 || max_nk <= 0 || split <= 0) return 0;
  const int64_t smax = (static_cast<int64_t>(max_nk) + split - 1) / split;
  const int64_t n = static_cast<int64_t>(batch) * hq * smax;
  // tot, carry (f64) | acc (f32 x 128) | mx, sm (f32)
  return n * (8 + 8 + 4 * kD + 4 + 4);
}

namespace {

// Validate the arguments of a decode call and fill its parameters; the
// workspace pointers are set by the caller.
int prepare_decode(const void* q, int64_t q_s_batch, int64_t q_s_head, int32_t batch, int32_t hq,
                   int32_t hkv, const int32_t* nk, int32_t max_nk, const cs_kv_source* kv,
                   const float* e, int32_t max_positions, int32_t split, void* out, int32_t* flags,
                   decode_params* pp) {
  CS_REQUIRE(q && nk && kv && e && out && flags, "null arguments");
  CS_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0 && hq / hkv <= kMaxGroup,
             "GQA group must be at most %d", kMaxGroup);
  CS_REQUIRE(max_positions >= 2 && max_positions <= kMaxPos, "max_positions must be in [2, %d]",
             kMaxPos);
  CS_REQUIRE(split >= 64 && split <= kMaxSplit && split % 64 == 0,
             "split must be a multiple of 64 in [64, %d]", kMaxSplit);
  CS_REQUIRE(max_nk >= 1, "max_nk must be positive");
  CS_REQUIRE(batch >= 0, "batch must be non-negative");
  CS_REQUIRE((reinterpret_cast<uintptr_t>(q) % 16) == 0 && q_s_batch % 8 == 0 && q_s_head % 8 == 0,
             "query rows must be 16-byte aligned");
  const int64_t smax = (static_cast<int64_t>(max_nk) + split - 1) / split;
  CS_REQUIRE(smax * hkv * batch < (int64_t(1) << 31), "too many splits for one launch");
  decode_params p{};
  p.q = static_cast<const uint16_t*>(q);
  p.q_sb = q_s_batch;
  p.q_sh = q_s_head;
  p.batch = batch;
  p.hq = hq;
  p.hkv = hkv;
  p.group = hq / hkv;
  p.nk = nk;
  p.max_nk = max_nk;
  if (kv->block_table || kv->slots) {
    CS_REQUIRE(kv->cache && kv->block_size > 0 && kv->num_blocks >= 0 &&
                   (reinterpret_cast<uintptr_t>(kv->cache) % 16) == 0 && kv->s_block % 8 == 0 &&
                   kv->s_head % 8 == 0 && kv->s_offset % 8 == 0,
               "paged cache rows must be 16-byte aligned");
    p.kv.cache = static_cast<const uint16_t*>(kv->cache);
    p.kv.s_block = kv->s_block;
    p.kv.s_head = kv->s_head;
    p.kv.s_offset = kv->s_offset;
    p.kv.block_size = kv->block_size;
    p.kv.num_blocks = kv->num_blocks;
    p.kv.bs_shift = -1;
    for (int sh = 0; sh < 31; ++sh)
      if ((1 << sh) == kv->block_size) p.kv.bs_shift = sh;
    if (kv->slots) {
      CS_REQUIRE(kv->slots_stride >= 0, "slot map stride must be non-negative");
      CS_REQUIRE(kv->slots_cols > 0, "slot map needs at least one column");
      CS_REQUIRE(kv->side_rows >= 0, "side_rows must be non-negative");
      if (kv->side_rows > 0)
        CS_REQUIRE(kv->side_k && kv->side_v && (reinterpret_cast<uintptr_t>(kv->side_k) % 16) == 0 &&
                       (reinterpret_cast<uintptr_t>(kv->side_v) % 16) == 0 &&
                       kv->side_s_row % 8 == 0 && kv->side_s_head % 8 == 0 &&
                       kv->side_s_row >= 0 && kv->side_s_head >= 0,
                   "sidecar rows must be 16-byte aligned");
      p.kv.slots = kv->slots;
      p.kv.slots_stride = kv->slots_stride;
      p.kv.slots_cols = kv->slots_cols;
      p.kv.native_slots = kv->num_blocks * kv->block_size;
      p.kv.side_k = static_cast<const uint16_t*>(kv->side_k);
      p.kv.side_v = static_cast<const uint16_t*>(kv->side_v);
      p.kv.side_sr = kv->side_s_row;
      p.kv.side_sh = kv->side_s_head;
      p.kv.side_rows = kv->side_rows;
    } else {
      p.kv.block_table = kv->block_table;
      p.kv.bt_stride = kv->bt_stride;
      p.kv.bt_cols = kv->bt_cols;
      CS_REQUIRE(p.kv.bt_cols > 0, "block table needs at least one column");
    }
  } else {
    CS_REQUIRE(kv->k && kv->v && (reinterpret_cast<uintptr_t>(kv->k) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(kv->v) % 16) == 0 && kv->k_s_tok % 8 == 0 &&
                   kv->v_s_tok % 8 == 0 && kv->k_s_head % 8 == 0 && kv->v_s_head % 8 == 0 &&
                   kv->k_s_batch % 8 == 0 && kv->v_s_batch % 8 == 0,
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
  p.smax = static_cast<int32_t>(smax);
  p.out = static_cast<uint16_t*>(out);
  p.flags = flags;
  *pp = p;
  return CS_OK;
}

// Carve the workspace of a prepared call and launch its kernels.
int launch_decode(decode_params& p, void* workspace, void* stream) {
  const int64_t n = static_cast<int64_t>(p.batch) * p.hq * p.smax;
  char* ws = static_cast<char*>(workspace);
  p.tot = reinterpret_cast<double*>(ws);
  p.carry = p.tot + n;
  p.acc = reinterpret_cast<float*>(ws + n * 16);
  p.mx = p.acc + n * kD;
  p.sm = p.mx + n;
  if (p.batch == 0) return CS_OK;
  hipStream_t s = as_stream(stream);
  switch (p.group) {
    case 1: launch_group<1>(p, s); break;
    case 2: launch_group<2>(p, s); break;
    case 3: launch_group<3>(p, s); break;
    case 4: launch_group<4>(p, s); break;
    case 5: launch_group<5>(p, s); break;
    case 6: launch_group<6>(p, s); break;
    case 7: launch_group<7>(p, s); break;
    default: launch_group<8>(p, s); break;
  }
  CS_LAUNCH_CHECK("ccpe_decode");
  return CS_OK;
}

// Workspace of cs_ccpe_decode_bf16_noalloc: a static device array, one copy
// per GPU, alive until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host it names a stand-in, not device memory): it
// uses the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[CS_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on the first
// call on that device.
int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("hipGetDevice: %s", hipGetErrorString(err));
    return CS_ELAUNCH;
  }
  CS_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal %d out of range", dev);
  if (stream != nullptr) {
    int sdev = -1;
    err = hipStreamGetDevice(as_stream(stream), &sdev);
    if (err != hipSuccess) {
      set_error("hipStreamGetDevice: %s", hipGetErrorString(err));
      return CS_ELAUNCH;
    }
    CS_REQUIRE(sdev == dev, "the stream belongs to device %d but device %d is current", sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch): %s", hipGetErrorString(err));
      return CS_ELAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CS_OK;
}

}  // namespace

extern "C" int cs_ccpe_decode_bf16_noalloc(const void* q, int64_t q_s_batch, int64_t q_s_head,
                                           int32_t batch, int32_t hq, int32_t hkv,
                                           const int32_t* nk, int32_t max_nk,
                                           const cs_kv_source* kv, const float* e,
                                           int32_t max_positions, int32_t split, void* out,
                                           int32_t* flags, void* stream) {
  decode_params p{};
  const int st = prepare_decode(q, q_s_batch, q_s_head, batch, hq, hkv, nk, max_nk, kv, e,
                                max_positions, split, out, flags, &p);
  if (st) return st;
  const int64_t need = cs_ccpe_decode_workspace_bytes(batch, hq, max_nk, split);
  CS_REQUIRE(need <= CS_DECODE_SCRATCH_BYTES,
             "the call needs %lld bytes of decode workspace; the static scratch holds %lld "
             "(lower batch x heads x ceil(max_nk / split), or use cs_ccpe_decode_bf16)",
             static_cast<long long>(need), static_cast<long long>(CS_DECODE_SCRATCH_BYTES));
  if (batch == 0) return CS_OK;
  void* ws = nullptr;
  const int sst = scratch_address(stream, &ws);
  if (sst) return sst;
  // every workspace field the kernels read is written earlier in the same call,
  // so the previous call's contents need no clearing
  return launch_decode(p, ws, stream);
}

extern "C" int cs_ccpe_decode_bf16(const void* q, int64_t q_s_batch, int64_t q_s_head,
                                   int32_t batch, int32_t hq, int32_t hkv, const int32_t* nk,
                                   int32_t max_nk, const cs_kv_source* kv, const float* e,
                                   int32_t max_positions, int32_t split, void* workspace,
                                   int64_t workspace_bytes, void* out, int32_t* flags,
                                   void* stream) {
  decode_params p{};
  const int st = prepare_decode(q, q_s_batch, q_s_head, batch, hq, hkv, nk, max_nk, kv, e,
                                max_positions, split, out, flags, &p);
  if (st) return st;
  const int64_t need = cs_ccpe_decode_workspace_bytes(batch, hq, max_nk, split);
  CS_REQUIRE(workspace != nullptr || batch == 0, "null workspace");
  CS_REQUIRE(workspace_bytes >= need, "decode workspace holds %lld bytes, the call needs %lld",
             static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  CS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) % 16) == 0, "workspace must be aligned");
  return launch_decode(p, workspace, stream);
}

// ---- decode over shared runs of blocks ---------------------------------------
namespace {

// One workgroup per (request, KV head), one thread per (head of the group,
// dim): the tail state and the head_items run states of each head combined
// against their common maximum (raw scores q.k, shifted bias: the two
// launches share the convention).  Thread t of a head reads the (max, sum)
// of state t - 1 (state -1: the tail), 128 at a time, so the maximum and the
// weights come from LDS reductions; the output loads of a thread are then
// independent of each other.  A head whose tail gate mass is below P-1 (or
// NaN) sets *gate: the caller's exact fallback then runs.
__global__ void __launch_bounds__(1024) shared_merge_kernel(const float* tail_o, const float* tail_ml,
                                                            const float* head_o, const float* head_ml,
                                                            int32_t batch, int32_t hq, int32_t group,
                                                            int32_t items, float top, uint16_t* out,
                                                            int32_t* gate) {
  __shared__ float wgt[8][kD];
  __shared__ float red[8][2];
  const int b = blockIdx.x / (hq / group), kvh = blockIdx.x % (hq / group);
  const int hl = threadIdx.x / kD, d = threadIdx.x % kD;  // blockDim = group * 128
  const int lane = threadIdx.x & 63, half = d >> 6;
  const int h = kvh * group + hl;
  constexpr float kC = kInvSqrtD * kLog2e;
  const int64_t th = static_cast<int64_t>(b) * hq + h;  // tail state [B, 1, Hq]
  auto state = [&](int i) -> int64_t { return (static_cast<int64_t>(i) * batch + b) * hq + h; };
  if (d == 0 && !(tail_ml[3 * th + 2] >= top)) atomicOr(gate, 1);
  // the common maximum
  float mx = -INFINITY;
  for (int t = d; t <= items; t += kD) mx = fmaxf(mx, t == 0 ? tail_ml[3 * th] : head_ml[3 * state(t - 1)]);
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) red[hl][half] = mx;
  __syncthreads();
  mx = fmaxf(red[hl][0], red[hl][1]);
  __syncthreads();
  float l_all = 0.f, o = 0.f;
  for (int t0 = 0; t0 <= items; t0 += kD) {
    // weights of states t0 - 1 .. t0 + 126
    float w = 0.f, lw = 0.f;
    const int t = t0 + d;
    if (t <= items && mx != -INFINITY) {
      const float* ml = t == 0 ? tail_ml + 3 * th : head_ml + 3 * state(t - 1);
      w = ml[0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((ml[0] - mx) * kC);
      lw = w * ml[1];
    }
    wgt[hl][d] = w;
    for (int off = 32; off > 0; off >>= 1) lw += __shfl_xor(lw, off, 64);
    if (lane == 0) red[hl][half] = lw;
    __syncthreads();
    l_all += red[hl][0] + red[hl][1];
    const int n = items + 1 - t0 < kD ? items + 1 - t0 : kD;
    int j = 0;
    for (; j + 16 <= n; j += 16) {
      float a[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int s2 = t0 + j + u;
        a[u] = s2 == 0 ? tail_o[th * kD + d] : head_o[state(s2 - 1) * kD + d];
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) o += wgt[hl][j + u] * a[u];
    }
    for (; j < n; ++j) {
      const int s2 = t0 + j;
      o += wgt[hl][j] * (s2 == 0 ? tail_o[th * kD + d] : head_o[state(s2 - 1) * kD + d]);
    }
    __syncthreads();
  }
  out[th * kD + d] = float_to_bf16(l_all > 0.f ? o / l_all : 0.f);
}

struct shared_ws {
  float* head_o;
  float* head_ml;
  float* tail_o;
  float* tail_ml;
  int32_t* gate;
  void* decode;
  int64_t decode_bytes;
  int64_t bytes;
};

shared_ws carve_shared(char* base, int32_t batch, int32_t hq, int32_t items, int32_t max_nk, int32_t split) {
  shared_ws w{};
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* at = base ? base + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  const int64_t rows_h = static_cast<int64_t>(items) * batch * hq, rows_t = static_cast<int64_t>(batch) * hq;
  w.head_o = reinterpret_cast<float*>(take(4 * rows_h * kD));
  w.head_ml = reinterpret_cast<float*>(take(4 * rows_h * 3));
  w.tail_o = reinterpret_cast<float*>(take(4 * rows_t * kD));
  w.tail_ml = reinterpret_cast<float*>(take(4 * rows_t * 3));
  w.gate = reinterpret_cast<int32_t*>(take(4));
  w.decode_bytes = cs_ccpe_decode_workspace_bytes(batch, hq, max_nk, split);
  w.decode = take(w.decode_bytes);
  w.bytes = off;
  return w;
}

}  // namespace

extern "C" int64_t cs_ccpe_decode_shared_workspace_bytes(int32_t batch, int32_t hq, int32_t head_items,
                                                         int32_t max_nk, int32_t split) {
  if (batch < 0 || hq <= 0 || head_items < 0 || max_nk < 0 || split <= 0) return 0;
  return carve_shared(nullptr, batch, hq, head_items, max_nk, split).bytes;
}

extern "C" int cs_ccpe_decode_shared_bf16(const cs_decode_shared_args* a, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  CS_REQUIRE(a != nullptr && a->kv != nullptr, "null arguments");
  CS_REQUIRE(a->kv->block_table != nullptr && a->kv->slots == nullptr,
             "the shared-run decode reads the cache through block tables");
  CS_REQUIRE(a->head_table && a->head_nk && a->head_qpos && a->tail_table && a->tail_nk && a->tail_qpos,
             "null shared-run arguments");
  CS_REQUIRE(a->head_items >= 0 && a->head_blocks > 0 && a->tail_cols > 0 && a->tail_stride >= a->tail_cols,
             "bad shared-run shapes");
  CS_REQUIRE(a->batch >= 0 && a->hq > 0 && a->hkv > 0 && a->hq % a->hkv == 0 && a->hq / a->hkv <= 8,
             "bad head counts");
  // the exact fallback, prepared first: it validates the call as cs_ccpe_decode_bf16 does
  decode_params p{};
  int st = prepare_decode(a->q, a->q_s_batch, a->q_s_head, a->batch, a->hq, a->hkv, a->nk, a->max_nk, a->kv, a->e,
                          a->max_positions, a->split, a->out, a->flags, &p);
  if (st) return st;
  const shared_ws need = carve_shared(nullptr, a->batch, a->hq, a->head_items, a->max_nk, a->split);
  CS_REQUIRE(workspace != nullptr && workspace_bytes >= need.bytes &&
                 (reinterpret_cast<uintptr_t>(workspace) % 256) == 0,
             "shared-run decode workspace holds %lld bytes, the call needs %lld (256-byte aligned)",
             static_cast<long long>(workspace_bytes), static_cast<long long>(need.bytes));
  if (a->batch == 0) return CS_OK;
  const shared_ws w = carve_shared(static_cast<char*>(workspace), a->batch, a->hq, a->head_items, a->max_nk,
                                   a->split);
  hipStream_t s = as_stream(stream);
  // head: every run once for all requests (rows = requests), positions P-1
  if (a->head_items > 0) {
    cs_kv_source kh = *a->kv;
    kh.block_table = a->head_table;
    kh.bt_stride = a->head_blocks;
    kh.bt_cols = a->head_blocks;
    st = cs::launch_prefill_states(a->q, 0, a->q_s_batch, a->q_s_head, a->head_qpos, a->batch, a->head_items,
                                   a->batch, a->hq, a->hkv, a->head_nk, &kh, a->e, a->max_positions, 1, 8,
                                   w.head_o, w.head_ml, nullptr, a->flags, s);
    if (st) return st;
  }
  // tail: one query row per request, exact positions, narrow workgroups;
  // the launch also clears the fallback's gate word
  cs_kv_source kt = *a->kv;
  kt.block_table = a->tail_table;
  kt.bt_stride = a->tail_stride;
  kt.bt_cols = a->tail_cols;
  st = cs::launch_prefill_states(a->q, a->q_s_batch, 0, a->q_s_head, a->tail_qpos, 1, a->batch, 1, a->hq, a->hkv,
                                 a->tail_nk, &kt, a->e, a->max_positions, 0, 2, w.tail_o, w.tail_ml, w.gate,
                                 a->flags, s);
  if (st) return st;
  const int group = a->hq / a->hkv;
  hipLaunchKernelGGL(shared_merge_kernel, dim3(static_cast<uint32_t>(a->batch) * a->hkv), dim3(kD * group), 0, s,
                     w.tail_o, w.tail_ml, w.head_o, w.head_ml, a->batch, a->hq, group, a->head_items,
                     static_cast<float>(a->max_positions - 1), static_cast<uint16_t*>(a->out), w.gate);
  CS_LAUNCH_CHECK("ccpe_decode_shared_merge");
  // the exact decode over the full block table, run only when some tail left a
  // head's positions below P-1
  p.gate = w.gate;
  return launch_decode(p, w.decode, stream);
}
