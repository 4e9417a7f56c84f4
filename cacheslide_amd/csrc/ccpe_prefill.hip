// CCPE prefill attention on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
// Computes, for every query row r (position qpos[r]) and query head h,
//   logit_j   = (q . k_j) / sqrt(128)                       position.py:157-164
//   p_j       = clamp(sum_{j' >= j, j' <= qpos} sigmoid(logit_j'), 0, P-1)
//                                                           position.py:295-307
//   bias_j    = QE[floor p] + frac * (QE[min(floor p + 1, P-1)] - QE[floor p]),
//               QE = q . E (unscaled q)                     position.py:309-344
//   out       = softmax_j(logit_j + bias_j) . V over keys j <= qpos
//                                                           position.py:518-550
// for keys 0..nk-1 (the cope_attention default key_positions = arange).
//
// Work decomposition.  A workgroup of 8 wavefronts owns 32 query rows x 4
// query heads of one GQA group (64 x 2 or 128 x 1 for group sizes 2 and 1);
// each wave owns 16 (row, head) pairs and all 8 waves share the K / V^T tile
// staged in LDS.  Key tiles of 64 are walked from the right-most causal key
// leftwards; each row carries the gate mass of the keys already visited, and
// once every row of a wave carries >= P-1 its remaining tiles are saturated
// (p = P-1, bias = QE[P-1]) and the sigmoid / scan / lerp work is skipped.
//
// MFMA data layout (16x16x32 bf16, lane l, g = l / 16, n = l % 16):
//   A[m][k]: lane holds row m = n, k = 8g .. 8g+7
//   B[k][n]: lane holds col n,     k = 8g .. 8g+7
//   C[m][n]: lane holds col n,     rows 4g .. 4g+3
// S^T = K Q^T puts the query row on the lane (n) and keys on the registers:
// lane group g of M-tile mt holds keys 16 mt + 4g .. +3, so the online-softmax
// statistics are per-lane scalars shared by the 4 lanes n, n+16, n+32, n+48.
// For O^T = V^T P^T the 32 keys of a k-step are ordered so that lane group g
// supplies the 8 S^T values it already holds (keys 32t + 4g + 0..3 and
// 32t + 16 + 4g + 0..3); V^T, staged transposed in LDS, is read in that order.

#include "common.h"

namespace cs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;          // head dim (K and V)
constexpr int kTileN = 64;       // keys per tile
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = 16;              // (row, head) pairs per wave
constexpr int kKStride = kD + 8;       // bf16 per K row in LDS (272 B)
constexpr int kVStride = kTileN + 8;   // bf16 per V^T row in LDS (144 B)
// The per-wave QE tables live in LDS next to the K / V^T tiles; P <= 128 keeps
// the workgroup at <= 102 KB, under the 160 KB a gfx950 workgroup may use.
constexpr int kMaxPos = 128;
constexpr size_t kStaticLds = sizeof(uint16_t) * (kTileN * kKStride + kD * kVStride) + 32;
constexpr size_t kLdsLimit = 160 * 1024;

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

struct prefill_params {
  const uint16_t* q;
  int64_t q_sb, q_st, q_sh;
  const int64_t* qpos;
  int64_t qpos_sb;
  int32_t batch, nq, hq, hkv, group, heads_per_wg, row_blocks;
  const int32_t* nk;
  kv_addr kv;
  const float* e;
  int32_t npos, pos_tiles, tab_stride;
  uint16_t* out;
  int32_t* flags;
  int32_t total_wg;
};

__device__ inline bf16x8 as_bf16x8(uint4 u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

// Flat workgroup id -> (batch, kv head, head group, row block).  Dispatch is
// round-robin over the 8 XCDs by id, so contiguous logical ranges are spread as
// one per XCD: a (batch, kv head)'s K/V stays in one XCD's L2.  The heaviest
// (right-most) row blocks go first.
__device__ inline void decode_wg(const prefill_params& p, int& b, int& kvh, int& hg, int& rb) {
  const int id = blockIdx.x;
  int logical = id;
  if (p.total_wg % 8 == 0) logical = (id % 8) * (p.total_wg / 8) + id / 8;
  const int hgroups = p.group / p.heads_per_wg;
  rb = p.row_blocks - 1 - (logical % p.row_blocks);
  int rest = logical / p.row_blocks;
  hg = rest % hgroups;
  rest /= hgroups;
  kvh = rest % p.hkv;
  b = rest / p.hkv;
}

__global__ void __launch_bounds__(kThreads, 2) ccpe_prefill_kernel(prefill_params p) {
  __shared__ __align__(16) uint16_t k_lds[kTileN * kKStride];
  __shared__ __align__(16) uint16_t v_lds[kD * kVStride];
  __shared__ int64_t wg_max_pos;
  extern __shared__ __align__(16) float tab_lds[];  // [kWaves][16][tab_stride]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;   // lane group: keys 4g..4g+3 of each 16-key M-tile
  const int ln = lane & 15;  // this lane's (row, head) pair within the wave

  int b, kvh, hg, rb;
  decode_wg(p, b, kvh, hg, rb);
  const int head_slot = wave % p.heads_per_wg;
  const int row_sub = wave / p.heads_per_wg;
  const int h = kvh * p.group + hg * p.heads_per_wg + head_slot;
  const int wg_rows = kRows * (kWaves / p.heads_per_wg);
  const int r = rb * wg_rows + row_sub * kRows + ln;
  const bool row_ok = r < p.nq;
  const int nk = p.nk[b];
  const int64_t qp = row_ok ? p.qpos[b * p.qpos_sb + r] : -1;

  if (tid == 0) wg_max_pos = 0;
  __syncthreads();
  // wave extremes of the query positions (for the key range and masking)
  int64_t wmax = qp, wmin = row_ok ? qp : INT64_MAX;
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t a = __shfl_xor(wmax, off, 64);
    const int64_t c = __shfl_xor(wmin, off, 64);
    wmax = a > wmax ? a : wmax;
    wmin = c < wmin ? c : wmin;
  }
  if (lane == 0)
    atomicMax(reinterpret_cast<unsigned long long*>(&wg_max_pos),
              static_cast<unsigned long long>(wmax < 0 ? 0 : wmax));
  __syncthreads();
  const int64_t kend = (wg_max_pos + 1) < nk ? (wg_max_pos + 1) : nk;  // keys [0, kend)

  // ---- Q as the B operand of S^T: 4 k-steps x 8 bf16 ------------------------
  bf16x8 qreg[4];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + static_cast<int64_t>(row_ok ? r : 0) * p.q_st + h * p.q_sh;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 u = row_ok ? *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * g)
                             : make_uint4(0, 0, 0, 0);
      qreg[s] = as_bf16x8(u);
    }
  }

  // ---- QE table: QE^T = E^T Q^T, E split into bf16 hi + lo (~fp32 product) ----
  float* tab = tab_lds + wave * kRows * p.tab_stride;
  for (int pt = 0; pt < p.pos_tiles; ++pt) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const int pos = pt * 16 + ln;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 ahi, alo;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ev = pos < p.npos ? p.e[(32 * s + 8 * g + i) * p.npos + pos] : 0.f;
        const __bf16 hb = static_cast<__bf16>(ev);
        ahi[i] = hb;
        alo[i] = static_cast<__bf16>(ev - static_cast<float>(hb));
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, qreg[s], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, qreg[s], acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int posv = pt * 16 + 4 * g + v;
      if (posv < p.npos) tab[ln * p.tab_stride + posv] = acc[v];
    }
  }
  __syncthreads();
  const float* trow = tab + ln * p.tab_stride;
  const float top = static_cast<float>(p.npos - 1);
  const float kLog2e = 1.4426950408889634f;
  const float logit_scale = 0.08838834764831845f;  // 1/sqrt(128)
  const float sat_bias2 = trow[p.npos - 1] * kLog2e;

  // ---- main loop --------------------------------------------------------------
  float carry = row_ok ? 0.f : 3.0e38f;  // padded rows count as saturated
  float m_run = -INFINITY;                // running max (log2 domain), per row
  float l_run = 0.f;                      // this lane's share of the row sum
  floatx4 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Global -> register staging: threads [0, 256) stage K (4 x 16 B), threads
  // [256, 512) stage V as 4 keys x 8 dims for the transposed store.
  uint4 st[4];
  bool bad_block = false;
  const bool k_stager = tid < 256;
  const int sid = tid & 255;
  // key (within a tile) and 16-byte chunk of this thread's staging slot rr
  auto slot_key = [&](int rr) { return k_stager ? ((sid + 256 * rr) >> 4) : 4 * (sid >> 4) + rr; };
  const int slot_dc = k_stager ? (sid & 15) : (sid & 15);
  // Block ids of the next tile to load are fetched one tile earlier, so each
  // iteration issues only the K/V loads (one global round trip, overlapped
  // with the current tile's compute).
  int32_t bid[4] = {0, 0, 0, 0};
  auto fetch_blocks = [&](int64_t base) {
    if (!p.kv.block_table) return;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int64_t j = base + slot_key(rr);
      bid[rr] = -1;
      if (j < kend) {
        const int64_t bi = p.kv.bs_shift >= 0 ? (j >> p.kv.bs_shift) : j / p.kv.block_size;
        if (bi < p.kv.bt_cols) bid[rr] = p.kv.block_table[b * p.kv.bt_stride + bi];
      }
    }
  };
  auto load_tile = [&](int64_t base) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int64_t j = base + slot_key(rr);
      st[rr] = make_uint4(0, 0, 0, 0);
      if (j < kend) {
        const uint16_t* row = nullptr;
        if (p.kv.block_table) {
          const int32_t blk = bid[rr];
          if (blk < 0 || blk >= p.kv.num_blocks) {
            bad_block = true;
          } else {
            const int64_t off = p.kv.bs_shift >= 0 ? (j & ((int64_t(1) << p.kv.bs_shift) - 1))
                                                   : j % p.kv.block_size;
            row = p.kv.cache + blk * p.kv.s_block + kvh * p.kv.s_head + off * p.kv.s_offset +
                  (k_stager ? 0 : kD);
          }
        } else {
          row = k_stager ? p.kv.k + b * p.kv.k_sb + j * p.kv.k_st + kvh * p.kv.k_sh
                         : p.kv.v + b * p.kv.v_sb + j * p.kv.v_st + kvh * p.kv.v_sh;
        }
        if (row) st[rr] = *reinterpret_cast<const uint4*>(row + 8 * slot_dc);
      }
    }
  };
  auto store_tile = [&]() {
    if (k_stager) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int c = sid + 256 * rr;
        *reinterpret_cast<uint4*>(&k_lds[(c >> 4) * kKStride + 8 * (c & 15)]) = st[rr];
      }
    } else {
      const int dc = sid & 15, kg = sid >> 4;
      const uint16_t* e0 = reinterpret_cast<const uint16_t*>(&st[0]);
      const uint16_t* e1 = reinterpret_cast<const uint16_t*>(&st[1]);
      const uint16_t* e2 = reinterpret_cast<const uint16_t*>(&st[2]);
      const uint16_t* e3 = reinterpret_cast<const uint16_t*>(&st[3]);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        uint2 w;
        w.x = static_cast<uint32_t>(e0[d]) | (static_cast<uint32_t>(e1[d]) << 16);
        w.y = static_cast<uint32_t>(e2[d]) | (static_cast<uint32_t>(e3[d]) << 16);
        *reinterpret_cast<uint2*>(&v_lds[(8 * dc + d) * kVStride + 4 * kg]) = w;
      }
    }
  };

  const int64_t ntiles = (kend + kTileN - 1) / kTileN;
  if (ntiles > 0) {
    fetch_blocks((ntiles - 1) * kTileN);
    load_tile((ntiles - 1) * kTileN);
    if (ntiles > 1) fetch_blocks((ntiles - 2) * kTileN);
  }
  for (int64_t t = ntiles - 1; t >= 0; --t) {
    const int64_t base = t * kTileN;
    __syncthreads();
    store_tile();
    __syncthreads();
    if (t > 0) load_tile((t - 1) * kTileN);
    if (t > 1) fetch_blocks((t - 2) * kTileN);

    // Waves whose rows all precede the tile contribute nothing to it.
    if (base > wmax) continue;

    // S^T for the four 16-key M-tiles: sacc[mt][v] = key 16 mt + 4g + v.
    floatx4 sacc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      sacc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = &k_lds[(16 * mt + ln) * kKStride + 8 * g];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 32 * s));
        sacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[s], sacc[mt], 0, 0, 0);
      }
    }

    // Masking is needed only when some key of the tile is past some row's
    // position (or past kend).
    const bool need_mask = (base + kTileN - 1 > wmin) || (base + kTileN > kend);
    if (need_mask) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t j = base + 16 * mt + 4 * g + v;
          if (!(j <= qp && j < kend)) sacc[mt][v] = -INFINITY;
        }
    }

    if (__all(carry >= top)) {
      // saturated: bias = QE[P-1]; score (log2 domain) = logit*scale*log2e + const
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) sacc[mt][v] = sacc[mt][v] * (logit_scale * kLog2e) + sat_bias2;
    } else {
      // gates, in-run suffix sums (runs of 4 keys), cross-lane suffix over runs
      float suf[4][4];
      float run[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        float acc = 0.f;
#pragma unroll
        for (int v = 3; v >= 0; --v) {
          const float xv = sacc[mt][v] * logit_scale;
          const float gate = sacc[mt][v] == -INFINITY ? 0.f : 1.f / (1.f + __expf(-xv));
          acc += gate;
          suf[mt][v] = acc;
        }
        run[mt] = acc;
      }
      // inclusive suffix over the 4 lane groups (g ascending = keys ascending)
      float incl[4], mt_total[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        float s1 = run[mt];
        float n1 = __shfl_down(s1, 16, 64);
        if (g < 3) s1 += n1;
        float n2 = __shfl_down(s1, 32, 64);
        if (g < 2) s1 += n2;
        incl[mt] = s1;
        mt_total[mt] = __shfl(s1, ln, 64);  // lane group 0 holds the M-tile total
      }
      float right = 0.f;  // gate mass of the M-tiles to the right of mt
#pragma unroll
      for (int mt = 3; mt >= 0; --mt) {
        const float before = carry + right + (incl[mt] - run[mt]);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float pos = before + suf[mt][v];
          pos = pos < top ? pos : top;
          pos = pos > 0.f ? pos : 0.f;  // also maps NaN to 0: table reads stay in range
          const float fl = floorf(pos);
          const int lo = static_cast<int>(fl);
          const int hi = lo + 1 < p.npos - 1 ? lo + 1 : p.npos - 1;
          const float lo_b = trow[lo];
          const float bias = lo_b + (pos - fl) * (trow[hi] - lo_b);
          sacc[mt][v] = (sacc[mt][v] * logit_scale + bias) * kLog2e;
        }
        right += mt_total[mt];
      }
      carry += right;
    }

    // Online softmax: row max over the 16 values and the 4 lanes of the row.
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) tmax = fmaxf(tmax, sacc[mt][v]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const bool live = m_new != -INFINITY;
    if (__any(m_new != m_run)) {
      const float corr = (live && m_run != -INFINITY) ? __builtin_amdgcn_exp2f(m_run - m_new) : (live ? 0.f : 1.f);
      l_run *= corr;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt] *= corr;
    }
    m_run = m_new;
    float psum = 0.f;
    bf16x8 pb[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float pv = live ? __builtin_amdgcn_exp2f(sacc[2 * kt + half][v] - m_new) : 0.f;
          psum += pv;
          pb[kt][4 * half + v] = static_cast<__bf16>(pv);
        }
      }
    }
    l_run += psum;

    // O^T += V^T P^T: A = V^T rows (dims), keys in the k-step order above.
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* vrow = &v_lds[(16 * dt + ln) * kVStride + 4 * g];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const uint2 lo4 = *reinterpret_cast<const uint2*>(vrow + 32 * kt);
        const uint2 hi4 = *reinterpret_cast<const uint2*>(vrow + 32 * kt + 16);
        const uint4 u = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(u), pb[kt], o[dt], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: O^T lane holds row ln, dims 16 dt + 4g + v ------------------
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok) {
    uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.nq + r) * p.hq + h) * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      bf16x4 w;
#pragma unroll
      for (int v = 0; v < 4; ++v) w[v] = static_cast<__bf16>(o[dt][v] * inv);
      *reinterpret_cast<bf16x4*>(orow + 16 * dt + 4 * g) = w;
    }
  }
  if (bad_block) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
}

}  // namespace
}  // namespace cs

using namespace cs;

namespace {
int fill_kv(const cs_kv_source* kv, cs::kv_addr* a) {
  CS_REQUIRE(kv != nullptr, "null kv source");
  cs::kv_addr r{};
  if (kv->block_table) {
    CS_REQUIRE(kv->cache && kv->block_size > 0 && kv->num_blocks > 0, "paged kv needs a cache");
    CS_REQUIRE(kv->s_block % 8 == 0 && kv->s_head % 8 == 0 && kv->s_offset % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(kv->cache) % 16) == 0,
               "paged cache rows must be 16-byte aligned");
    r.cache = static_cast<const uint16_t*>(kv->cache);
    r.s_block = kv->s_block;
    r.s_head = kv->s_head;
    r.s_offset = kv->s_offset;
    r.block_size = kv->block_size;
    r.bs_shift = -1;
    for (int s = 0; s < 31; ++s)
      if ((1 << s) == kv->block_size) r.bs_shift = s;
    r.num_blocks = kv->num_blocks;
    r.block_table = kv->block_table;
    r.bt_stride = kv->bt_stride;
    r.bt_cols = kv->bt_cols;
    CS_REQUIRE(r.bt_cols > 0, "block table needs at least one column");
  } else {
    CS_REQUIRE(kv->k && kv->v, "dense kv needs k and v");
    CS_REQUIRE(kv->k_s_tok % 8 == 0 && kv->k_s_head % 8 == 0 && kv->v_s_tok % 8 == 0 &&
                   kv->v_s_head % 8 == 0 && kv->k_s_batch % 8 == 0 && kv->v_s_batch % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(kv->k) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(kv->v) % 16) == 0,
               "dense K/V rows must be 16-byte aligned");
    r.k = static_cast<const uint16_t*>(kv->k);
    r.v = static_cast<const uint16_t*>(kv->v);
    r.k_sb = kv->k_s_batch;
    r.k_st = kv->k_s_tok;
    r.k_sh = kv->k_s_head;
    r.v_sb = kv->v_s_batch;
    r.v_st = kv->v_s_tok;
    r.v_sh = kv->v_s_head;
  }
  *a = r;
  return CS_OK;
}
}  // namespace

extern "C" int cs_ccpe_prefill_bf16(const void* q, int64_t q_s_batch, int64_t q_s_tok,
                                    int64_t q_s_head, const int64_t* qpos, int64_t qpos_s_batch,
                                    int32_t batch, int32_t nq, int32_t hq, int32_t hkv,
                                    const int32_t* nk, const cs_kv_source* kv, const float* e,
                                    int32_t max_positions, void* out, int32_t* flags,
                                    void* stream) {
  CS_REQUIRE(q && qpos && nk && e && out && flags, "null arguments");
  CS_REQUIRE(batch >= 0 && nq >= 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts");
  CS_REQUIRE(max_positions >= 2 && max_positions <= kMaxPos, "max_positions must be in [2, %d]",
             kMaxPos);
  CS_REQUIRE(q_s_tok % 8 == 0 && q_s_head % 8 == 0 && q_s_batch % 8 == 0 &&
                 (reinterpret_cast<uintptr_t>(q) % 16) == 0,
             "query rows must be 16-byte aligned");
  const int group = hq / hkv;
  int heads_per_wg;
  if (group % 4 == 0) heads_per_wg = 4;
  else if (group == 2) heads_per_wg = 2;
  else if (group == 1) heads_per_wg = 1;
  else {
    set_error("GQA group size %d is not supported by the MFMA prefill kernel", group);
    return CS_EUNSUPPORTED;
  }
  cs::prefill_params p{};
  int st = fill_kv(kv, &p.kv);
  if (st) return st;
  if (batch == 0 || nq == 0) return CS_OK;
  p.q = static_cast<const uint16_t*>(q);
  p.q_sb = q_s_batch;
  p.q_st = q_s_tok;
  p.q_sh = q_s_head;
  p.qpos = qpos;
  p.qpos_sb = qpos_s_batch;
  p.batch = batch;
  p.nq = nq;
  p.hq = hq;
  p.hkv = hkv;
  p.group = group;
  p.heads_per_wg = heads_per_wg;
  const int wg_rows = kRows * (kWaves / heads_per_wg);
  p.row_blocks = static_cast<int32_t>(ceil_div(nq, wg_rows));
  p.nk = nk;
  p.e = e;
  p.npos = max_positions;
  p.pos_tiles = (max_positions + 15) / 16;
  p.tab_stride = p.pos_tiles * 16 + 1;
  p.out = static_cast<uint16_t*>(out);
  p.flags = flags;
  int64_t total = static_cast<int64_t>(batch) * hkv * (group / heads_per_wg) * p.row_blocks;
  CS_REQUIRE(total < (1ll << 31), "grid too large");
  p.total_wg = static_cast<int32_t>(total);
  size_t smem = sizeof(float) * kWaves * kRows * p.tab_stride;
  if (smem + kStaticLds > kLdsLimit) {
    set_error("prefill LDS %zu bytes exceeds the workgroup limit", smem + kStaticLds);
    return CS_EUNSUPPORTED;
  }
  hipLaunchKernelGGL(ccpe_prefill_kernel, dim3(p.total_wg), dim3(kThreads), smem,
                     as_stream(stream), p);
  CS_LAUNCH_CHECK("ccpe_prefill");
  return CS_OK;
}
