// CCPE prefill attention on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16).
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
// Work decomposition.  A workgroup (4 wavefronts) owns 32 query rows x 4 query
// heads of one GQA group (or 64/128 rows for group sizes 2/1), so every wave
// shares the K/V tile staged in LDS.  Key tiles of 64 are walked from the
// right-most causal key leftwards; each row carries the gate mass of the keys
// already visited, and once every row of a wave carries >= P-1 the remaining
// tiles are saturated (p = P-1, bias = QE[P-1]) and the sigmoid / scan / lerp
// work is skipped.
//
// MFMA data layout (32x32x16 bf16, lane l, g = l / 32):
//   A[m][k]: lane holds row m = l % 32, k = 8g .. 8g+7
//   B[k][n]: lane holds col n = l % 32, k = 8g .. 8g+7
//   C[m][n]: lane holds col n = l % 32, value v -> row 8(v/4) + 4g + (v%4)
// S^T = K Q^T puts the query row on the lane (n) and keys on the registers, so
// the online-softmax statistics are per-lane scalars.  K rows are fed to the A
// operand through the permutation pi(m) that swaps bits 2 and 3 of m; then C
// register v of lane group g holds physical key 16(v/8) + 8g + (v%8), i.e. every
// lane holds runs of 8 consecutive keys, which is exactly the B-operand layout
// P^T needs for O^T = V^T P^T (keys 8g..8g+7 of each 16-key k-step).  V^T is
// staged transposed in LDS so its A operand is one 16-byte read per lane.

#include "common.h"

namespace cs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned short ushort8 __attribute__((ext_vector_type(8)));

constexpr int kD = 128;          // head dim (K and V)
constexpr int kTileN = 64;       // keys per tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKStride = kD + 8;       // bf16 per K row in LDS (272 B)
constexpr int kVStride = kTileN + 8;   // bf16 per V^T row in LDS (144 B)
// The per-wave QE tables live in LDS next to the K / V^T tiles; P <= 128 keeps
// the workgroup at <= 101 KB, under the 160 KB a gfx950 workgroup may use.
constexpr int kMaxPos = 128;
constexpr size_t kStaticLds = sizeof(uint16_t) * (kTileN * kKStride + kD * kVStride) + 16;
constexpr size_t kLdsLimit = 160 * 1024;

struct kv_addr {
  const uint16_t* cache;
  int64_t s_block, s_head, s_offset;
  int32_t block_size;
  int64_t num_blocks;
  const int32_t* block_table;
  int64_t bt_stride;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;
};

struct prefill_params {
  const uint16_t* q;
  int64_t q_sb, q_st, q_sh;
  const int64_t* qpos;
  int64_t qpos_sb;
  int32_t batch, nq, hq, hkv, group, heads_per_wg, rows_per_wave_group, row_blocks;
  const int32_t* nk;
  kv_addr kv;
  const float* e;
  int32_t npos, pos_tiles, tab_stride;
  uint16_t* out;
  int32_t* flags;
  int32_t total_wg;
};

// Row pointer of K (or V when is_v) for key j of batch b, kv head kvh, or null.
__device__ inline const uint16_t* kv_row(const kv_addr& a, int b, int kvh, int64_t j, bool is_v,
                                         bool* bad) {
  if (a.block_table) {
    int64_t bi = j / a.block_size;
    int32_t blk = a.block_table[b * a.bt_stride + bi];
    if (blk < 0 || blk >= a.num_blocks) {
      *bad = true;
      return nullptr;
    }
    int64_t off = j % a.block_size;
    return a.cache + blk * a.s_block + kvh * a.s_head + off * a.s_offset + (is_v ? kD : 0);
  }
  return is_v ? a.v + b * a.v_sb + j * a.v_st + kvh * a.v_sh
              : a.k + b * a.k_sb + j * a.k_st + kvh * a.k_sh;
}

__device__ inline bf16x8 as_bf16x8(uint4 u) {
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(float_to_bf16(lo)) | (static_cast<uint32_t>(float_to_bf16(hi)) << 16);
}

// Map a flat workgroup id to (batch, kv head, head group, row block), spreading
// contiguous logical ranges over the 8 XCDs (dispatch is round-robin by id) so
// that one (batch, kv head)'s K/V stays in one XCD's L2, and visiting the
// heaviest (right-most) row blocks first.
__device__ inline void decode_wg(const prefill_params& p, int& b, int& kvh, int& hg, int& rb) {
  int id = blockIdx.x;
  int logical = id;
  if (p.total_wg % 8 == 0) {
    int per = p.total_wg / 8;
    logical = (id % 8) * per + id / 8;
  }
  int hgroups = p.group / p.heads_per_wg;
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
  extern __shared__ __align__(16) float tab_lds[];  // [kWaves][32][tab_stride]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;   // lane group
  const int ln = lane & 31;  // row within the wave

  int b, kvh, hg, rb;
  decode_wg(p, b, kvh, hg, rb);
  const int head_slot = wave % p.heads_per_wg;
  const int row_sub = wave / p.heads_per_wg;
  const int h = kvh * p.group + hg * p.heads_per_wg + head_slot;
  const int wg_rows = 32 * (kWaves / p.heads_per_wg);
  const int row0 = rb * wg_rows;
  const int r = row0 + row_sub * 32 + ln;  // this lane's query row
  const bool row_ok = r < p.nq;
  const int nk = p.nk[b];
  const int64_t qp = row_ok ? p.qpos[b * p.qpos_sb + r] : -1;

  // Right-most key of the workgroup: max causal key over its rows.
  __shared__ int64_t wg_max_pos;
  if (tid == 0) wg_max_pos = 0;
  __syncthreads();
  {
    int64_t m = qp;
    for (int off = 32; off > 0; off >>= 1) {
      int64_t o = __shfl_xor(m, off, 64);
      m = o > m ? o : m;
    }
    if (lane == 0) atomicMax(reinterpret_cast<unsigned long long*>(&wg_max_pos),
                             static_cast<unsigned long long>(m < 0 ? 0 : m));
  }
  __syncthreads();
  const int64_t kend = (wg_max_pos + 1) < nk ? (wg_max_pos + 1) : nk;  // keys [0, kend)

  // ---- Q as the B operand of S^T (8 k-steps x 8 bf16) -----------------
  bf16x8 qreg[8];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + static_cast<int64_t>(row_ok ? r : 0) * p.q_st + h * p.q_sh;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      uint4 u = row_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * s + 8 * g) : make_uint4(0, 0, 0, 0);
      qreg[s] = as_bf16x8(u);
    }
  }

  // ---- QE table: QE^T = E^T Q^T with E split into bf16 hi + lo ---------
  float* tab = tab_lds + wave * 32 * p.tab_stride;
  for (int pt = 0; pt < p.pos_tiles; ++pt) {
    floatx16 acc = {};
    const int pos = pt * 32 + ln;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      ushort8 hi8, lo8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float ev = pos < p.npos ? p.e[(16 * s + 8 * g + i) * p.npos + pos] : 0.f;
        uint16_t hb = float_to_bf16(ev);
        float rem = ev - bf16_to_float(hb);
        hi8[i] = hb;
        lo8[i] = float_to_bf16(rem);
      }
      bf16x8 ahi, alo;
      __builtin_memcpy(&ahi, &hi8, 16);
      __builtin_memcpy(&alo, &lo8, 16);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi, qreg[s], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo, qreg[s], acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      int posv = pt * 32 + 8 * (v / 4) + 4 * g + (v % 4);
      if (posv < p.npos) tab[ln * p.tab_stride + posv] = acc[v];
    }
  }
  __syncthreads();
  const float qe_last = tab[ln * p.tab_stride + (p.npos - 1)];
  const float top = static_cast<float>(p.npos - 1);

  // ---- main loop --------------------------------------------------------
  const float kLog2e = 1.4426950408889634f;
  const float logit_scale = 0.08838834764831845f;  // 1/sqrt(128)
  float carry = row_ok ? 0.f : 3.0e38f;  // padded rows count as saturated
  float m_run = -INFINITY;                // running max (log2 domain)
  float l_run = 0.f;                      // this lane's share of the row sum
  floatx16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = floatx16{};

  // K rows for the A operand: lane loads key pi(ln) of each 32-key M-tile.
  const int pim = ((ln >> 4) << 4) | (((ln >> 2) & 1) << 3) | (((ln >> 3) & 1) << 2) | (ln & 3);

  // Global->register staging (prefetch of the next tile).
  uint4 kst[4], vst[4];
  bool bad_block = false;
  auto load_tile = [&](int64_t base) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      int c = tid + kThreads * rr;
      int key = c >> 4, dc = c & 15;
      int64_t j = base + key;
      kst[rr] = make_uint4(0, 0, 0, 0);
      if (j < kend) {
        const uint16_t* kr = kv_row(p.kv, b, kvh, j, false, &bad_block);
        if (kr) kst[rr] = *reinterpret_cast<const uint4*>(kr + 8 * dc);
      }
    }
    {
      int dc = tid & 15, kg = tid >> 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int64_t j = base + 4 * kg + i;
        vst[i] = make_uint4(0, 0, 0, 0);
        if (j < kend) {
          const uint16_t* vr = kv_row(p.kv, b, kvh, j, true, &bad_block);
          if (vr) vst[i] = *reinterpret_cast<const uint4*>(vr + 8 * dc);
        }
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      int c = tid + kThreads * rr;
      int key = c >> 4, dc = c & 15;
      *reinterpret_cast<uint4*>(&k_lds[key * kKStride + 8 * dc]) = kst[rr];
    }
    {
      int dc = tid & 15, kg = tid >> 4;
      const uint16_t* e0 = reinterpret_cast<const uint16_t*>(&vst[0]);
      const uint16_t* e1 = reinterpret_cast<const uint16_t*>(&vst[1]);
      const uint16_t* e2 = reinterpret_cast<const uint16_t*>(&vst[2]);
      const uint16_t* e3 = reinterpret_cast<const uint16_t*>(&vst[3]);
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
  if (ntiles > 0) load_tile((ntiles - 1) * kTileN);
  for (int64_t t = ntiles - 1; t >= 0; --t) {
    const int64_t base = t * kTileN;
    __syncthreads();
    store_tile();
    __syncthreads();
    if (t > 0) load_tile((t - 1) * kTileN);

    // S^T for the two 32-key halves of the tile.
    floatx16 sacc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      sacc[mt] = floatx16{};
      const uint16_t* krow = &k_lds[(32 * mt + pim) * kKStride + 8 * g];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 16 * s));
        sacc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[s], sacc[mt], 0, 0, 0);
      }
    }

    // Causal masking is needed unless every key of the tile is <= every row.
    const bool wave_sat = __all(carry >= top);
    const int64_t tile_last = base + kTileN - 1;
    // Logits (log2 domain) with masked keys at -inf; keys of run (mt, v/8).
    float x[2][16];
    bool any_masked = false;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int64_t j = base + 32 * mt + 16 * (v / 8) + 8 * g + (v % 8);
        bool ok = row_ok && j <= qp && j < kend;
        any_masked |= !ok;
        x[mt][v] = ok ? sacc[mt][v] * logit_scale : -INFINITY;
      }
    (void)tile_last;

    if (wave_sat) {
      const float bl = qe_last;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) x[mt][v] = (x[mt][v] + bl) * kLog2e;
    } else {
      // gates and in-run suffix sums (runs of 8 keys, right to left)
      float gsuf[2][16];
      float run_tot[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int rb2 = 0; rb2 < 2; ++rb2) {
          float acc = 0.f;
#pragma unroll
          for (int i = 7; i >= 0; --i) {
            int v = 8 * rb2 + i;
            float xv = x[mt][v];
            float gate = xv == -INFINITY ? 0.f : 1.f / (1.f + __expf(-xv));
            acc += gate;
            gsuf[mt][v] = acc;
          }
          run_tot[2 * mt + rb2] = acc;
        }
      // Run R = 4mt + 2rb2 + g in physical key order; the partner lane (g^1)
      // holds the other parity.  Exclusive suffix over runs.
      float other[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) other[i] = __shfl_xor(run_tot[i], 32, 64);
      float tot[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        tot[2 * i + g] = run_tot[i];
        tot[2 * i + (1 - g)] = other[i];
      }
      float excl[8];
      float accr = 0.f;
#pragma unroll
      for (int R = 7; R >= 0; --R) {
        excl[R] = accr;
        accr += tot[R];
      }
      const float* trow = tab + ln * p.tab_stride;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          int R = 4 * mt + 2 * (v / 8) + g;
          float pos = carry + excl[R] + gsuf[mt][v];
          pos = pos < top ? pos : top;
          pos = pos > 0.f ? pos : 0.f;  // also maps NaN to 0: table reads stay in range
          float fl = floorf(pos);
          int lo = static_cast<int>(fl);
          int hi = lo + 1 < p.npos - 1 ? lo + 1 : p.npos - 1;
          float lo_b = trow[lo];
          float hi_b = trow[hi];
          float bias = lo_b + (pos - fl) * (hi_b - lo_b);
          x[mt][v] = (x[mt][v] + bias) * kLog2e;
        }
      carry += accr;
    }
    (void)any_masked;

    // Online softmax (per lane = per query row, partner lane shares the row).
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) tmax = fmaxf(tmax, x[mt][v]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
    bf16x8 pb[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        ushort8 packed;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float xv = x[mt][8 * half + i];
          float pv = (m_new == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(xv - m_new);
          psum += pv;
          packed[i] = float_to_bf16(pv);
        }
        __builtin_memcpy(&pb[2 * mt + half], &packed, 16);
      }
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] *= corr;

    // O^T += V^T P^T
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint16_t* vrow = &v_lds[(32 * dt + ln) * kVStride + 8 * g];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(vrow + 16 * ks));
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[dt], 0, 0, 0);
      }
    }
  }

  // ---- epilogue ---------------------------------------------------------
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok) {
    uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.nq + r) * p.hq + h) * kD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        int dim = 32 * dt + 8 * q4 + 4 * g;
        uint2 w;
        w.x = pack_bf16x2(o[dt][4 * q4 + 0] * inv, o[dt][4 * q4 + 1] * inv);
        w.y = pack_bf16x2(o[dt][4 * q4 + 2] * inv, o[dt][4 * q4 + 3] * inv);
        *reinterpret_cast<uint2*>(orow + dim) = w;
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
    r.num_blocks = kv->num_blocks;
    r.block_table = kv->block_table;
    r.bt_stride = kv->bt_stride;
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
  const int wg_rows = 32 * (kWaves / heads_per_wg);
  p.row_blocks = static_cast<int32_t>(ceil_div(nq, wg_rows));
  p.nk = nk;
  p.e = e;
  p.npos = max_positions;
  p.pos_tiles = (max_positions + 31) / 32;
  p.tab_stride = p.pos_tiles * 32 + 1;
  p.out = static_cast<uint16_t*>(out);
  p.flags = flags;
  int64_t total = static_cast<int64_t>(batch) * hkv * (group / heads_per_wg) * p.row_blocks;
  CS_REQUIRE(total < (1ll << 31), "grid too large");
  p.total_wg = static_cast<int32_t>(total);
  size_t smem = sizeof(float) * kWaves * 32 * p.tab_stride;
  if (smem + kStaticLds > kLdsLimit) {
    set_error("prefill LDS %zu bytes exceeds the workgroup limit", smem + kStaticLds);
    return CS_EUNSUPPORTED;
  }
  hipLaunchKernelGGL(ccpe_prefill_kernel, dim3(p.total_wg), dim3(kThreads), smem,
                     as_stream(stream), p);
  CS_LAUNCH_CHECK("ccpe_prefill");
  return CS_OK;
}
