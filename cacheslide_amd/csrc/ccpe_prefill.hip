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
// Softmax is invariant to a per-row constant, so the kernel adds
// bias_j - QE[P-1] instead of bias_j: keys whose position saturates at P-1
// add nothing, and a tile whose columns all carry gate mass >= P-1 is plain
// attention.  The score MFMAs accumulate onto minus the column's running max,
// so a probability is exp2 of one multiply of the accumulator; the scores
// themselves stay unscaled fp32 sums of exact bf16 products, which keeps the
// gates (whose errors add up along the position sum) at fp32 accuracy.
//
// Work decomposition.  A workgroup of 4 wavefronts owns 128 (row, head)
// columns of one GQA group: 128/G rows x the G query heads of one KV head
// (column c = row_local * G + head_local); each wave owns 32 columns.  Key
// tiles of 32 are walked from the right-most causal key leftwards through three
// LDS stages filled by direct global->LDS loads (global_load_lds_dwordx4),
// two tiles ahead.
//
// MFMA layout (32x32x16 bf16, lane l, n = l % 32, h = l / 32):
//   A[m][k]: lane holds row m = n, k = 8h .. 8h+7
//   B[k][n]: lane holds col n,     k = 8h .. 8h+7
//   C[m][n]: lane holds col n,     rows 8(v/4) + 4h + v%4, v = 0..15
// S^T = K Q^T puts the column on the lane and the 32 keys of the tile on the
// 16 accumulator registers (runs of 4 keys alternating between h = 0 and 1),
// so the online-softmax statistics are per-lane scalars shared by lanes n and
// n + 32.  O^T = V^T P^T takes P^T straight from those registers: k-step ks
// uses keys 16ks + 4h + 0..3 and 16ks + 8 + 4h + 0..3 as k = 8h .. 8h+7, and
// the V^T operand is read in the same order from the row-major V tile with
// ds_read_b64_tr_b16 (lane i of a 16-lane group receives element i of the
// four 4-element rows addressed by lanes 4e .. 4e+3).
//
// LDS tile layouts (16-byte chunk c of key k, in 16-byte slots), chosen so
// every read is one per-lane base plus an immediate offset and no two lanes
// of a 16-lane phase share a bank:
//   K: slot (k / 4) * 64 + (c ^ (k / 4 % 4)) * 4 + k % 4   (A reads: 16 keys x one chunk)
//   V: slot (k / 4) * 64 + c * 4 + k % 4                   (transposed reads: 4 keys x 2 chunks)
// so one direct load (64 lanes x 16 bytes = slots 64 j .. 64 j + 63) covers the
// same four keys 4j .. 4j+3 in K and in V, and each lane loads key 4j + lane % 4
// of both: the record address of a key is computed once for K and V.
//
// K/V sources (MODE): dense K/V rows (0); the paged cache through a block table
// (1); the paged cache through a per-token slot map whose slots past the native
// pool name sidecar rows (2).  Modes 1 and 2 keep a window of the table (block
// ids, or one entry per key) in LDS, and a load whose four keys share one block
// in consecutive offsets takes the scalar-base form; other loads address each
// lane's record.

#include <cstdlib>
#include <mutex>

#include "common.h"
#include "ccpe_path.h"
#include "prefill_shared.h"

namespace cs {
namespace {

constexpr int kStages = 3;
constexpr size_t kStaticLds = kStages * 2 * kStageSlots * 16 + 4 * kBtWindow + 16;

// WAVES wavefronts of 32 columns each (2, 4 or 8); registers for two
// wavefronts per SIMD.  POLICY (dense K/V only): CanonicalPositionPolicy and
// SelectedAssociationPolicy.  A selected fixed row sees one fixed key, its
// own, at its canonical position; a fixed row that is not selected sees every
// fixed key at its canonical position (the calibration-layer call, and
// selected_attention "all"); other rows keep their contextual positions.
template <int MODE, int WAVES, bool POLICY = false>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) ccpe_prefill_kernel(prefill_params p) {
  constexpr bool PAGED = MODE != 0;
  constexpr bool SLOTS = MODE == 2;
  constexpr int kThreads = 64 * WAVES;
  constexpr int kInstr = 8 / WAVES;  // 64-slot loads per wave for each of K and V
  __shared__ __align__(16) stage_t st0;
  __shared__ __align__(16) stage_t st1;
  __shared__ __align__(16) stage_t st2;
  // block ids of blocks [bt_lo, bt_lo + kBtWindow), or (slot map) the entries
  // of keys [bt_lo, bt_lo + kBtWindow)
  __shared__ int32_t bt_lds[kBtWindow];
  __shared__ int64_t wg_max_pos;
  __shared__ int32_t quiet_lds[WAVES];  // POLICY: the wave's columns all skip tiles of fixed keys
  // [32 WAVES columns][tab_stride] QE log2(e), fp32
  extern __shared__ __align__(16) float tab[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (an SGPR)
  const int n = lane & 31;  // column within the wave
  const int h = lane >> 5;  // k half of the MFMA operands

  int b, kvh, rb;
  // Key split (POLICY, split_role > 0): part 0 of a split row block walks
  // tiles [t_split, ntiles), the keys down from every row's diagonal; part
  // s > 0 an equal share of [0, t_split) with the positions taken as
  // saturated.  Each part leaves its softmax state in slot slot0 + part.
  int part = 0, nparts = 1, slot0 = 0, t_split = 0;
  if (!POLICY || p.split_role == 0) {
    decode_wg(p, b, kvh, rb);
  } else {
    int logical;
    if (p.split_role == 1) {
      if (static_cast<int>(blockIdx.x) < p.split_extra) {
        const int32_t item = uniform_load(p.split_items, static_cast<int64_t>(blockIdx.x));
        if (item < 0) return;  // an unused extra part: the whole workgroup, before any barrier
        logical = item >> 4;
        part = item & 15;
      } else {
        logical = logical_wg(p, static_cast<int>(blockIdx.x) - p.split_extra);
      }
      nparts = uniform_load(p.split_plan, 3 * static_cast<int64_t>(logical));
      slot0 = uniform_load(p.split_plan, 3 * static_cast<int64_t>(logical) + 1);
      t_split = uniform_load(p.split_plan, 3 * static_cast<int64_t>(logical) + 2);
    } else {
      // fix-up: a split block whose part 0 left some column's positions below
      // P-1 (its other parts then took unsaturated keys as saturated) is
      // walked again unsplit; every other workgroup ends here
      logical = uniform_load(p.split_blocks, static_cast<int64_t>(blockIdx.x));
      if (logical < 0) return;
      const int s0 = uniform_load(p.split_plan, 3 * static_cast<int64_t>(logical) + 1);
      const float* carries = p.part_ml + (static_cast<int64_t>(s0) * 3 + 2) * 256;
      const bool low = tid < kCols * WAVES && carries[tid] < static_cast<float>(p.npos - 1);
      if (!__syncthreads_or(low ? 1 : 0)) return;
    }
    decode_logical(p, logical, b, kvh, rb);
  }
  const int c = wave * kCols + n;  // column within the workgroup
  const int row = rb * p.rows_per_wg + c / p.group;
  const int head = kvh * p.group + c % p.group;
  const bool row_ok = row < p.nq;
  const int nk = p.nk[b];
  // The prologue's loads -- the row's position, its Q row and the first 64
  // positions of E -- go out together and unconditionally, from clamped
  // addresses (a row past nq reads row 0, a position past P reads position
  // 0; select drops the values), so their latencies overlap instead of
  // following one another behind the reduction of the positions.
  const int row_c = row_ok ? row : 0;
  const int64_t qp_raw = p.qpos[b * p.qpos_sb + row_c];
  uint4 qraw[8];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + static_cast<int64_t>(row_c) * p.q_st + head * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qraw[ks] = *reinterpret_cast<const uint4*>(qrow + 16 * ks + 8 * h);
  }
  // item (position pc + i % 64, dims 8 (i / 64) .. + 7) for i = tid + kThreads r:
  // its 8 values become one 16-byte chunk of E^T hi and one of lo
  constexpr int kItems = kPosChunk * kChunks / kThreads;
  float ev[kItems][8];
  auto load_e = [&](int pc) {
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
      const int i = tid + kThreads * r;
      const int pos = i % kPosChunk, dg = i / kPosChunk;
      const int pp = pc + pos < p.npos ? pc + pos : 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) ev[r][e] = p.e[(8 * dg + e) * p.npos + pp];
    }
  };
  load_e(0);
  const int64_t qp = row_ok ? qp_raw : -1;
  bool sel_col = false;   // the column's row is selected: fixed keys other than its own are invisible
  float canon_self = 0.f;  // canonical position of the column's own key (NaN: contextual)
  // a fixed row that is not selected: its profile row, canonical positions
  // of every fixed key
  const float* canon_row = nullptr;
  bool canon_wave = false;
  if constexpr (POLICY) {
    canon_self = __builtin_nanf("");
    if (row_ok) {
      sel_col = p.sel_rows ? p.sel_rows[row] != 0 : false;
      if (p.canon_self) canon_self = p.canon_self[static_cast<int64_t>(head) * p.nq + row];
      const int64_t qo = p.canon && p.q_ord ? p.q_ord[row] : -1;
      if (!sel_col && qo >= 0) canon_row = p.canon + head * p.c_s0 + qo * p.c_s1;
    }
    canon_wave = __builtin_amdgcn_readfirstlane(__any(canon_row != nullptr) ? 1 : 0) != 0;
  }

  if (tid == 0) wg_max_pos = 0;
  if (tid == 0 && blockIdx.x == 0 && p.zero_word != nullptr) *p.zero_word = 0;
  __syncthreads();
  int64_t wmax = qp, wmin = row_ok ? qp : INT64_MAX;
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t a = __shfl_xor(wmax, off, 64);
    const int64_t d = __shfl_xor(wmin, off, 64);
    wmax = a > wmax ? a : wmax;
    wmin = d < wmin ? d : wmin;
  }
  if (lane == 0 && wmax >= 0)
    atomicMax(reinterpret_cast<unsigned long long*>(&wg_max_pos), static_cast<unsigned long long>(wmax));

  // ---- Q^T as the B operand of S^T: 8 k-steps of 16 dims ---------------------
  bf16x8 qb[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qb[ks] = as_bf16x8(row_ok ? qraw[ks] : make_uint4(0, 0, 0, 0));

  // ---- QE table: QE^T = E^T Q^T on MFMA, E split into bf16 hi + lo ------------
  // E^T hi / lo for kPosChunk positions are staged in the (still unused) K / V
  // stages, swizzled like K: chunk c of position pos at c ^ (pos % 16).
  uint16_t* ehi = reinterpret_cast<uint16_t*>(&st0);  // [64 pos][128 dims], 16 KB
  uint16_t* elo = reinterpret_cast<uint16_t*>(&st1);
  float* tcol = tab + c * p.tab_stride;
  // (a saturated call never reads the table: no gate, suffix sum or lerp)
  const int table_npos = p.saturated ? 0 : p.npos;
  // the column's QE for positions 32 k + 8 (v / 4) + 4 h + v % 4 in qe[k][v]
  constexpr int kPb = kMaxPos / 32;
  floatx16 qe[kPb];
#pragma unroll
  for (int k = 0; k < kPb; ++k) qe[k] = floatx16{};
#pragma unroll
  for (int pc = 0; pc < kMaxPos; pc += kPosChunk) {
    if (pc >= table_npos) break;
    if (pc > 0) load_e(pc);  // the first chunk was loaded with Q
    __syncthreads();  // the previous chunk's MFMAs have read the stage
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
      const int i = tid + kThreads * r;
      const int pos = i % kPosChunk, dg = i / kPosChunk;
      const bool pos_ok = pc + pos < p.npos;
      bf16x8 hv, lv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = pos_ok ? ev[r][e] : 0.f;
        hv[e] = static_cast<__bf16>(x);
        lv[e] = static_cast<__bf16>(x - static_cast<float>(hv[e]));
      }
      const int slot = pos * kChunks + (dg ^ (pos & 15));
      *reinterpret_cast<bf16x8*>(ehi + slot * 8) = hv;
      *reinterpret_cast<bf16x8*>(elo + slot * 8) = lv;
    }
    __syncthreads();
#pragma unroll
    for (int pb = 0; pb < kPosChunk / 32; ++pb) {
      if (pc + 32 * pb >= p.npos) break;
      floatx16 acc = {};
      const int pos = 32 * pb + n;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const int slot = pos * kChunks + ((2 * ks + h) ^ (pos & 15));
        const bf16x8 ah = as_bf16x8(*reinterpret_cast<const uint4*>(ehi + slot * 8));
        const bf16x8 al = as_bf16x8(*reinterpret_cast<const uint4*>(elo + slot * 8));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qb[ks], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, qb[ks], acc, 0, 0, 0);
      }
      qe[pc / 32 + pb] = acc;
    }
  }
  // Entries in raw-score units, finite (clamped to +-1e30, NaN to -1e30, so
  // bias + (-inf) stays -inf), each shifted by the column's QE[P-1] (the bias
  // of saturated keys; softmax is invariant to it), and entry P repeating
  // entry P-1: a position p reads entries lo = floor(min(p, P-1)) and lo + 1
  // with no clamp, and a saturated key adds 0.  QE[P-1] comes from the
  // registers of the lane of the column that holds it, so every entry is
  // written once, already shifted.
  if (table_npos > 0) {
    auto clamp_qe = [](float x) { return fminf(fmaxf(x * kSqrtD, -1e30f), 1e30f); };
    const int p1 = p.npos - 1;
    const int kt = p1 >> 5, rt = p1 & 31;
    const int vt = 4 * (rt >> 3) + (rt & 3), ht = (rt >> 2) & 1;
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < kPb; ++k)
#pragma unroll
      for (int v = 0; v < 16; ++v) t = k == kt && v == vt ? qe[k][v] : t;
    const float t_other = __shfl_xor(t, 32, 64);
    const float top_qe = clamp_qe(h == ht ? t : t_other);
    // every register of the chunks that start below entry P is stored,
    // without a branch: entries from P-1 up are 0, and indices past P store
    // entry P (which the last line stores in any case)
#pragma unroll
    for (int k = 0; k < kPb; ++k) {
      if (32 * k >= p.npos) break;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int pv = 32 * k + 8 * (v >> 2) + 4 * h + (v & 3);
        tcol[pv < p.npos ? pv : p.npos] = pv < p1 ? clamp_qe(qe[k][v]) - top_qe : 0.f;
      }
    }
    if (h == 0) tcol[p.npos] = 0.f;
  }
  __syncthreads();

  const int64_t wgmax = wg_max_pos;
  const int64_t kend = wgmax + 1 < nk ? wgmax + 1 : (nk > 0 ? nk : 0);  // keys [0, kend)
  const int ntiles = static_cast<int>((kend + kTileN - 1) / kTileN);
  // key coordinates of the tile loop fit in 32 bits (kend <= nk < 2^31)
  const int qp32 = qp < 0 ? -1 : static_cast<int>(qp);
  const int kend32 = static_cast<int>(kend);
  // wave extremes are wave-uniform after the reduction; keep them scalar so the
  // tile tests below are uniform branches
  const int wmax32 = __builtin_amdgcn_readfirstlane(wmax < 0 ? -1 : static_cast<int>(wmax));
  const int wmin32 = __builtin_amdgcn_readfirstlane(wmin > kend ? kend32 : static_cast<int>(wmin));

  // ---- block ids: the table entries of a window of tiles are copied to LDS
  // before the window's tile loop, so that loop issues no vector-memory
  // operation other than the tile loads themselves.
  int64_t bt_lo = 0;
  auto load_window = [&](int tlo, int thi) {  // blocks (or slots) of keys [32 tlo, 32 thi)
    if constexpr (SLOTS) {
      const int klo = tlo * kTileN, n_win = (thi - tlo) * kTileN;
      const int64_t* srow = p.kv.slots + b * p.kv.slots_stride;
      for (int i = tid; i < n_win; i += kThreads) {
        const int key = klo + i;
        uint32_t ent = kNoSlot;
        if (key < kend && key < p.kv.slots_cols) {
          const int64_t slot = srow[key];
          if (slot >= 0 && slot < p.kv.native_slots)
            ent = static_cast<uint32_t>(slot);
          else if (slot >= p.kv.native_slots && slot - p.kv.native_slots < p.kv.side_rows)
            ent = kSideTag | static_cast<uint32_t>(slot - p.kv.native_slots);
        }
        bt_lds[i] = static_cast<int32_t>(ent);
      }
      bt_lo = klo;
    } else {
      const int64_t blo = (static_cast<int64_t>(tlo) * kTileN) >> p.kv.bs_shift;
      const int64_t bhi = (static_cast<int64_t>(thi) * kTileN - 1) >> p.kv.bs_shift;
      for (int64_t i = tid; i <= bhi - blo; i += kThreads)
        bt_lds[i] = blo + i < p.kv.bt_cols ? p.kv.block_table[b * p.kv.bt_stride + blo + i] : -1;
      bt_lo = blo;
    }
  };

  // ---- tile loads.  Load j (0..7) of a stage fills slots [64 j, 64 j + 64) of
  // K and of V with keys 4j .. 4j+3, lane l taking key 4j + l % 4: K chunk
  // (l / 4) ^ (j % 4), V chunk l / 4.  Wave w issues loads j = kInstr w ..
  // kInstr w + kInstr - 1, so its lanes need kInstr records per tile.
  const int chunk = lane >> 2;
  bool bad_block = false;
  // record base of this request / KV head; per-key offsets below are 32-bit
  // products (the host checks that the strides fit)
  const uint16_t* rec_base = PAGED ? p.kv.cache + kvh * p.kv.s_head
                                   : p.kv.k + b * p.kv.k_sb + kvh * p.kv.k_sh;
  const uint16_t* vrec_base = PAGED ? rec_base + kD : p.kv.v + b * p.kv.v_sb + kvh * p.kv.v_sh;
  const uint32_t s_blk = static_cast<uint32_t>(PAGED ? p.kv.s_block : p.kv.k_st);
  const uint32_t s_off = static_cast<uint32_t>(PAGED ? p.kv.s_offset : 0);
  const uint32_t v_st = static_cast<uint32_t>(PAGED ? p.kv.s_block : p.kv.v_st);
  const uint32_t off_mask = PAGED ? (1u << p.kv.bs_shift) - 1u : 0u;
  const int nblocks = PAGED ? static_cast<int>(p.kv.num_blocks < INT32_MAX ? p.kv.num_blocks : INT32_MAX) : 0;
  const uint16_t* zrec = reinterpret_cast<const uint16_t*>(g_zero_record);
  // LDS byte addresses of the stages; K at +0, V at +kStageSlots * 16
  const uint32_t st_lds[kStages] = {lds_address(&st0), lds_address(&st1), lds_address(&st2)};
  // Per-lane byte offsets within the four records of a load (key 4j + lane % 4),
  // fixed for the kernel: K chunk (lane / 4) ^ (j % 4) for each of the wave's
  // loads, V chunk lane / 4.
  const uint32_t key_stride_k = 2u * (PAGED ? s_off : s_blk);  // bytes between keys of a load
  const uint32_t key_stride_v = 2u * (PAGED ? s_off : v_st);
  uint32_t lane_koff[kInstr];
#pragma unroll
  for (int i = 0; i < kInstr; ++i)
    lane_koff[i] = (lane & 3) * key_stride_k + 16u * (chunk ^ ((kInstr * wave + i) & 3));
  const uint32_t lane_voff = (lane & 3) * key_stride_v + 16u * chunk + (PAGED ? 2u * kD : 0u);
  const uint64_t kbase_bytes = reinterpret_cast<uint64_t>(rec_base);
  const uint64_t vbase_bytes = PAGED ? kbase_bytes : reinterpret_cast<uint64_t>(vrec_base);
  // Paged fast-path record offsets of the wave's loads, 64 tiles at a time:
  // lane L holds, for tile fo_top - L, the byte offset from rec_base of the
  // record of the first key of load i, or ~0 in the high word when that load
  // takes the per-lane path (a key at or past kend, an invalid block, blocks
  // of fewer than 4 keys, a tile outside the block-table window).
  uint32_t fo_lo[kInstr], fo_hi[kInstr];
  int fo_top = 0, win_lo = 0;
  auto preload = [&](int ttop) {
    fo_top = ttop;
    const int tl = ttop - lane;
#pragma unroll
    for (int i = 0; i < kInstr; ++i) {
      const int key0 = tl * kTileN + 4 * (kInstr * wave + i);
      bool ok = tl >= win_lo && key0 + 3 < kend32 && p.kv.bs_shift >= 2;
      int blk;
      uint32_t offs;
      if constexpr (SLOTS) {
        // the four keys' slots are native, consecutive and in one block
        const int idx = ok ? key0 - static_cast<int>(bt_lo) : 0;
        const uint32_t s0 = static_cast<uint32_t>(bt_lds[idx]);
        ok = ok && (s0 & kSideTag) == 0u && (s0 & off_mask) + 3u <= off_mask &&
             static_cast<uint32_t>(bt_lds[idx + 1]) == s0 + 1u &&
             static_cast<uint32_t>(bt_lds[idx + 2]) == s0 + 2u &&
             static_cast<uint32_t>(bt_lds[idx + 3]) == s0 + 3u;
        blk = static_cast<int>(s0 >> p.kv.bs_shift);
        offs = s0 & off_mask;
      } else {
        const int idx = ok ? (key0 >> p.kv.bs_shift) - static_cast<int>(bt_lo) : 0;
        blk = bt_lds[idx];
        ok = ok && blk >= 0 && blk < nblocks;
        offs = static_cast<uint32_t>(key0) & off_mask;
      }
      const uint64_t off = 2ull * (static_cast<uint64_t>(static_cast<uint32_t>(blk)) * s_blk +
                                   static_cast<uint64_t>(offs) * s_off);
      fo_lo[i] = ok ? static_cast<uint32_t>(off) : 0u;
      fo_hi[i] = ok ? static_cast<uint32_t>(off >> 32) : 0xFFFFFFFFu;
    }
  };
  auto issue = [&](int t, int stage) {
    if constexpr (PAGED) {
      if (t <= fo_top - 64) preload(t);
    }
    const uint32_t kbase = st_lds[stage], vbase = kbase + kStageSlots * 16;
#pragma unroll
    for (int i = 0; i < kInstr; ++i) {
      const int j = kInstr * wave + i;
      const int key0 = t * kTileN + 4 * j;  // wave-uniform first key of the load
      // Fast path: all four keys before kend and (paged) their block valid and
      // at least 4 keys long, so the four keys share it: the record base is
      // wave-uniform and computed in scalar registers.
      bool fast = key0 + 3 < kend32;
      uint64_t sk = 0, sv = 0;
      if constexpr (PAGED) {
        const int L = fo_top - t;
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fo_hi[i]), L));
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fo_lo[i]), L));
        fast = hi != 0xFFFFFFFFu;
        sk = kbase_bytes + ((static_cast<uint64_t>(hi) << 32) | lo);
        sv = sk;
      } else {
        sk = kbase_bytes + 2ull * static_cast<uint64_t>(static_cast<uint32_t>(key0)) * s_blk;
        sv = vbase_bytes + 2ull * static_cast<uint64_t>(static_cast<uint32_t>(key0)) * v_st;
      }
      if (fast) {
        lds_dma16_s(lane_koff[i], sk, kbase + 1024 * j);
        lds_dma16_s(lane_voff, sv, vbase + 1024 * j);
      } else {
        // K and V rows of key key0 + lane % 4; the zero record when the key is
        // past kend or its block is invalid
        const int key = key0 + (lane & 3);
        const bool in = key < kend32;
        const uint16_t* kr;
        const uint16_t* vr;
        if constexpr (SLOTS) {
          const uint32_t ent = in ? static_cast<uint32_t>(bt_lds[key - static_cast<int>(bt_lo)]) : kNoSlot;
          const bool ok = ent != kNoSlot;
          bad_block |= in && !ok;
          if (ok && (ent & kSideTag)) {
            const int64_t so = static_cast<int64_t>(ent & ~kSideTag) * p.kv.side_sr + kvh * p.kv.side_sh;
            kr = p.kv.side_k + so;
            vr = p.kv.side_v + so;
          } else {
            const uint64_t off = static_cast<uint64_t>(ent >> p.kv.bs_shift) * s_blk +
                                 static_cast<uint64_t>(ent & off_mask) * s_off;
            kr = ok ? rec_base + off : zrec;
            vr = kr + kD;
          }
        } else if constexpr (PAGED) {
          const int blk = bt_lds[(key >> p.kv.bs_shift) - static_cast<int>(bt_lo)];
          const bool ok = in && blk >= 0 && blk < nblocks;
          bad_block |= in && !ok;
          const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(blk)) * s_blk +
                               static_cast<uint64_t>(static_cast<uint32_t>(key) & off_mask) * s_off;
          kr = ok ? rec_base + off : zrec;
          vr = kr + kD;
        } else {
          kr = in ? rec_base + static_cast<uint64_t>(static_cast<uint32_t>(key)) * s_blk : zrec;
          vr = in ? vrec_base + static_cast<uint64_t>(static_cast<uint32_t>(key)) * v_st : zrec + kD;
        }
        lds_dma16(kr + 8 * (chunk ^ (j & 3)), kbase + 1024 * j);
        lds_dma16(vr + 8 * chunk, vbase + 1024 * j);
      }
    }
  };
  // wait until this wave's loads of the current tile have landed, with the
  // next tile's loads (2 kInstr of them) possibly still in flight
  // (and, with canonical cells fetched after those loads, those 4 as well)
  auto wait_tile = [&](bool next_in_flight, bool cells_after) {
    if (next_in_flight && cells_after)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kInstr + 4));
    else if (next_in_flight)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kInstr));
    else if (cells_after)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(4));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  };

  // ---- per-tile compute -------------------------------------------------------
  const float top = static_cast<float>(p.npos - 1);
  // padded columns count as saturated, and so do the columns of a split part
  // below the keys next to the diagonals and those of a saturated call
  float carry = !row_ok ? 3.0e38f : (part > 0 || p.saturated ? top : 0.f);
  // Running max of the column's raw scores q.k.  S^T accumulates onto minit =
  // -m_base in every register (m_base = m_run once finite, 0 before), so the
  // scores arrive shifted by the running max: exp2 of a score is one multiply
  // away, with no per-score subtract.
  float m_run = -INFINITY;
  float m_base = 0.f;
  floatx16 minit = {};
  float l_run = 0.f;                     // this lane's share of the column sum
  floatx16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = floatx16{};

  const int j16 = lane & 15;
  // element offset of this lane's transposed V read within a stage
  const int vrd_off = 512 * h + 32 * (2 * ((lane >> 4) & 1) + ((j16 & 3) >> 1)) + 8 * (j16 >> 2) + 4 * (j16 & 1);
  // Canonical cells of a tile for the columns of fixed rows that are not
  // selected, issued before the tile's barrier (behind the loads of the next
  // tile, ahead of those of the tile after) so that their latency overlaps
  // the barrier and the score MFMAs.  Per run of 4 keys (8 j4 + 4h + 0..3):
  // one 16-byte load when the run is a whole aligned group (cgo >= 0, its
  // first ordinal), else the zero record (the cells are then read key by key).
  const float* zero_f = reinterpret_cast<const float*>(g_zero_record);
  auto fetch = [&](int t, floatx4 (&cv)[4], int (&cgo)[4]) -> bool {
    if constexpr (POLICY) {
      if (!canon_wave || t * kTileN > wmax32) return false;
      if (uniform_load(p.fixed_bits, t) == 0u) return false;
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const int32_t g0 = uniform_load(p.grp, 8 * static_cast<int64_t>(t) + 2 * j4);
        const int32_t g1 = uniform_load(p.grp, 8 * static_cast<int64_t>(t) + 2 * j4 + 1);
        const int32_t go = canon_row ? (h ? g1 : g0) : -1;
        cgo[j4] = go;
        cv[j4] = load_f4_untracked(go >= 0 ? canon_row + go : zero_f);
      }
      return true;
    }
    return false;
  };
  // (dma_after: this tile's K/V loads were issued after the canonical cells)
  auto compute = [&](int t, const uint4* kst, const uint4* vst, floatx4 (&cv)[4], const int (&cgo)[4],
                     bool dma_after) {
    const int base = t * kTileN;
    if (base > wmax32) return;  // every column of the wave precedes the tile
    uint32_t fixed_word = 0;
    if constexpr (POLICY) {
      // A tile of fixed keys is invisible to selected columns except at their
      // own key, and a saturated column's positions no longer depend on its
      // gates: when that holds for the whole wave, the tile adds nothing.
      fixed_word = uniform_load(p.fixed_bits, t);
      if (fixed_word == 0xFFFFFFFFu && __all(!row_ok || (sel_col && carry >= top))) return;
    }
    // all K operands first, then the 8 MFMAs of S^T
    // key n, chunk 2 ks + h: slot (n / 4) * 64 + ((2 ks + h) ^ g) * 4 + n % 4 with
    // g = n / 4 % 4, i.e. one of two per-lane bases (ks even / odd) + 16 (ks / 2)
    bf16x8 ka[8];
    const int g = (n >> 2) & 3;
    const uint4* krd0 = kst + (n >> 2) * 64 + (n & 3) + 4 * (h ^ g);
    const uint4* krd1 = kst + (n >> 2) * 64 + (n & 3) + 4 * ((2 + h) ^ g);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) ka[ks] = as_bf16x8((ks & 1 ? krd1 : krd0)[16 * (ks >> 1)]);
    floatx16 s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[0], qb[0], minit, 0, 0, 0);
#pragma unroll
    for (int ks = 1; ks < 8; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[ks], qb[ks], s, 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // the 8 LDS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // then the 8 MFMAs
    const bool need_mask = (base + kTileN - 1 > wmin32) || (base + kTileN > kend32);
    // key v of the tile (8 (v/4) + 4h + v%4) is visible to the column when
    // 8 (v/4) + v%4 <= lim
    const int lim = (qp32 < kend32 - 1 ? qp32 : kend32 - 1) - base - 4 * h;
    // s holds the raw scores minus m_base; the causal mask first, for both
    // paths (a masked score stays -inf through the bias, and its gate is
    // dropped by the visibility test below)
    if (need_mask) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (8 * (v >> 2) + (v & 3) > lim) s[v] = -INFINITY;
    }
    const bool unsat = !__all(carry >= top);
    bool canon_tile = false;
    if constexpr (POLICY) canon_tile = canon_wave && fixed_word != 0u;
    if (unsat || canon_tile) {
      float pos[16];
      if (unsat) {
        const float gate_off = -m_base * (kInvSqrtD * kLog2e);
        // gates; runs of 4 keys (8 j4 + 4h + 0..3) and their in-run suffix sums.
        // A key past the causal end holds a -inf score (masked above whenever
        // the tile reaches past any column's row): its gate is 0.
        float gsuf[16], run[4];
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          float acc = 0.f;
#pragma unroll
          for (int i = 3; i >= 0; --i) {
            const int v = 4 * j4 + i;
            // sigmoid(q.k / sqrt(D)) = 1 / (1 + 2^(-(s + m_base) log2(e) / sqrt(D)))
            const float e = __builtin_amdgcn_exp2f(fmaf(s[v], -kInvSqrtD * kLog2e, gate_off));
            acc += __builtin_amdgcn_rcpf(1.f + e);
            gsuf[v] = acc;
          }
          run[j4] = acc;
        }
        float other[4];
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          float a, c2;
          swap_halves(run[j4], a, c2);
          other[j4] = h ? a : c2;
        }
        // gate mass of the runs with larger keys: (j4, h=1) follows (j4, h=0)
        float after[4];
        float acc = 0.f;
#pragma unroll
        for (int j4 = 3; j4 >= 0; --j4) {
          after[j4] = acc + (h == 0 ? other[j4] : 0.f);
          acc += run[j4] + other[j4];
        }
        // the canonical position replaces the contextual one at a selected
        // row's own key (its other fixed x fixed cells are invisible)
        int self_v = -1;
        if constexpr (POLICY) {
          const int self_key = static_cast<int>(qp) - base - 4 * h;  // 8 j4 + i for this lane's half
          if (!__builtin_isnan(canon_self) && self_key >= 0 && self_key < kTileN - 4 * h &&
              (self_key & 4) == 0)
            self_v = 4 * (self_key >> 3) + (self_key & 3);
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          // position of the key: the carry, the runs with larger keys, the suffix in its run
          pos[v] = (carry + after[v >> 2]) + gsuf[v];
          if constexpr (POLICY) pos[v] = v == self_v ? canon_self : pos[v];
        }
        carry += acc;
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) pos[v] = top;  // saturated: every contextual position is P-1
      }
      if constexpr (POLICY) {
        if (canon_tile) {
          // the cells fetched before this tile's K/V loads have landed
          if (dma_after)
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kInstr));
          else
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
#pragma unroll
          for (int j4 = 0; j4 < 4; ++j4) asm volatile("" : "+v"(cv[j4]));
          if (canon_row) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int j4 = v >> 2, i = v & 3;
              const int kt = 8 * j4 + 4 * h + i;  // key within the tile
              if ((fixed_word >> kt) & 1u) {
                const float c = cgo[j4] >= 0 ? cv[j4][i] : canon_row[p.code[base + kt] * p.c_s2];
                pos[v] = fmaxf(c, 0.f);  // negative or NaN cells (the checker rejects them) read entry 0
              }
            }
          }
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        // positions are >= 0; NaN becomes P-1: table reads stay in range
        const float pv = fminf(pos[v], top);
        const uint32_t lo = static_cast<uint32_t>(pv);
        const float frac = __builtin_amdgcn_fractf(pv);
        const float t0 = tcol[lo], t1 = tcol[lo + 1];
        // raw score plus the bias in raw units; a masked key stays -inf
        // (table entries are finite)
        s[v] += fmaf(frac, t1 - t0, t0);
      }
    }
    if constexpr (POLICY) {
      // SelectedAssociationPolicy: fixed keys other than the row's own are
      // invisible to selected rows (after the gates: the positions above
      // still count them).  Lane (n, h) holds keys 8 j4 + 4h + i.
      const int self_key = static_cast<int>(qp) - base;  // in [0, 32) when in this tile
      uint32_t hide = sel_col ? fixed_word : 0u;
      if (self_key >= 0 && self_key < kTileN) hide &= ~(1u << self_key);
      hide = (hide >> (4 * h)) & 0x0F0F0F0Fu;
      if (__any(hide != 0u)) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if ((hide >> (8 * (v >> 2) + (v & 3))) & 1u) s[v] = -INFINITY;
      }
    }
    // V^T operands, read after the bias work (not live across it, which keeps
    // registers for the 8 K operands above) and consumed after the softmax.
    // Byte offset of this lane's read = 1024 h + 64 chunk-in-block +
    // 16 (key % 4) + 8 half, plus 4096 ks + 2048 r + 256 db.
    bf16x8 va[8];
    const uint16_t* vrd = reinterpret_cast<const uint16_t*>(vst) + vrd_off;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x4_tr lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (CS_LDS bf16x4_tr*)(vrd + 2048 * ks + 128 * db));
        const bf16x4_tr hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (CS_LDS bf16x4_tr*)(vrd + 2048 * ks + 1024 + 128 * db));
        va[4 * ks + db] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    // Online softmax.  The probabilities are taken against the running max as
    // it stands (the scores arrive shifted by it); a tile only needs the max
    // when its probabilities could grow too large (a lane's sum above 2^16) or
    // when the column has no max yet.  Such a tile (rare: the first one, or
    // scores rising well above every earlier key) takes the exact max, moves
    // the running max to it, rescales O and the sum, and recomputes.
    const bf16x2 ones = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
    uint32_t pw[8];
    auto probs = [&]() {
      float sum = 0.f;
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const float p0 = __builtin_amdgcn_exp2f(s[v] * (kInvSqrtD * kLog2e));
        const float p1 = __builtin_amdgcn_exp2f(s[v + 1] * (kInvSqrtD * kLog2e));
        pw[v >> 1] = pack_bf16x2(p0, p1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[i]), ones, sum, false);
      return sum;
    };
    float psum = probs();
    if (__any(!(psum <= 65536.f) || m_run == -INFINITY)) {
      float tmax = s[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) tmax = fmaxf(tmax, s[v]);
      {
        float a, c2;
        swap_halves(tmax, a, c2);
        tmax = fmaxf(a, c2);
      }
      // move to the tile max when it lies above the running max (always when
      // there is none yet); a fully masked tile (-inf) leaves it alone
      const bool move = tmax > (m_run == -INFINITY ? -INFINITY : 0.f);
      const float shift = move ? tmax : 0.f;
      const float m_new = move ? m_base + tmax : m_run;
      const float corr = move ? __builtin_amdgcn_exp2f((m_run - m_new) * (kInvSqrtD * kLog2e)) : 1.f;
      l_run *= corr;  // corr = 0 when the max was -inf: nothing accumulated yet
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] *= corr;
#pragma unroll
      for (int v = 0; v < 16; ++v) s[v] -= shift;
      m_run = m_new;
      m_base = m_new == -INFINITY ? 0.f : m_new;
#pragma unroll
      for (int v = 0; v < 16; ++v) minit[v] = -m_base;
      psum = probs();
    }
    l_run += psum;
    const bf16x8 pb0 = __builtin_bit_cast(bf16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
    const bf16x8 pb1 = __builtin_bit_cast(bf16x8, make_uint4(pw[4], pw[5], pw[6], pw[7]));
    // O^T += V^T P^T
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[4 * ks + db], ks ? pb1 : pb0, o[db], 0, 0, 0);
  };

  // POLICY: a tile of fixed keys adds nothing once every column of the
  // workgroup is a selected row with saturated positions (see compute); its
  // loads are then not issued.  Each wave publishes that state before the
  // tile barrier and reads every wave's behind it, so the decision, like the
  // state (carry only grows), holds for the whole workgroup from then on.
  bool wg_quiet = false;
  auto publish_quiet = [&]() __attribute__((always_inline)) {
    if constexpr (POLICY) {
      const bool q = __all(!row_ok || (sel_col && carry >= top));
      if (lane == 0) quiet_lds[wave] = q ? 1 : 0;
    }
  };
  auto read_quiet = [&]() __attribute__((always_inline)) {
    if constexpr (POLICY) {
      int q = 1;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) q &= quiet_lds[w];
      wg_quiet = __builtin_amdgcn_readfirstlane(q) != 0;
    }
  };
  // POLICY: once the workgroup is quiet, tiles below dyn_floor (all fixed
  // keys) add nothing: the walk ends there.
  int dyn_floor = 0;
  if constexpr (POLICY) dyn_floor = uniform_load(p.dyn_floor, 0);
  auto load_tile = [&](int u, int stage) __attribute__((always_inline)) -> bool {
    if constexpr (POLICY) {
      if (wg_quiet && uniform_load(p.fixed_bits, u) == 0xFFFFFFFFu) return false;
    }
    issue(u, stage);
    return true;
  };

  // ---- main loop: windows of tiles right to left; inside a window, tiles right
  // to left through three LDS stages with the loads two tiles ahead.  Each wave
  // waits for its own loads of a tile before the one barrier of the tile, which
  // both publishes that stage and frees the stage of the tile before, into
  // which the loads of the tile two ahead are then issued.
  // Every prologue load (Q, E, positions) has landed: without this the
  // compiler keeps a full vector-memory wait inside the tile loop for them.
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  int tiles_per_window = ntiles;
  if constexpr (SLOTS)
    tiles_per_window = kBtWindow / kTileN;
  else if constexpr (PAGED)
    tiles_per_window = static_cast<int>(((static_cast<int64_t>(kBtWindow) - 1) << p.kv.bs_shift) / kTileN);
  if (tiles_per_window < 1) tiles_per_window = 1;
  int t_top = ntiles, t_bot = 0;  // this workgroup's tiles [t_bot, t_top)
  if (nparts > 1) {
    const int ts = t_split < ntiles ? t_split : ntiles;
    if (part == 0) {
      t_bot = ts;
    } else {
      t_bot = static_cast<int>(static_cast<int64_t>(part - 1) * ts / (nparts - 1));
      t_top = static_cast<int>(static_cast<int64_t>(part) * ts / (nparts - 1));
    }
  }
  for (int thi = t_top; thi > t_bot;) {
    const int tlo = thi - tiles_per_window > t_bot ? thi - tiles_per_window : t_bot;
    if constexpr (PAGED) {
      __syncthreads();
      load_window(tlo, thi);
      __syncthreads();
      win_lo = tlo;
      preload(thi - 1);
    }
    issue(thi - 1, 0);
    bool iss1 = thi - 2 >= tlo;  // the loads of the next tile to compute were issued
    if (iss1) issue(thi - 2, 1);
    for (int t = thi - 1; t >= tlo; t -= 3) {
      floatx4 cv[4];
      int cgo[4];
      bool got = fetch(t, cv, cgo);
      wait_tile(iss1, got);
      publish_quiet();
      __syncthreads();
      read_quiet();
      if (POLICY && wg_quiet && t < dyn_floor) goto walk_done;
      const bool iss2 = t - 2 >= tlo && load_tile(t - 2, 2);
      compute(t, st0.k, st0.v, cv, cgo, iss2);
      if (t - 1 < tlo) break;
      got = fetch(t - 1, cv, cgo);
      wait_tile(iss2, got);
      publish_quiet();
      __syncthreads();
      read_quiet();
      if (POLICY && wg_quiet && t - 1 < dyn_floor) goto walk_done;
      const bool iss3 = t - 3 >= tlo && load_tile(t - 3, 0);
      compute(t - 1, st1.k, st1.v, cv, cgo, iss3);
      if (t - 2 < tlo) break;
      got = fetch(t - 2, cv, cgo);
      wait_tile(iss3, got);
      publish_quiet();
      __syncthreads();
      read_quiet();
      if (POLICY && wg_quiet && t - 2 < dyn_floor) goto walk_done;
      const bool iss4 = t - 4 >= tlo && load_tile(t - 4, 1);
      compute(t - 2, st2.k, st2.v, cv, cgo, iss4);
      iss1 = iss4;
    }
    thi = tlo;
  }
walk_done:
  // tile loads and canonical cells still in flight (a walk that ended early)
  // land before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

  // ---- epilogue: O^T lane holds column n, dims 32 db + 8 (v/4) + 4h + v%4 ----------
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (p.state_o != nullptr) {
    // the column's softmax state, for a merge with states over other keys
    if (bad_block) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
    if (row_ok) {
      const int64_t rh = (static_cast<int64_t>(b) * p.nq + row) * p.hq + head;
      float* so = p.state_o + rh * kD;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          floatx4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = o[db][4 * j4 + e];
          *reinterpret_cast<floatx4*>(so + 32 * db + 8 * j4 + 4 * h) = w;
        }
      if (h == 0) {
        p.state_ml[3 * rh] = m_run;
        p.state_ml[3 * rh + 1] = l_tot;
        p.state_ml[3 * rh + 2] = carry;
      }
    }
    return;
  }
  if (nparts > 1) {
    // a part's softmax state for policy_split_merge_kernel: O unnormalised
    // against the part's running max, that max, the sum and the carry
    const int64_t slot = slot0 + part;
    float* po = p.part_o + slot * kD * 256;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) po[(32 * db + 8 * (v >> 2) + 4 * h + (v & 3)) * 256 + c] = o[db][v];
    if (h == 0) {
      float* pm = p.part_ml + slot * 3 * 256;
      pm[c] = m_run;
      pm[256 + c] = l_tot;
      pm[512 + c] = carry;
    }
    return;
  }
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok) {
    uint16_t* orow = p.out + ((static_cast<int64_t>(b) * p.nq + row) * p.hq + head) * kD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<__bf16>(o[db][4 * j4 + e] * inv);
        *reinterpret_cast<bf16x4*>(orow + 32 * db + 8 * j4 + 4 * h) = w;
      }
  }
  if (bad_block) atomicOr(p.flags, CS_FLAG_BLOCK_INVALID);
}

}  // namespace
}  // namespace cs

using namespace cs;

namespace {
// A second stream per device for the policy checker, so that the check runs
// beside the attention kernel: an event forks it from the caller's stream
// once the shared inputs are staged, and the caller's stream waits for its
// end event.  Default priority; created on first use, kept until the
// process ends.  The mutex covers the fork, the launches and the join.
struct side_lane {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kSideDevices = 64;
std::mutex g_side_mutex;
side_lane g_side[kSideDevices];

int side_lane_of_current(side_lane** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("hipGetDevice: %s", hipGetErrorString(err));
    return CS_ELAUNCH;
  }
  CS_REQUIRE(dev >= 0 && dev < kSideDevices, "device ordinal %d out of range", dev);
  side_lane& l = g_side[dev];
  if (l.stream == nullptr) {
    if ((err = hipStreamCreateWithFlags(&l.stream, hipStreamNonBlocking)) != hipSuccess ||
        (err = hipEventCreateWithFlags(&l.fork, hipEventDisableTiming)) != hipSuccess ||
        (err = hipEventCreateWithFlags(&l.join, hipEventDisableTiming)) != hipSuccess) {
      set_error("policy check stream: %s", hipGetErrorString(err));
      return CS_ELAUNCH;
    }
  }
  *out = &l;
  return CS_OK;
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    cus[dev] = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0 ? v : 256;
  }
  return cus[dev];
}

int fill_kv(const cs_kv_source* kv, cs::kv_addr* a) {
  CS_REQUIRE(kv != nullptr, "null kv source");
  cs::kv_addr r{};
  if (kv->block_table || kv->slots) {
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
    if (kv->slots) {
      CS_REQUIRE(kv->slots_stride >= 0 && kv->side_rows >= 0 && kv->slots_cols > 0, "bad slot map");
      CS_REQUIRE(kv->num_blocks * kv->block_size < (int64_t(1) << 31) && kv->side_rows < (int64_t(1) << 31),
                 "the slot-map prefill needs fewer than 2^31 native slots and sidecar rows");
      if (kv->side_rows > 0)
        CS_REQUIRE(kv->side_k && kv->side_v && (reinterpret_cast<uintptr_t>(kv->side_k) % 16) == 0 &&
                       (reinterpret_cast<uintptr_t>(kv->side_v) % 16) == 0 &&
                       kv->side_s_row % 8 == 0 && kv->side_s_head % 8 == 0 &&
                       kv->side_s_row >= 0 && kv->side_s_head >= 0,
                   "sidecar rows must be 16-byte aligned");
      r.slots = kv->slots;
      r.slots_stride = kv->slots_stride;
      r.slots_cols = kv->slots_cols;
      r.native_slots = kv->num_blocks * kv->block_size;
      r.side_k = static_cast<const uint16_t*>(kv->side_k);
      r.side_v = static_cast<const uint16_t*>(kv->side_v);
      r.side_sr = kv->side_s_row;
      r.side_sh = kv->side_s_head;
      r.side_rows = kv->side_rows;
    } else {
      r.block_table = kv->block_table;
      r.bt_stride = kv->bt_stride;
      r.bt_cols = kv->bt_cols;
      CS_REQUIRE(r.bt_cols > 0, "block table needs at least one column");
    }
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

namespace {

// Validate a prefill call and fill its parameters, LDS size and wave count
// (CS_OK, or an error code with the message set).
int prepare_prefill(const void* q, int64_t q_s_batch, int64_t q_s_tok, int64_t q_s_head,
                    const int64_t* qpos, int64_t qpos_s_batch, int32_t batch, int32_t nq, int32_t hq,
                    int32_t hkv, const int32_t* nk, const cs_kv_source* kv, const float* e,
                    int32_t max_positions, void* out, int32_t* flags, cs::prefill_params* pp,
                    int* waves_out, size_t* smem_out, int max_waves = 8) {
  CS_REQUIRE(q && qpos && nk && e && out && flags, "null arguments");
  CS_REQUIRE(batch >= 0 && nq >= 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "bad head counts");
  CS_REQUIRE(max_positions >= 2 && max_positions <= kMaxPos, "max_positions must be in [2, %d]",
             kMaxPos);
  CS_REQUIRE(q_s_tok % 8 == 0 && q_s_head % 8 == 0 && q_s_batch % 8 == 0 &&
                 (reinterpret_cast<uintptr_t>(q) % 16) == 0,
             "query rows must be 16-byte aligned");
  const int group = hq / hkv;
  if (kCols % group != 0) {
    set_error("GQA group size %d is not supported by the MFMA prefill kernel (it must divide %d)",
              group, kCols);
    return CS_EUNSUPPORTED;
  }
  cs::prefill_params p{};
  int st = fill_kv(kv, &p.kv);
  if (st) return st;
  const bool paged = p.kv.block_table || p.kv.slots;
  if (paged ? (p.kv.s_block >= (1ll << 31) || p.kv.s_offset >= (1ll << 31) || p.kv.s_block < 0 ||
                          p.kv.s_offset < 0)
                       : (p.kv.k_st >= (1ll << 31) || p.kv.v_st >= (1ll << 31) || p.kv.k_st < 0 ||
                          p.kv.v_st < 0)) {
    set_error("the MFMA prefill kernel needs non-negative block / token strides below 2^31");
    return CS_EUNSUPPORTED;
  }
  if (paged && p.kv.bs_shift < 0) {
    set_error("the MFMA prefill kernel needs a power-of-two block size (got %d)", kv->block_size);
    return CS_EUNSUPPORTED;
  }
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
  // fp32 QE table rows of an odd number of words (no bank conflicts between
  // columns).  4 wavefronts (128 columns) while two such workgroups fit in a
  // CU, so one workgroup's prologue and barriers overlap the other's tile
  // loop; else 8 wavefronts (one workgroup, still two waves per SIMD) while
  // its table fits, else 4.
  // P + 1 entries per column (entry P repeats P-1), an odd number of words
  const int tab_stride = (max_positions + 1) | 1;
  auto tab_bytes = [&](int w) { return sizeof(float) * kCols * w * static_cast<size_t>(tab_stride); };
  int waves = 2 * (tab_bytes(4) + kStaticLds) <= kLdsLimit ? 4 : (tab_bytes(8) + kStaticLds <= kLdsLimit ? 8 : 4);
  // A launch of fewer 4-wave workgroups than two per CU (a selective call's
  // few hundred rows) runs 2-wave workgroups: twice as many workgroups share
  // the longest key walks.
  if (static_cast<int64_t>(batch) * hkv * ceil_div(nq, kCols * 4 / group) < 2 * device_cus() &&
      2 * (tab_bytes(2) + kStaticLds) <= kLdsLimit)
    waves = 2;
  // a caller with few rows per workgroup (one per request) asks for narrow ones
  while (waves > max_waves && waves > 2) waves /= 2;
  p.rows_per_wg = kCols * waves / group;
  p.row_blocks = static_cast<int32_t>(ceil_div(nq, p.rows_per_wg));
  p.nk = nk;
  p.e = e;
  p.npos = max_positions;
  p.tab_stride = tab_stride;
  p.out = static_cast<uint16_t*>(out);
  p.flags = flags;
  const int64_t total = static_cast<int64_t>(batch) * hkv * p.row_blocks;
  CS_REQUIRE(total < (1ll << 31), "grid too large");
  p.total_wg = static_cast<int32_t>(total);
  const size_t smem = tab_bytes(waves);
  if (smem + kStaticLds > kLdsLimit) {
    set_error("prefill LDS %zu bytes exceeds the workgroup limit", smem + kStaticLds);
    return CS_EUNSUPPORTED;
  }
  *pp = p;
  *waves_out = waves;
  *smem_out = smem;
  return CS_OK;
}

// Fixed-key bitmap, the dynamic keys beside a fixed key (ascending), the key
// count, and for the checker one code per key: the fixed ordinal (>= 0), -2 - s
// for the dynamic key in boundary slot s, -1 for other dynamic keys.  The fixed
// keys are the selected-association lowering's, or without it the keys with a
// profile ordinal.  One workgroup.
constexpr int kPackThreads = 1024;
constexpr int kMaxBoundary = cs::kPolicyMaxBoundary;

__global__ void __launch_bounds__(kPackThreads) policy_pack_kernel(const uint8_t* fixed_keys,
                                                                  const int64_t* k_ord, int64_t nk,
                                                                  uint32_t* bits, int32_t* bnd_count,
                                                                  int32_t* bnd_keys, int32_t* code,
                                                                  int32_t* nk_dev, int32_t* flags) {
  __shared__ int wave_count[kPackThreads / 64];
  __shared__ int running;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  auto is_fixed = [&](int64_t j) { return fixed_keys ? fixed_keys[j] != 0 : k_ord[j] >= 0; };
  if (tid == 0) {
    running = 0;
    nk_dev[0] = static_cast<int32_t>(nk);
  }
  __shared__ int floor_tile;
  if (tid == 0) floor_tile = INT32_MAX;
  __syncthreads();
  // one pass over the keys, 1024 at a time: the fixed-key bitmap from each
  // wave's ballot (two 32-key words), the lowest word that is not all fixed,
  // and the boundary keys (dynamic keys beside a fixed key) in key order
  for (int64_t base = 0; base < nk; base += kPackThreads) {
    const int64_t j = base + tid;
    const bool fixed = j < nk && is_fixed(j);
    const unsigned long long fm = __ballot(fixed);
    const int64_t w0 = (base + 64 * wave) / 32;  // first word of this wave's 64 keys
    if (lane < 2 && 32 * (w0 + lane) < nk) {
      const uint32_t word = static_cast<uint32_t>(fm >> (32 * lane));
      bits[w0 + lane] = word;
      if (word != 0xFFFFFFFFu) atomicMin(&floor_tile, static_cast<int>(w0 + lane));
    }
    bool bnd = false;
    if (j < nk && !fixed)
      bnd = (j > 0 && is_fixed(j - 1)) || (j + 1 < nk && is_fixed(j + 1));
    const unsigned long long m = __ballot(bnd);
    if (lane == 0) wave_count[wave] = __popcll(m);
    __syncthreads();
    int before = running;
    for (int w = 0; w < wave; ++w) before += wave_count[w];
    before += __popcll(m & ((1ull << lane) - 1ull));
    if (j < nk) {
      const bool kept = bnd && before < kMaxBoundary;
      const int64_t ko = k_ord ? k_ord[j] : -1;
      code[j] = ko >= 0 ? static_cast<int32_t>(ko) : (kept ? -2 - before : -1);
      if (kept) bnd_keys[before] = static_cast<int32_t>(j);
      if (bnd && !kept) atomicOr(flags, CS_FLAG_POLICY_GENERIC);  // more boundary keys than the checker holds
    }
    __syncthreads();
    if (tid == 0) {
      int add = 0;
      for (int w = 0; w < kPackThreads / 64; ++w) add += wave_count[w];
      running += add;
    }
    __syncthreads();
  }
  if (tid == 0) nk_dev[1] = floor_tile;
  if (tid == 0) bnd_count[0] = running < kMaxBoundary ? running : kMaxBoundary;
}

// Per block of 256 keys, for the checker: the offset o when every key j of
// the block is fixed with ordinal j - o, -1 when every key is a dynamic key
// with no fixed neighbour (or past the end), -2 otherwise (the checker then
// reads the block's codes).  One wave per block.
__global__ void __launch_bounds__(256) policy_blocks_kernel(const int32_t* code, int64_t nk, int32_t* blk) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t nb = (nk + 255) / 256;
  if (t >= nb) return;
  const int64_t j0 = t * 256 + 4 * lane;
  int32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = j0 + i < nk ? code[j0 + i] : -1;
  const int64_t first = code[t * 256];
  const int64_t off = t * 256 - first;
  bool affine = first >= 0 && t * 256 + 255 < nk;
  bool plain = true;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    affine = affine && c[i] == j0 + i - off;
    plain = plain && c[i] == -1;
  }
  affine = __all(affine);
  plain = __all(plain);
  if (lane == 0) blk[t] = affine ? static_cast<int32_t>(off) : (plain ? -1 : -2);
}

// Per group of 4 keys (8 groups per 32-key tile, the last tile's padded): the
// ordinal of its first key when all four are fixed with consecutive ordinals
// and their canonical cells can be read as one aligned 16-byte load (aligned:
// the profile's unit key stride and 16-byte rows), else -1.
__global__ void policy_groups_kernel(const int32_t* code, int64_t nk, int32_t aligned, int64_t ngroups,
                                     int32_t* grp) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (g >= ngroups) return;
  const int64_t j = 4 * g;
  int32_t v = -1;
  if (aligned && j + 3 < nk) {
    const int32_t o = code[j];
    if (o >= 0 && (o & 3) == 0 && code[j + 1] == o + 1 && code[j + 2] == o + 2 && code[j + 3] == o + 3) v = o;
  }
  grp[g] = v;
}

// Canonical position of each (head, row)'s own key, NaN when the row is not a
// fixed row the profile covers: canonical[h][q_ord[row]][k_ord[qpos[row]]].
__global__ void policy_self_kernel(const float* canon, int64_t c_s0, int64_t c_s1, int64_t c_s2,
                                   const int64_t* q_ord, const int64_t* k_ord, const int64_t* qpos,
                                   int32_t nq, int32_t hq, int64_t nk, float* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(nq) * hq) return;
  const int h = static_cast<int>(i / nq), row = static_cast<int>(i % nq);
  float v = __builtin_nanf("");
  const int64_t qo = q_ord[row];
  const int64_t qp = qpos[row];
  if (qo >= 0 && qp >= 0 && qp < nk) {
    const int64_t ko = k_ord[qp];
    if (ko >= 0) v = canon[h * c_s0 + qo * c_s1 + ko * c_s2];
  }
  out[i] = v;
}

// ---- key splits of the policy call ------------------------------------------
// A row block holding a row other than a selected fixed row walks every
// causal key (selected rows skip the tiles of fixed keys once their positions
// saturate); the reuse call's few such blocks, the question rows, would
// otherwise hold a handful of compute units for the whole call.
constexpr int kSplitExtra = 256;       // extra-part workgroups of one call, at most
constexpr int kSplitMaxParts = 8;      // parts per row block
constexpr int kSplitMarginTiles = 16;  // tiles part 0 walks below the row block's lowest diagonal
constexpr int kSplitMinTiles = 32;     // tiles per far part, at least
constexpr int kSplitSlots = 2 * kSplitExtra;  // part states: every split block has >= 1 extra part
constexpr int kPlanThreads = 1024;

// One workgroup, batch item 0.  Per row block, last first (the heaviest):
// parts, first slot and split tile, the same for every KV head.  A row block
// is eligible when it holds a row that is not a selected fixed row and its
// lowest row lies at least kSplitMarginTiles + 2 kSplitMinTiles tiles from
// key 0; the kSplitExtra extra parts are shared among the eligible blocks in
// proportion to the tiles below their split (a block whose share rounds to 0
// stays whole), at most kSplitMaxParts parts and kSplitMinTiles tiles per far
// part.  split_items lists the extra parts, split_blocks the split
// workgroups; unused entries are -1.
__global__ void __launch_bounds__(kPlanThreads) policy_split_plan_kernel(cs::prefill_params p, int32_t* plan,
                                                                        int32_t* items, int32_t* blocks) {
  __shared__ int wave_sum[2][kPlanThreads / 64];
  __shared__ int running[2];
  __shared__ unsigned long long total_far;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kSplitExtra; i += kPlanThreads) {
    items[i] = -1;
    blocks[i] = -1;
  }
  if (tid == 0) {
    running[0] = running[1] = 0;
    total_far = 0;
  }
  __syncthreads();
  const int nk = p.nk[0];
  // tiles below the split of the k-th heaviest row block, 0 when not eligible
  auto far_of = [&](int k) -> int64_t {
    const int rb = p.row_blocks - 1 - k;
    int64_t lo = INT64_MAX, hi = -1;
    bool heavy = false;
    const int r0 = rb * p.rows_per_wg;
    const int r1 = r0 + p.rows_per_wg < p.nq ? r0 + p.rows_per_wg : p.nq;
    for (int r = r0; r < r1; ++r) {
      const int64_t q = p.qpos[r];
      lo = q < lo ? q : lo;
      hi = q > hi ? q : hi;
      heavy = heavy || !(p.sel_rows && p.sel_rows[r]);
    }
    const int64_t far = (lo < nk ? lo : nk) / kTileN - kSplitMarginTiles;
    return heavy && hi >= 0 && far >= 2 * kSplitMinTiles ? far : 0;
  };
  for (int k = tid; k < p.row_blocks; k += kPlanThreads) {
    const int64_t f = far_of(k);
    if (f > 0) atomicAdd(&total_far, static_cast<unsigned long long>(f));
  }
  __syncthreads();
  const int64_t sum_far = static_cast<int64_t>(total_far);
  const int64_t budget = kSplitExtra / p.hkv;  // extra parts per KV head
  for (int base = 0; base < p.row_blocks; base += kPlanThreads) {
    const int k = base + tid;  // k-th heaviest row block
    int parts = 1, t_split = 0;
    if (k < p.row_blocks) {
      const int64_t far = far_of(k);
      if (far > 0) {
        int64_t extra = budget * far / sum_far;
        extra = extra < kSplitMaxParts - 1 ? extra : kSplitMaxParts - 1;
        extra = extra < far / kSplitMinTiles - 1 ? extra : far / kSplitMinTiles - 1;
        if (extra >= 1) {
          parts = static_cast<int>(1 + extra);
          t_split = static_cast<int>(far);
        }
      }
    }
    // exclusive scans of the split blocks and of their parts (per KV head)
    int cnt[2] = {parts > 1 ? 1 : 0, parts > 1 ? parts : 0};
    int incl[2] = {cnt[0], cnt[1]};
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int v = __shfl_up(incl[j], off, 64);
        if (lane >= off) incl[j] += v;
      }
    }
    if (lane == 63) {
      wave_sum[0][wave] = incl[0];
      wave_sum[1][wave] = incl[1];
    }
    __syncthreads();
    int before[2] = {running[0] + incl[0] - cnt[0], running[1] + incl[1] - cnt[1]};
    for (int w = 0; w < wave; ++w) {
      before[0] += wave_sum[0][w];
      before[1] += wave_sum[1][w];
    }
    if (k < p.row_blocks) {
      // per KV head: before[0] blocks and before[1] parts precede, so
      // before[1] - before[0] extra parts; slots are the parts
      const int extra0 = p.hkv * (before[1] - before[0]);
      for (int kvh = 0; kvh < p.hkv; ++kvh) {
        const int logical = kvh * p.row_blocks + k;
        plan[3 * logical] = parts;
        plan[3 * logical + 1] = parts > 1 ? p.hkv * before[1] + kvh * parts : 0;
        plan[3 * logical + 2] = t_split;
        if (parts > 1) {
          blocks[p.hkv * before[0] + kvh] = logical;
          for (int q = 1; q < parts; ++q) items[extra0 + kvh * (parts - 1) + q - 1] = logical * 16 + q;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 0; w < kPlanThreads / 64; ++w) {
        running[0] += wave_sum[0][w];
        running[1] += wave_sum[1][w];
      }
    }
    __syncthreads();
  }
}

// The output of the split row blocks: per column, the parts' states combined
// against their common maximum (the softmax over the union of the parts'
// keys).  16 workgroups per split block (8 dims each), one thread per column.
constexpr int kMergeDims = 8;
__global__ void __launch_bounds__(256) policy_split_merge_kernel(cs::prefill_params p) {
  const int i = static_cast<int>(blockIdx.x) / (kD / kMergeDims);
  const int d0 = static_cast<int>(blockIdx.x % (kD / kMergeDims)) * kMergeDims;
  const int logical = p.split_blocks[i];
  if (logical < 0) return;
  const int nparts = p.split_plan[3 * logical];
  const int64_t slot0 = p.split_plan[3 * logical + 1];
  int b, kvh, rb;
  decode_logical(p, logical, b, kvh, rb);
  const int c = threadIdx.x;
  const int row = rb * p.rows_per_wg + c / p.group;
  if (c >= p.rows_per_wg * p.group || row >= p.nq) return;
  const int head = kvh * p.group + c % p.group;
  constexpr float kC = kInvSqrtD * kLog2e;
  float mx = -INFINITY;
  for (int s = 0; s < nparts; ++s) mx = fmaxf(mx, p.part_ml[(slot0 + s) * 3 * 256 + c]);
  float wt[kSplitMaxParts];
  float l = 0.f;
#pragma unroll
  for (int s = 0; s < kSplitMaxParts; ++s) {
    wt[s] = 0.f;
    if (s < nparts && mx != -INFINITY) {
      const float* pm = p.part_ml + (slot0 + s) * 3 * 256;
      wt[s] = pm[c] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((pm[c] - mx) * kC);
      l += wt[s] * pm[256 + c];
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float acc[kMergeDims] = {};
#pragma unroll
  for (int s = 0; s < kSplitMaxParts; ++s) {
    if (s < nparts) {
      const float* po = p.part_o + (slot0 + s) * kD * 256 + d0 * 256 + c;
#pragma unroll
      for (int j = 0; j < kMergeDims; ++j) acc[j] += wt[s] * po[j * 256];
    }
  }
  uint4 packed;
  packed.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  packed.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  packed.z = pack_bf16x2(acc[4] * inv, acc[5] * inv);
  packed.w = pack_bf16x2(acc[6] * inv, acc[7] * inv);
  *reinterpret_cast<uint4*>(p.out + (static_cast<int64_t>(row) * p.hq + head) * kD + d0) = packed;
}

// CS_POLICY_KEY_SPLIT=0 in the environment turns the key splits off, for
// timing the split launch against the unsplit one.
bool no_split() {
  static const bool off = [] {
    const char* v = std::getenv("CS_POLICY_KEY_SPLIT");
    return v != nullptr && v[0] == '0';
  }();
  return off;
}

constexpr int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

struct policy_ws {
  int32_t* nk_dev;
  uint32_t* bits;
  int32_t* bnd_count;
  int32_t* bnd_keys;
  int32_t* code;
  int32_t* blk;
  float* canon_self;
  int32_t* grp;
  int64_t ngroups;
  int32_t* plan;
  int32_t* items;
  int32_t* blocks;
  float* part_o;
  float* part_ml;
  bool split;  // the key range is long enough for a split
  int64_t bytes;
};

policy_ws carve_policy(char* base, int32_t nq, int32_t hq, int64_t nk) {
  policy_ws w{};
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* at = base ? base + off : nullptr;
    off += align256(bytes);
    return at;
  };
  w.nk_dev = reinterpret_cast<int32_t*>(take(16));
  w.bits = reinterpret_cast<uint32_t*>(take(4 * ((nk + 31) / 32)));
  w.bnd_count = reinterpret_cast<int32_t*>(take(16));
  w.bnd_keys = reinterpret_cast<int32_t*>(take(4 * kMaxBoundary));
  w.code = reinterpret_cast<int32_t*>(take(4 * nk));
  w.blk = reinterpret_cast<int32_t*>(take(4 * ((nk + 255) / 256)));
  w.canon_self = reinterpret_cast<float*>(take(4 * static_cast<int64_t>(nq) * hq));
  w.ngroups = 8 * ((nk + 31) / 32);
  w.grp = reinterpret_cast<int32_t*>(take(4 * w.ngroups));
  // key splits: a plan entry per logical workgroup (at most
  // Hq (nq / 64 + 1): 64 / G rows per 2-wave workgroup), and the part states
  w.split = nk >= static_cast<int64_t>(kTileN) * (kSplitMarginTiles + 2 * kSplitMinTiles);
  if (w.split) {
    w.plan = reinterpret_cast<int32_t*>(take(4 * 3 * static_cast<int64_t>(hq) * (nq / 64 + 1)));
    w.items = reinterpret_cast<int32_t*>(take(4 * kSplitExtra));
    w.blocks = reinterpret_cast<int32_t*>(take(4 * kSplitExtra));
    w.part_o = reinterpret_cast<float*>(take(4ll * kSplitSlots * kD * 256));
    w.part_ml = reinterpret_cast<float*>(take(4ll * kSplitSlots * 3 * 256));
  }
  w.bytes = off;
  return w;
}

}  // namespace

extern "C" int cs_ccpe_prefill_bf16(const void* q, int64_t q_s_batch, int64_t q_s_tok,
                                    int64_t q_s_head, const int64_t* qpos, int64_t qpos_s_batch,
                                    int32_t batch, int32_t nq, int32_t hq, int32_t hkv,
                                    const int32_t* nk, const cs_kv_source* kv, const float* e,
                                    int32_t max_positions, void* out, int32_t* flags,
                                    void* stream) {
  cs::prefill_params p{};
  int waves = 4;
  size_t smem = 0;
  const int st = prepare_prefill(q, q_s_batch, q_s_tok, q_s_head, qpos, qpos_s_batch, batch, nq, hq,
                                 hkv, nk, kv, e, max_positions, out, flags, &p, &waves, &smem);
  if (st) return st;
  if (batch == 0 || nq == 0) return CS_OK;
  const dim3 grid(p.total_wg), block(64 * waves);
  hipStream_t s = as_stream(stream);
  const int mode = p.kv.slots ? 2 : (p.kv.block_table ? 1 : 0);
  if (mode == 2 && waves == 8)
    hipLaunchKernelGGL((ccpe_prefill_kernel<2, 8>), grid, block, smem, s, p);
  else if (mode == 2 && waves == 2)
    hipLaunchKernelGGL((ccpe_prefill_kernel<2, 2>), grid, block, smem, s, p);
  else if (mode == 2)
    hipLaunchKernelGGL((ccpe_prefill_kernel<2, 4>), grid, block, smem, s, p);
  else if (mode == 1 && waves == 8)
    hipLaunchKernelGGL((ccpe_prefill_kernel<1, 8>), grid, block, smem, s, p);
  else if (mode == 1 && waves == 2)
    hipLaunchKernelGGL((ccpe_prefill_kernel<1, 2>), grid, block, smem, s, p);
  else if (mode == 1)
    hipLaunchKernelGGL((ccpe_prefill_kernel<1, 4>), grid, block, smem, s, p);
  else if (waves == 8)
    hipLaunchKernelGGL((ccpe_prefill_kernel<0, 8>), grid, block, smem, s, p);
  else if (waves == 2)
    hipLaunchKernelGGL((ccpe_prefill_kernel<0, 2>), grid, block, smem, s, p);
  else
    hipLaunchKernelGGL((ccpe_prefill_kernel<0, 4>), grid, block, smem, s, p);
  CS_LAUNCH_CHECK("ccpe_prefill");
  return CS_OK;
}

namespace cs {

// The paged MFMA prefill writing softmax states (state_o, state_ml: see
// prefill_params) instead of output rows; saturated: every position taken as
// P-1; zero_word (may be null) is set to 0.  Workgroups of at most max_waves
// wavefronts.
int launch_prefill_states(const void* q, int64_t q_s_batch, int64_t q_s_tok, int64_t q_s_head,
                          const int64_t* qpos, int64_t qpos_s_batch, int32_t batch, int32_t nq, int32_t hq,
                          int32_t hkv, const int32_t* nk, const cs_kv_source* kv, const float* e,
                          int32_t max_positions, int32_t saturated, int max_waves, float* state_o,
                          float* state_ml, int32_t* zero_word, int32_t* flags, hipStream_t s) {
  CS_REQUIRE(state_o && state_ml, "null state buffers");
  cs::prefill_params p{};
  int waves = 4;
  size_t smem = 0;
  const int st = prepare_prefill(q, q_s_batch, q_s_tok, q_s_head, qpos, qpos_s_batch, batch, nq, hq, hkv, nk, kv,
                                 e, max_positions, state_o, flags, &p, &waves, &smem, max_waves);
  if (st) return st;
  if (batch == 0 || nq == 0) return CS_OK;
  p.state_o = state_o;
  p.state_ml = state_ml;
  p.saturated = saturated ? 1 : 0;
  p.zero_word = zero_word;
  const dim3 grid(p.total_wg), block(64 * waves);
  const int mode = p.kv.slots ? 2 : (p.kv.block_table ? 1 : 0);
  CS_REQUIRE(mode == 1, "softmax states are written for block-table calls only");
  if (waves == 8)
    hipLaunchKernelGGL((ccpe_prefill_kernel<1, 8>), grid, block, smem, s, p);
  else if (waves == 2)
    hipLaunchKernelGGL((ccpe_prefill_kernel<1, 2>), grid, block, smem, s, p);
  else
    hipLaunchKernelGGL((ccpe_prefill_kernel<1, 4>), grid, block, smem, s, p);
  CS_LAUNCH_CHECK("ccpe_prefill_states");
  return CS_OK;
}

}  // namespace cs

extern "C" int cs_prepare_device(void) {
  std::lock_guard<std::mutex> lock(g_side_mutex);
  side_lane* side = nullptr;
  return side_lane_of_current(&side);
}

extern "C" int64_t cs_ccpe_prefill_policy_workspace_bytes(int32_t nq, int32_t hq, int64_t nk) {
  if (nq < 0 || hq <= 0 || nk < 0) return 0;
  return carve_policy(nullptr, nq, hq, nk).bytes;
}

extern "C" int cs_ccpe_prefill_policy_bf16(const cs_ccpe_args* a, void* workspace,
                                           int64_t workspace_bytes, void* stream) {
  CS_REQUIRE(a != nullptr, "null arguments");
  const cs_view& qv = a->q;
  const cs_view& kv = a->k;
  const cs_view& vv = a->v;
  const cs_view& ev = a->e;
  CS_REQUIRE(qv.data && kv.data && vv.data && ev.data && a->out.data && a->qpos && a->flags,
             "null arguments");
  CS_REQUIRE(qv.ndim == 3 && kv.ndim == 3 && vv.ndim == 3 && a->out.ndim == 3,
             "q, k, v and out must be [tokens, heads, 128]");
  CS_REQUIRE(qv.dtype == CS_BF16 && kv.dtype == CS_BF16 && vv.dtype == CS_BF16 && a->out.dtype == CS_BF16,
             "the MFMA policy prefill takes bf16 q, k, v and out");
  CS_REQUIRE(qv.shape[2] == kD && kv.shape[2] == kD && vv.shape[2] == kD && a->out.shape[2] == kD,
             "the MFMA policy prefill needs head dim 128");
  CS_REQUIRE(kv.shape[0] == vv.shape[0] && kv.shape[1] == vv.shape[1], "K and V must match");
  CS_REQUIRE(a->out.shape[0] == qv.shape[0] && a->out.shape[1] == qv.shape[1] && a->out.stride[2] == 1 &&
                 a->out.stride[1] == kD && a->out.stride[0] == kD * qv.shape[1],
             "out must be contiguous [nq, Hq, 128]");
  CS_REQUIRE(qv.stride[2] == 1 && kv.stride[2] == 1 && vv.stride[2] == 1, "rows must be contiguous");
  CS_REQUIRE(ev.dtype == CS_F32 && ev.ndim == 2 && ev.shape[0] == kD && ev.stride[1] == 1 &&
                 ev.stride[0] == ev.shape[1],
             "e must be contiguous fp32 [128, P]");
  CS_REQUIRE(a->kpos == nullptr, "the MFMA policy prefill takes the default key coordinates 0..nk-1");
  CS_REQUIRE(!a->attn_mask.data && !a->vis_mask.data && !a->fixed_pos.data && !a->pos_out.data,
             "the MFMA policy prefill takes no masks, fixed positions or position output");
  const bool canon = a->canonical.data != nullptr;
  CS_REQUIRE((a->sel_rows && a->fixed_keys) || (!a->sel_rows && !a->fixed_keys && canon),
             "the MFMA policy prefill needs the selected-row lowering, a canonical profile or both");
  if (canon) {
    const cs_view& c = a->canonical;
    CS_REQUIRE(c.ndim == 3 && c.shape[0] == qv.shape[1] && c.dtype == CS_F32 && a->q_ord && a->k_ord &&
                   a->chunk_flags && a->chunk_rows > 0,
               "canonical must be fp32 [Hq, F, F] with ordinal maps and chunk flags");
  }
  const int64_t nq64 = qv.shape[0], nk = kv.shape[0];
  CS_REQUIRE(nq64 < (1ll << 31) && nk < (1ll << 31), "too many rows or keys");
  const int32_t nq = static_cast<int32_t>(nq64), hq = static_cast<int32_t>(qv.shape[1]);
  const int32_t hkv = static_cast<int32_t>(kv.shape[1]);
  const policy_ws need = carve_policy(nullptr, nq, hq, nk);
  CS_REQUIRE(workspace != nullptr && workspace_bytes >= need.bytes &&
                 (reinterpret_cast<uintptr_t>(workspace) % 256) == 0,
             "policy workspace holds %lld bytes, the call needs %lld (256-byte aligned)",
             static_cast<long long>(workspace_bytes), static_cast<long long>(need.bytes));
  const policy_ws w = carve_policy(static_cast<char*>(workspace), nq, hq, nk);
  cs_kv_source src{};
  src.k = kv.data;
  src.v = vv.data;
  src.k_s_tok = kv.stride[0];
  src.k_s_head = kv.stride[1];
  src.v_s_tok = vv.stride[0];
  src.v_s_head = vv.stride[1];
  cs::prefill_params p{};
  int waves = 4;
  size_t smem = 0;
  const int st = prepare_prefill(qv.data, 0, qv.stride[0], qv.stride[1], a->qpos, 0, 1, nq, hq, hkv, w.nk_dev,
                                 &src, static_cast<const float*>(ev.data), static_cast<int32_t>(ev.shape[1]),
                                 a->out.data, a->flags, &p, &waves, &smem);
  if (st) return st;
  if (nq == 0) return CS_OK;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(policy_pack_kernel, dim3(1), dim3(kPackThreads), 0, s, a->fixed_keys,
                     canon ? a->k_ord : nullptr, nk, w.bits, w.bnd_count, w.bnd_keys, w.code, w.nk_dev,
                     a->flags);
  p.sel_rows = a->sel_rows;
  p.fixed_bits = w.bits;
  p.dyn_floor = w.nk_dev + 1;
  if (canon) {
    const cs_view& c = a->canonical;
    const int64_t cells = static_cast<int64_t>(nq) * hq;
    hipLaunchKernelGGL(policy_self_kernel, dim3(static_cast<uint32_t>((cells + 255) / 256)), dim3(256), 0, s,
                       static_cast<const float*>(c.data), c.stride[0], c.stride[1], c.stride[2], a->q_ord,
                       a->k_ord, a->qpos, nq, hq, nk, w.canon_self);
    p.canon_self = w.canon_self;
    p.q_ord = a->q_ord;
    // fixed rows that are not selected read their canonical cells directly
    const bool aligned = c.stride[2] == 1 && c.stride[0] % 4 == 0 && c.stride[1] % 4 == 0 &&
                         (reinterpret_cast<uintptr_t>(c.data) % 16) == 0;
    hipLaunchKernelGGL(policy_groups_kernel, dim3(static_cast<uint32_t>((w.ngroups + 255) / 256)), dim3(256), 0,
                       s, w.code, static_cast<int64_t>(nk), aligned ? 1 : 0, w.ngroups, w.grp);
    p.canon = static_cast<const float*>(c.data);
    p.c_s0 = c.stride[0];
    p.c_s1 = c.stride[1];
    p.c_s2 = c.stride[2];
    p.grp = w.grp;
    p.code = w.code;
  }
  // Key splits of the row blocks that walk every causal key (planned on the
  // device from the rows' positions and the selected set), when no checker
  // runs beside the attention: with one, the two kernels already fill the
  // device, the checker's reads bound the call, and the split parts only take
  // compute units from it (1.39 against 1.30 ms per reuse call at 16k keys).
  const bool split = w.split && !canon && !no_split();
  if (split) {
    p.split_extra = kSplitExtra;
    p.split_plan = w.plan;
    p.split_items = w.items;
    p.split_blocks = w.blocks;
    p.part_o = w.part_o;
    p.part_ml = w.part_ml;
    hipLaunchKernelGGL(policy_split_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p, w.plan, w.items, w.blocks);
  }
  // The attention kernel is queued first, so that its longest workgroups
  // (rows whose walks cover every causal key) are dispatched at once; the
  // checker, forked after the lowering kernels and the checker's block
  // descriptors (queued here, ahead of the attention, so that they do not
  // wait behind it for compute units), then fills the compute units the
  // attention's short workgroups leave.
  std::unique_lock<std::mutex> side_lock(g_side_mutex, std::defer_lock);
  side_lane* side = nullptr;
  if (canon) {
    const int64_t nb = (static_cast<int64_t>(nk) + 255) / 256;
    if (nb > 0)
      hipLaunchKernelGGL(policy_blocks_kernel, dim3(static_cast<uint32_t>((nb + 3) / 4)), dim3(256), 0, s,
                         w.code, static_cast<int64_t>(nk), w.blk);
    side_lock.lock();
    const int sst = side_lane_of_current(&side);
    if (sst) return sst;
    hipError_t err = hipEventRecord(side->fork, s);
    if (err == hipSuccess) err = hipStreamWaitEvent(side->stream, side->fork, 0);
    if (err != hipSuccess) {
      set_error("policy check fork: %s", hipGetErrorString(err));
      return CS_ELAUNCH;
    }
  }
  auto launch_attention = [&](const cs::prefill_params& lp, uint32_t wgs) {
    const dim3 grid(wgs), block(64 * waves);
    if (waves == 8)
      hipLaunchKernelGGL((ccpe_prefill_kernel<0, 8, true>), grid, block, smem, s, lp);
    else if (waves == 2)
      hipLaunchKernelGGL((ccpe_prefill_kernel<0, 2, true>), grid, block, smem, s, lp);
    else
      hipLaunchKernelGGL((ccpe_prefill_kernel<0, 4, true>), grid, block, smem, s, lp);
  };
  if (split) {
    // the extra parts first: they are as long as the longest whole blocks
    p.split_role = 1;
    launch_attention(p, static_cast<uint32_t>(kSplitExtra) + static_cast<uint32_t>(p.total_wg));
    CS_LAUNCH_CHECK("ccpe_prefill_policy");
    hipLaunchKernelGGL(policy_split_merge_kernel, dim3(kSplitExtra * (kD / kMergeDims)), dim3(256), 0, s, p);
    CS_LAUNCH_CHECK("ccpe_prefill_policy_merge");
    cs::prefill_params fix = p;
    fix.split_role = 2;
    launch_attention(fix, kSplitExtra);
    CS_LAUNCH_CHECK("ccpe_prefill_policy_fixup");
  } else {
    launch_attention(p, static_cast<uint32_t>(p.total_wg));
    CS_LAUNCH_CHECK("ccpe_prefill_policy");
  }
  if (canon) {
    cs::policy_check_args c{};
    c.q = static_cast<const uint16_t*>(qv.data);
    c.q_s_tok = qv.stride[0];
    c.q_s_head = qv.stride[1];
    c.k = static_cast<const uint16_t*>(kv.data);
    c.k_s_tok = kv.stride[0];
    c.k_s_head = kv.stride[1];
    c.qpos = a->qpos;
    c.nq = nq;
    c.hq = hq;
    c.group = hq / hkv;
    c.nk = nk;
    c.canon = static_cast<const float*>(a->canonical.data);
    c.c_s0 = a->canonical.stride[0];
    c.c_s1 = a->canonical.stride[1];
    c.c_s2 = a->canonical.stride[2];
    c.q_ord = a->q_ord;
    c.code = w.code;
    c.blk = w.blk;
    c.bnd_count = w.bnd_count;
    c.bnd_keys = w.bnd_keys;
    c.npos = static_cast<int32_t>(ev.shape[1]);
    c.strict = a->strict;
    c.chunk_rows = a->chunk_rows;
    c.chunk_flags = a->chunk_flags;
    const int cst = cs::launch_policy_check(c, side->stream);
    if (cst) return cst;
    hipError_t err = hipEventRecord(side->join, side->stream);
    if (err == hipSuccess) err = hipStreamWaitEvent(s, side->join, 0);
    if (err != hipSuccess) {
      set_error("policy check join: %s", hipGetErrorString(err));
      return CS_ELAUNCH;
    }
  }
  return CS_OK;
}
