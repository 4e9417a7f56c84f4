// Declarations of the MFMA prefill kernel (ccpe_prefill.hip): operand types,
// tile geometry, the K/V addressing and launch parameters, and the direct
// global -> LDS tile loads.
#pragma once

#include "common.h"

namespace cs {

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
  const int64_t* slots;  // per-token slot map (mode 2)
  int64_t slots_stride, slots_cols;
  int64_t native_slots;  // num_blocks * block_size (< 2^31)
  const uint16_t* side_k;
  const uint16_t* side_v;
  int64_t side_sr, side_sh, side_rows;
};

// Slot-map window entries (mode 2): a native slot (< 2^31), kSideTag | sidecar
// row, or kNoSlot for an invalid slot.
constexpr uint32_t kSideTag = 0x80000000u;
constexpr uint32_t kNoSlot = 0xFFFFFFFFu;

struct prefill_params {
  const uint16_t* q;
  int64_t q_sb, q_st, q_sh;
  const int64_t* qpos;
  int64_t qpos_sb;
  int32_t batch, nq, hq, hkv, group, rows_per_wg, row_blocks, total_wg;
  const int32_t* nk;
  kv_addr kv;
  const float* e;
  int32_t npos, tab_stride;
  uint16_t* out;
  int32_t* flags;
  // Policy lowering (dense calls of the POLICY variant): selected rows, fixed
  // keys as a bitmap (bit j % 32 of word j / 32), the canonical position of
  // each (head, row)'s own key (NaN: no substitution) and the fixed-row map.
  const uint8_t* sel_rows;
  const uint32_t* fixed_bits;
  const float* canon_self;  // [hq, nq]
  const int64_t* q_ord;     // -1: not a fixed row
  // CanonicalPositionPolicy for fixed rows that are not selected: every fixed
  // key takes canonical[head][q_ord[row]][ordinal of the key] (strides in
  // floats); grp[g] is the ordinal of key 4g when keys 4g .. 4g+3 are fixed
  // with consecutive ordinals (else -1), code[j] the ordinal of fixed key j.
  const float* canon;
  int64_t c_s0, c_s1, c_s2;
  const int32_t* grp;
  const int32_t* code;
  // the lowest tile whose 32 keys are not all fixed (INT32_MAX: none)
  const int32_t* dyn_floor;
  // Key splits of the POLICY variant (split_role 0: none).  Role 1, the
  // attention launch: workgroups [0, split_extra) run the extra parts listed
  // in split_items (-1: unused), the others the row blocks in the usual
  // order, part 0 of a split block.  Role 2, the fix-up launch: workgroup i
  // walks split block split_blocks[i] (-1: none) unsplit when its part 0 left
  // a column's positions below P-1, and writes the output.
  int32_t split_role, split_extra;
  const int32_t* split_plan;    // per logical workgroup: parts, first slot, split tile
  const int32_t* split_items;   // extra parts: logical workgroup * 16 + part
  const int32_t* split_blocks;  // logical workgroups that are split
  float* part_o;                // [slot][128 dims][256 columns] unnormalised output
  float* part_ml;               // [slot][3][256 columns] running max, sum, carry
  // Softmax states instead of output rows (state_o non-null): per (batch
  // item, row, head) the output unnormalised against the running max of the
  // raw scores q.k, and (max, sum, carry).  saturated: every position is
  // taken as P-1 (the carry starts there), for keys whose positions the
  // caller has shown to be saturated.
  float* state_o;   // [B, nq, Hq, 128]
  float* state_ml;  // [B, nq, Hq, 3]
  int32_t saturated;
  int32_t* zero_word;  // when non-null, set to 0 by the launch (a flag a later launch raises)
};

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_tr;
#define CS_LDS __attribute__((address_space(3)))

constexpr int kD = 128;
constexpr int kCols = 32;  // (row, head) columns per wave
constexpr int kTileN = 32;               // keys per tile
constexpr int kChunks = 16;              // 16-byte chunks of a 256-byte K or V row
constexpr int kStageSlots = kTileN * kChunks;  // uint4 slots of one K (or V) stage
constexpr int kMaxPos = 128;
constexpr int kPosChunk = 64;  // E^T positions staged per pass (bf16 hi and lo, 16 KB each)
constexpr int kBtWindow = 1024;  // block-table (or slot-map) entries held in LDS at a time
constexpr size_t kLdsLimit = 160 * 1024;
constexpr float kInvSqrtD = 0.08838834764831845f;  // 1/sqrt(128)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kSqrtD = 11.313708498984761f;  // sqrt(128)
constexpr float kLn2 = 0.6931471805599453f;

// Exchange with lane l ^ 32: v_permlane32_swap of x with itself leaves
// {x[l], x[l ^ 32]} in the two results, in an order that depends on the half.
__device__ inline void swap_halves(float x, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}

__device__ inline uint32_t pack_bf16x2(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in [15:14]).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Keys past the causal range and keys of invalid blocks are loaded from this
// zero record (256 bf16), so every tile load is issued unconditionally.
__device__ __attribute__((aligned(16))) uint32_t g_zero_record[kD] = {};

__device__ inline bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Direct global -> LDS load of 16 bytes per lane: lane i's bytes land at LDS
// byte address lds + 16 i (lds wave-uniform, in an SGPR).  Issued through
// inline assembly so the compiler does not tie later LDS reads to it;
// completion is made visible only by the explicit vmcnt wait and barrier of
// the tile loop.
__device__ inline void lds_dma16(const void* gptr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               : : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(gptr) : "memory", "m0");
}

// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// byte offset (the instruction's saddr form): no per-lane address arithmetic.
__device__ inline void lds_dma16_s(uint32_t voff, uint64_t sbase, uint32_t lds) {
  // readfirstlane returns int: each half goes through uint32_t so that widening
  // never sign-extends the low word
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(sbase >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(sbase)));
  const uint64_t base = (static_cast<uint64_t>(hi) << 32) | lo;
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               : : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(base) : "memory", "m0");
}

// Element i of a read-only array at a wave-uniform index, through the
// constant address space: a scalar load, which the vector-memory waits of
// the tile loop do not count.
template <typename T>
__device__ inline T uniform_load(const T* ptr, int64_t i) {
  return ((const __attribute__((address_space(4))) T*)ptr)[i];
}

// 16 bytes of global memory into registers without the compiler tracking the
// load: the caller waits for it with an explicit vmcnt wait and then passes
// the value through an empty asm before its first use.
__device__ inline floatx4 load_f4_untracked(const float* ptr) {
  floatx4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(ptr) : "memory");
  return r;
}

// LDS byte address of a __shared__ object (the generic -> LDS conversion,
// done once outside the tile loop)
__device__ inline uint32_t lds_address(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((CS_LDS const void*)p)));
}

// Flat workgroup id -> logical workgroup -> (batch, kv head, row block).
// Dispatch is round-robin over the 8 XCDs by id, so contiguous logical
// ranges are spread as one per XCD: a (batch, kv head)'s K/V stays in one
// XCD's L2.  The heaviest (right-most) row blocks go first.
__device__ inline int logical_wg(const prefill_params& p, int id) {
  return p.total_wg % 8 == 0 ? (id % 8) * (p.total_wg / 8) + id / 8 : id;
}

__device__ inline void decode_logical(const prefill_params& p, int logical, int& b, int& kvh, int& rb) {
  rb = p.row_blocks - 1 - (logical % p.row_blocks);
  const int rest = logical / p.row_blocks;
  kvh = rest % p.hkv;
  b = rest / p.hkv;
}

__device__ inline void decode_wg(const prefill_params& p, int& b, int& kvh, int& rb) {
  decode_logical(p, logical_wg(p, static_cast<int>(blockIdx.x)), b, kvh, rb);
}

struct stage_t {
  uint4 k[kStageSlots];
  uint4 v[kStageSlots];
};

}  // namespace
}  // namespace cs
