// The strict contextual-path checks of validate_contextual_path
// (position.py:98-114), shared by the generic CCPE kernel and the policy
// checker of the MFMA prefill.
#pragma once

#include "common.h"

namespace cs {

template <typename TP> struct pos_traits;
template <> struct pos_traits<float> {
  __device__ static float eps() { return 1.1920928955078125e-07f; }  // 2^-23
};
template <> struct pos_traits<double> {
  __device__ static double eps() { return 2.220446049250313e-16; }  // 2^-52
};

// The strict path checks of validate_contextual_path (position.py:98-114) for
// one valid cell and (optionally) its valid right-hand neighbour, evaluated
// with the reference's operation order and no contraction.
template <typename TP>
__device__ inline int path_violations(TP p, bool valid, TP p_right, bool pair_valid,
                                      int64_t qp, int64_t kp, int64_t kp_right, TP atol) {
#pragma clang fp contract(off)
  int bits = 0;
  if (!valid) return 0;
  const TP eps = pos_traits<TP>::eps();
  TP rounding = eps * (p < 0 ? -p : p);
  TP neg_tol = atol + rounding;
  if (p < -neg_tol) bits |= CS_FLAG_PATH_NEGATIVE;
  int64_t diff = qp - kp;
  TP available = static_cast<TP>(diff);
  if (available < TP(-1)) available = TP(-1);
  available = available + TP(1);
  TP upper = available + atol;
  upper = upper + rounding;
  if (p > upper) bits |= CS_FLAG_PATH_AVAILABLE;
  if (pair_valid) {
    TP r_right = eps * (p_right < 0 ? -p_right : p_right);
    TP d = p - p_right;
    TP pair_tol = atol + rounding;
    pair_tol = pair_tol + r_right;
    if (d < -pair_tol) bits |= CS_FLAG_PATH_INCREASING;
    TP gap = static_cast<TP>(kp_right - kp);
    TP gap_tol = gap + pair_tol;
    if (d > gap_tol) bits |= CS_FLAG_PATH_GAP;
  }
  return bits;
}

// path_violations<float> for keys at coordinates 0..n-1 (a unit gap to the
// right-hand neighbour), with diff = qp - kp >= 0: the same operations in the
// same order, 32-bit coordinates.
__device__ inline int path_violations_unit(float p, bool valid, float p_right, bool pair_valid, int32_t diff,
                                           float atol) {
#pragma clang fp contract(off)
  int bits = 0;
  if (!valid) return 0;
  const float eps = pos_traits<float>::eps();
  const float rounding = eps * (p < 0 ? -p : p);
  const float neg_tol = atol + rounding;
  if (p < -neg_tol) bits |= CS_FLAG_PATH_NEGATIVE;
  float available = static_cast<float>(diff);
  available = available + 1.f;
  float upper = available + atol;
  upper = upper + rounding;
  if (p > upper) bits |= CS_FLAG_PATH_AVAILABLE;
  if (pair_valid) {
    const float r_right = eps * (p_right < 0 ? -p_right : p_right);
    const float d = p - p_right;
    float pair_tol = atol + rounding;
    pair_tol = pair_tol + r_right;
    if (d < -pair_tol) bits |= CS_FLAG_PATH_INCREASING;
    const float gap_tol = 1.f + pair_tol;
    if (d > gap_tol) bits |= CS_FLAG_PATH_GAP;
  }
  return bits;
}

// chunk bits of the canonical-policy lowering (besides CS_FLAG_PATH_*)
constexpr int32_t kChunkHasFixedRow = 1 << 30;       // the chunk holds a fixed query row
constexpr int32_t kChunkUnknownRow = 1 << 29;        // ... whose ordinal the profile lacks
constexpr int32_t kChunkCanonOutOfRange = 1 << 28;   // a substituted canonical cell outside [0, P-1]

// Dynamic keys beside a fixed key that the MFMA policy path's checker holds.
constexpr int kPolicyMaxBoundary = 256;

// Checker of the MFMA policy prefill (CanonicalPositionPolicy over dense bf16
// keys 0..nk-1): one wave per (query row, head) of a fixed row.
struct policy_check_args {
  const uint16_t* q;
  int64_t q_s_tok, q_s_head;
  const uint16_t* k;
  int64_t k_s_tok, k_s_head;
  const int64_t* qpos;
  int32_t nq, hq, group;
  int64_t nk;
  const float* canon;
  int64_t c_s0, c_s1, c_s2;
  const int64_t* q_ord;
  const int32_t* code;       // per key: fixed ordinal (>= 0), -2 - s (boundary slot s), -1
  const int32_t* blk;        // per block of 256 keys: offset o (code = key - o), -1 (all -1), -2 (read code)
  const int32_t* bnd_count;  // dynamic keys beside a fixed key: count
  const int32_t* bnd_keys;   // and the keys, ascending
  int32_t npos, strict, chunk_rows;
  int32_t* chunk_flags;
};

int launch_policy_check(const policy_check_args& a, hipStream_t stream);

// The paged MFMA prefill (ccpe_prefill.hip) writing per (batch item, row,
// head) softmax states: fp32 state_o [B, nq, Hq, 128] (the output
// unnormalised against the running max of the raw scores q.k, with the
// positional bias shifted so that a saturated key adds 0) and state_ml
// [B, nq, Hq, 3] (max, sum, carry: the gate mass counted from the row's key,
// >= P-1 once saturated).  saturated != 0: every position taken as P-1.
// zero_word (may be null): set to 0 by the launch.
int launch_prefill_states(const void* q, int64_t q_s_batch, int64_t q_s_tok, int64_t q_s_head,
                          const int64_t* qpos, int64_t qpos_s_batch, int32_t batch, int32_t nq, int32_t hq,
                          int32_t hkv, const int32_t* nk, const cs_kv_source* kv, const float* e,
                          int32_t max_positions, int32_t saturated, int max_waves, float* state_o,
                          float* state_ml, int32_t* zero_word, int32_t* flags, hipStream_t s);

}  // namespace cs
