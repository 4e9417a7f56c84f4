// Checks of the CanonicalPositionPolicy transform for the MFMA policy prefill
// (attention.py:32-57 over position.py:485-516), over dense bf16 keys at
// coordinates 0..nk-1 with no attention mask.
//
// For a fixed query row the transform's result is the contextual row with the
// fixed-key cells replaced by the profile's canonical row.  Its bounds check
// (position.py:500-515: every cell a finite value in [0, P-1]) can only fail
// at a canonical cell, and of the strict path checks (position.py:98-114)
// contextual cells and pairs of adjacent contextual cells pass by
// construction: a contextual position is a clamped suffix sum of the gates of
// the keys from it to the query, each gate in [0, 1].  What remains is the
// canonical cells, the pairs of adjacent fixed keys, and the pairs of a fixed
// key with a dynamic neighbour; the latter need the contextual position of
// that dynamic key, which is recomputed here the way the generic kernel forms
// it (fp32 logits and sigmoid gates, fp64 suffix sum rounded once, clamped),
// stopping once the sum reaches P-1.  One wave per (query row, head); rows
// that are not fixed return at once.

#include "common.h"
#include "ccpe_path.h"

namespace cs {
namespace {

constexpr int kWaves = 4;
constexpr int kD = 128;

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ void __launch_bounds__(64 * kWaves) policy_check_kernel(policy_check_args a) {
  __shared__ float qs[kWaves][kD];
  __shared__ float bctx[kWaves][kPolicyMaxBoundary];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (item >= static_cast<int64_t>(a.nq) * a.hq) return;  // no block barrier follows
  const int row = static_cast<int>(item / a.hq), h = static_cast<int>(item % a.hq);
  const int64_t qo = a.q_ord[row];
  if (qo == -1) return;
  int32_t* chunk = a.chunk_flags + row / a.chunk_rows;
  if (qo < 0) {  // a fixed row the profile has no trace for: the lookup raises
    if (lane == 0) atomicOr(chunk, kChunkHasFixedRow | kChunkUnknownRow);
    return;
  }
  const int64_t qp = a.qpos[row];
  const int64_t kend = qp + 1 < a.nk ? qp + 1 : a.nk;  // causal keys [0, kend)
  const float top = static_cast<float>(a.npos - 1);
  const float* crow = a.canon + h * a.c_s0 + qo * a.c_s1;
  const int kvh = h / a.group;

  if (a.strict) {
    // contextual positions of the dynamic keys beside a fixed key
    const uint16_t* qrow = a.q + row * a.q_s_tok + h * a.q_s_head;
    for (int d = lane; d < kD; d += 64) qs[wave][d] = bf16_to_float(qrow[d]);
    wave_sync();
    const float sqrt_d = static_cast<float>(sqrt(static_cast<double>(kD)));
    const int nb = *a.bnd_count;
    for (int bi = 0; bi < nb; ++bi) {
      const int64_t key = a.bnd_keys[bi];
      float val = 0.f;
      if (key < kend) {
        double sum = 0.0;  // wave-uniform after each reduction
        for (int64_t base = key; base < kend && sum < static_cast<double>(top); base += 64) {
          const int64_t i = base + lane;
          double g = 0.0;
          if (i < kend) {
            const uint16_t* kr = a.k + i * a.k_s_tok + kvh * a.k_s_head;
            float dot = 0.f;
            for (int d = 0; d < kD; ++d) dot += qs[wave][d] * bf16_to_float(kr[d]);
            const float logit = dot / sqrt_d;
            g = static_cast<double>(1.f / (1.f + expf(-logit)));
          }
          sum += wave_sum(g);
        }
        float pc = static_cast<float>(sum);
        if (pc < 0.f) pc = 0.f;
        if (pc > top) pc = top;
        val = pc;
      }
      if (lane == 0) bctx[wave][bi] = val;
    }
    wave_sync();
  }

  // Right to left over blocks of 256 keys, lane l holding keys 4l .. 4l+3 of
  // a block: the right-hand neighbour of its last key is the next lane's
  // first, and that of lane 63's last key the first key of the block to the
  // right.  Blocks past the query need only the bounds check.  Blocks go in
  // groups of kGroup, all of a group's canonical cells loaded together, the
  // codes of the next group in flight while a group is checked.  A block
  // whose keys are all fixed with consecutive ordinals (descriptor o >= 0:
  // code = key - o) computes its codes and, on a contiguous profile row,
  // reads each lane's 4 cells as one 16-byte load; a block of plain dynamic
  // keys (-1) reads nothing; only the other blocks (-2) read their codes.
  constexpr int kGroup = 4;
  int bits = 0;
  bool out_of_range = false;
  float prev_p = 0.f;
  bool prev_known = false, prev_fixed = false;
  const float atol = static_cast<float>(1e-6);
  auto load_codes = [&](int64_t t, int32_t* code) {
    const int64_t j0 = t * 256 + 4 * lane;
    if (t < 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) code[i] = -1;
    } else if (j0 + 3 < a.nk) {
      const int4 c4 = *reinterpret_cast<const int4*>(a.code + j0);
      code[0] = c4.x;
      code[1] = c4.y;
      code[2] = c4.z;
      code[3] = c4.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) code[i] = j0 + i < a.nk ? a.code[j0 + i] : -1;
    }
  };
  // (all_fixed: every key of the block is fixed, descriptor >= 0)
  auto check_block = [&](int64_t t, const int32_t* code, const float* pcell, bool all_fixed) {
    const int64_t j0 = t * 256 + 4 * lane;
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = pcell[i];
      if (code[i] >= 0 && !(pv[i] >= 0.f && pv[i] <= top)) out_of_range = true;  // NaN included
    }
    if (!a.strict) return;
    if (t * 256 >= kend) {  // no causal key in the block
      prev_known = false;
      return;
    }
    if (all_fixed && (t + 1) * 256 <= kend) {
      // Every key of the block fixed and causal: every cell is checked and
      // paired with its right-hand neighbour (lane 63's last cell with the
      // block to the right, when that key is checked).  A cell with p >= 0,
      // p <= q - k + 1 and, paired, 0 <= p - p_right <= 1 passes every test of
      // path_violations_unit, whose tolerances are all >= 0 (so its bounds
      // are these or looser, in the same float arithmetic); only a block in
      // which some cell misses this screen takes the exact checks below.
      float right = __shfl_down(pv[0], 1, 64);
      bool right_pair = true;
      if (lane == 63) {
        right = prev_p;
        right_pair = prev_known;
      }
      bool ok = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = i < 3 ? pv[i + 1] : right;
        const bool paired = i < 3 ? true : right_pair;
        const float d = pv[i] - pr;
        // q - k + 1 exactly as path_violations_unit forms it
        const float available = static_cast<float>(static_cast<int32_t>(qp - (j0 + i))) + 1.f;
        ok = ok && pv[i] >= 0.f && pv[i] <= available && (!paired || (d >= 0.f && d <= 1.f));
      }
      if (__all(ok)) {
        prev_p = __shfl(pv[0], 0, 64);
        prev_known = true;
        prev_fixed = true;
        return;
      }
    }
    bool known[4], fixed[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fixed[i] = code[i] >= 0;
      known[i] = j0 + i < kend && (fixed[i] || code[i] <= -2);
      if (known[i] && code[i] <= -2) pv[i] = bctx[wave][-2 - code[i]];  // a dynamic key beside a fixed key
    }
    float right = __shfl_down(pv[0], 1, 64);
    bool right_known = __shfl_down(known[0] ? 1 : 0, 1, 64) != 0;
    bool right_fixed = __shfl_down(fixed[0] ? 1 : 0, 1, 64) != 0;
    if (lane == 63) {
      right = prev_p;
      right_known = prev_known;
      right_fixed = prev_fixed;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pr = i < 3 ? pv[i + 1] : right;
      const bool kr = i < 3 ? known[i + 1] : right_known;
      const bool fr = i < 3 ? fixed[i + 1] : right_fixed;
      const bool pair = known[i] && kr && (fixed[i] || fr);
      // causal keys only reach here (diff >= 0, below 2^31 for keys 0..nk-1)
      bits |= path_violations_unit(pv[i], known[i], pr, pair, static_cast<int32_t>(qp - (j0 + i)), atol);
    }
    prev_p = __shfl(pv[0], 0, 64);
    prev_known = __shfl(known[0] ? 1 : 0, 0, 64) != 0;
    prev_fixed = __shfl(fixed[0] ? 1 : 0, 0, 64) != 0;
  };
  auto fetch = [&](int64_t t, int32_t& d, int32_t* code) {
    if (t < 0) {
      d = -1;
    } else {
      d = a.blk[t];  // wave-uniform
    }
    const int64_t j0 = t * 256 + 4 * lane;
    if (d >= 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) code[i] = static_cast<int32_t>(j0 + i - d);
    } else if (d == -1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) code[i] = -1;
    } else {
      load_codes(t, code);
    }
  };
  const bool row16 = a.c_s2 == 1 && (reinterpret_cast<uintptr_t>(crow) & 15) == 0;
  const int64_t last = (a.nk + 255) / 256 - 1;
  int32_t desc[kGroup], codes[kGroup][4];
#pragma unroll
  for (int g = 0; g < kGroup; ++g) fetch(last - g, desc[g], codes[g]);
  for (int64_t t0 = last; t0 >= 0; t0 -= kGroup) {
    float cells[kGroup][4];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
      if (desc[g] >= 0 && row16 && (desc[g] & 3) == 0) {
        const float4 v4 = *reinterpret_cast<const float4*>(crow + codes[g][0]);
        cells[g][0] = v4.x;
        cells[g][1] = v4.y;
        cells[g][2] = v4.z;
        cells[g][3] = v4.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          cells[g][i] = codes[g][i] >= 0 ? crow[static_cast<int64_t>(codes[g][i]) * a.c_s2] : 0.f;
      }
    }
    int32_t ndesc[kGroup], next[kGroup][4];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) fetch(t0 - kGroup - g, ndesc[g], next[g]);
#pragma unroll
    for (int g = 0; g < kGroup; ++g)
      if (t0 - g >= 0) check_block(t0 - g, codes[g], cells[g], desc[g] >= 0);
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
      desc[g] = ndesc[g];
#pragma unroll
      for (int i = 0; i < 4; ++i) codes[g][i] = next[g][i];
    }
  }
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off, 64);
  const bool any_oob = __any(out_of_range);
  if (lane == 0) atomicOr(chunk, bits | (any_oob ? kChunkCanonOutOfRange : 0) | kChunkHasFixedRow);
}

}  // namespace

int launch_policy_check(const policy_check_args& a, hipStream_t stream) {
  const int64_t items = static_cast<int64_t>(a.nq) * a.hq;
  if (items == 0) return CS_OK;
  const int64_t blocks = (items + kWaves - 1) / kWaves;
  CS_REQUIRE(blocks < (int64_t(1) << 31), "too many rows for the policy checker");
  hipLaunchKernelGGL(policy_check_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(64 * kWaves), 0, stream,
                     a);
  CS_LAUNCH_CHECK("ccpe_policy_check");
  return CS_OK;
}

}  // namespace cs
