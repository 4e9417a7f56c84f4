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
// 16 zero bytes: the load of a block whose cells are not read as one 16-byte load
__device__ __align__(16) float g_zero_cells[4];
constexpr int kD = 128;

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Running state of a wave's walk over its row's blocks.
struct check_state {
  int bits = 0;               // CS_FLAG_PATH_* of this lane's cells
  bool out_of_range = false;  // a canonical cell of this lane outside [0, P-1]
  // the first cell of the block to the right (lane 0's first key), and
  // whether it is checked / fixed
  float prev_p = 0.f;
  bool prev_known = false, prev_fixed = false;
};

// The exact checks of block t (keys 256 t .. 256 t + 255, lane l holding
// 4l .. 4l+3) with descriptor d (>= 0: code = key - d; -2: read the codes);
// fc holds the block's cells when wide.  Bounds of every fixed cell
// (position.py:500-515) and, in strict mode, path_violations_unit on every
// causal cell that is fixed or a dynamic key beside a fixed key, paired with
// its right-hand neighbour when either of the two is fixed.
// Returns the state after the block (passed and returned by value, so that
// it stays in registers).
__device__ __noinline__ check_state check_block_exact(int64_t t, int32_t d, float4 fc, bool wide, int lane,
                                                      int64_t qp, int64_t kend, float top, const float* crow,
                                                      int64_t c_s2, const int32_t* codes, int64_t nk, bool strict,
                                                      const float* bctx, check_state st) {
  const float atol = static_cast<float>(1e-6);
  const int64_t j0 = t * 256 + 4 * lane;
  int32_t code[4];
  if (d >= 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) code[i] = static_cast<int32_t>(j0 + i - d);
  } else if (j0 + 3 < nk) {
    const int4 c4 = *reinterpret_cast<const int4*>(codes + j0);
    code[0] = c4.x;
    code[1] = c4.y;
    code[2] = c4.z;
    code[3] = c4.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) code[i] = j0 + i < nk ? codes[j0 + i] : -1;
  }
  float pv[4] = {fc.x, fc.y, fc.z, fc.w};
  if (!wide) {
#pragma unroll
    for (int i = 0; i < 4; ++i) pv[i] = code[i] >= 0 ? crow[static_cast<int64_t>(code[i]) * c_s2] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (code[i] >= 0 && !(pv[i] >= 0.f && pv[i] <= top)) st.out_of_range = true;  // NaN included
  if (!strict) return st;
  if (t * 256 >= kend) {  // no causal key in the block
    st.prev_known = false;
    return st;
  }
  bool known[4], fixed[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    fixed[i] = code[i] >= 0;
    known[i] = j0 + i < kend && (fixed[i] || code[i] <= -2);
    if (known[i] && code[i] <= -2) pv[i] = bctx[-2 - code[i]];  // a dynamic key beside a fixed key
  }
  float right = __shfl_down(pv[0], 1, 64);
  bool right_known = __shfl_down(known[0] ? 1 : 0, 1, 64) != 0;
  bool right_fixed = __shfl_down(fixed[0] ? 1 : 0, 1, 64) != 0;
  if (lane == 63) {
    right = st.prev_p;
    right_known = st.prev_known;
    right_fixed = st.prev_fixed;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float pr = i < 3 ? pv[i + 1] : right;
    const bool kr = i < 3 ? known[i + 1] : right_known;
    const bool fr = i < 3 ? fixed[i + 1] : right_fixed;
    const bool pair = known[i] && kr && (fixed[i] || fr);
    // causal keys only reach here (diff >= 0, below 2^31 for keys 0..nk-1)
    st.bits |= path_violations_unit(pv[i], known[i], pr, pair, static_cast<int32_t>(qp - (j0 + i)), atol);
  }
  st.prev_p = __shfl(pv[0], 0, 64);
  st.prev_known = __shfl(known[0] ? 1 : 0, 0, 64) != 0;
  st.prev_fixed = __shfl(fixed[0] ? 1 : 0, 0, 64) != 0;
  return st;
}

__global__ void __launch_bounds__(64 * kWaves) policy_check_kernel(policy_check_args a) {
  __shared__ float qs[kWaves][kD];
  __shared__ float bctx[kWaves][kPolicyMaxBoundary];
  const int lane = threadIdx.x & 63;
  // wave-uniform (a scalar), so that the row, its positions and addresses are too
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
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
  // right.  Blocks past the query need only the bounds check.  A block whose
  // keys are all fixed with consecutive ordinals (descriptor o >= 0: code =
  // key - o) computes its codes and, on a contiguous profile row, reads each
  // lane's 4 cells as one 16-byte load whose address depends only on the
  // block, the descriptor (a scalar) and the lane; a block of plain dynamic
  // keys (-1) reads nothing; only the other blocks (-2) read their codes.
  // The 16-byte loads of a group of kGroup blocks and of the group after it
  // are in flight together (a block without one loads a zero record), so the
  // wave waits for memory once per group, not once per block.
  constexpr int kGroup = 4;
  check_state st;
  const bool row16 = a.c_s2 == 1 && (reinterpret_cast<uintptr_t>(crow) & 15) == 0;
  // wave-uniform: the cells of block t come from one 16-byte load per lane
  auto wide = [&](int64_t t, int32_t d) { return t >= 0 && d >= 0 && row16 && (d & 3) == 0; };
  // descriptors through the constant address space: scalar loads (the array
  // is written by an earlier launch and only read here)
  const __attribute__((address_space(4))) int32_t* const blk =
      (const __attribute__((address_space(4))) int32_t*)a.blk;
  auto desc_at = [&](int64_t t) -> int32_t { return t >= 0 ? blk[t] : -1; };
  const float* const zero_cells = g_zero_cells;
  auto issue_cells = [&](int64_t t, int32_t d) -> float4 {
    const float* src = wide(t, d) ? crow + (t * 256 + 4 * lane - d) : zero_cells;
    return *reinterpret_cast<const float4*>(src);
  };
  // Screens.  A float's bit pattern read as an unsigned integer is at most
  // that of a finite x >= 0 exactly when the float lies in [+0, x] (negative
  // values, -0 and NaN have larger patterns), so one unsigned maximum over
  // the cells bounds them all.  A screened cell passes every exact test:
  //   bounds (position.py:500-515): 0 <= p <= P-1;
  //   path_violations_unit, whose tolerances are all >= 0 (so its bounds are
  //   these or looser, in the same float arithmetic): p >= 0,
  //   p <= q - k + 1, and paired with its right-hand neighbour
  //   0 <= p - p_right <= 1.
  // q - k + 1 is formed as float(q - k) + 1, exact while q + 1 <= 2^24, and so
  // is (q - j0 + 1) - i; with p not NaN, (q - k + 1) - p >= 0 exactly when
  // p <= q - k + 1.  A block with a cell outside a screen takes the exact
  // checks.
  const uint32_t top_bits = __float_as_uint(top);
  const uint32_t one_bits = __float_as_uint(1.f);
  const bool exact_avail = qp + 1 <= (int64_t(1) << 24);
  // block t with descriptor d; fc: its cells when wide(t, d)
  auto check_block = [&](int64_t t, int32_t d, const float4& fc) {
    const int64_t j0 = t * 256 + 4 * lane;
    if (d == -1) {  // no fixed key: nothing to check, no cell to pair with
      st.prev_known = false;
      return;
    }
    float pv[4] = {fc.x, fc.y, fc.z, fc.w};
    if (wide(t, d)) {
      // every key of the block fixed (the screens read only these cells, so
      // that the wait for them counts the loads in flight behind them)
      const uint32_t pmax = max(max(__float_as_uint(pv[0]), __float_as_uint(pv[1])),
                                max(__float_as_uint(pv[2]), __float_as_uint(pv[3])));
      const bool in_range = pmax <= top_bits;
      if (!a.strict || t * 256 >= kend) {
        // the bounds check only (no causal key in the block, or mixed mode)
        if (__all(in_range)) {
          st.prev_known = false;
          return;
        }
      } else if ((t + 1) * 256 <= kend && exact_avail) {
        // every cell causal, checked and paired with its right-hand neighbour
        // (lane 63's last cell with the block to the right, when that key is
        // checked)
        float right = __shfl_down(pv[0], 1, 64);
        if (lane == 63) right = st.prev_known ? st.prev_p : pv[3];
        const uint32_t dmax = max(max(__float_as_uint(pv[0] - pv[1]), __float_as_uint(pv[1] - pv[2])),
                                  max(__float_as_uint(pv[2] - pv[3]), __float_as_uint(pv[3] - right)));
        bool ok = in_range && dmax <= one_bits;
        // q - k + 1 >= P - 1 >= p for every key of the block unless the block
        // reaches within P - 1 keys of the query (wave-uniform)
        if (qp - (t * 256 + 255) + 1 < static_cast<int64_t>(top)) {
          const float avail = static_cast<float>(static_cast<int32_t>(qp - j0)) + 1.f;
          const float slack = fminf(fminf(avail - pv[0], (avail - 1.f) - pv[1]),
                                    fminf((avail - 2.f) - pv[2], (avail - 3.f) - pv[3]));
          ok = ok && slack >= 0.f;
        }
        if (__all(ok)) {
          st.prev_p = __shfl(pv[0], 0, 64);
          st.prev_known = true;
          st.prev_fixed = true;
          return;
        }
      }
    }
    // the exact checks (out of line: inlined, their loads and waits would make
    // the compiler wait for every cell load in flight before each screen)
    st = check_block_exact(t, d, fc, wide(t, d), lane, qp, kend, top, crow, a.c_s2, a.code, a.nk, a.strict != 0,
                           &bctx[wave][0], st);
  };
  const int64_t last = (a.nk + 255) / 256 - 1;
  // two groups' descriptors and cells, used in turn (no copies between them,
  // which would wait for every load in flight)
  int32_t desc_a[kGroup], desc_b[kGroup];
  float4 cells_a[kGroup], cells_b[kGroup];
  auto issue_group = [&](int64_t t0, int32_t (&d)[kGroup], float4 (&c)[kGroup]) {
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
      d[g] = desc_at(t0 - g);
      c[g] = issue_cells(t0 - g, d[g]);
    }
  };
  auto check_group = [&](int64_t t0, const int32_t (&d)[kGroup], const float4 (&c)[kGroup]) {
#pragma unroll
    for (int g = 0; g < kGroup; ++g)
      if (t0 - g >= 0) check_block(t0 - g, d[g], c[g]);
  };
  issue_group(last, desc_a, cells_a);
  for (int64_t t0 = last; t0 >= 0; t0 -= 2 * kGroup) {
    issue_group(t0 - kGroup, desc_b, cells_b);
    check_group(t0, desc_a, cells_a);
    if (t0 - kGroup < 0) break;
    issue_group(t0 - 2 * kGroup, desc_a, cells_a);
    check_group(t0 - kGroup, desc_b, cells_b);
  }
  int bits = st.bits;
  for (int off = 32; off > 0; off >>= 1) bits |= __shfl_xor(bits, off, 64);
  const bool any_oob = __any(st.out_of_range);
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
