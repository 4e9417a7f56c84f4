/*
 * cacheslide_hip.h -- C ABI of libcacheslide_hip.so, the gfx950 (MI355X) kernels
 * behind the cacheslide_amd Python package.
 *
 * Every entry point takes plain device pointers, element strides and sizes, a
 * hipStream_t passed as void*, and returns an int status (CS_OK == 0).  On a
 * nonzero status cs_last_error() returns a message for the calling thread.
 * No entry point allocates device memory; scratch space is passed in by the
 * caller.  Data-dependent conditions that the reference reports as Python
 * exceptions (nonfinite values, invalid contextual paths, ...) are written as
 * bits into a caller-supplied int32 device flag word, so the host can raise the
 * reference's exception after one readback.
 *
 * Reference interfaces replaced (paths relative to the CacheSlide repository):
 *   src/cacheslide_vllm/position.py   cope_attention, CoPE, validate_contextual_path
 *   src/cacheslide_vllm/attention.py  CanonicalPositionPolicy, SelectedAssociationPolicy
 *   src/cacheslide_vllm/wca.py        squared_deviation, adaptation_weight,
 *                                     mean_head_cosine, WCAState
 *   src/cacheslide_vllm/paged.py      NativePagedKV._write_slots / gather
 *   src/cacheslide_vllm/slide.py      LayerSlotMap._fresh_slot (free-slot order)
 *   src/cacheslide_vllm/runtime.py    CacheSlideRuntime._prefill row bookkeeping
 */
#ifndef CACHESLIDE_HIP_H
#define CACHESLIDE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of a view. */
enum cs_dtype { CS_F32 = 0, CS_F16 = 1, CS_BF16 = 2, CS_F64 = 3, CS_I32 = 4, CS_I64 = 5, CS_U8 = 6 };

/* Return codes. */
enum cs_status {
  CS_OK = 0,
  CS_EINVAL = 1,       /* argument error: shapes, dtypes, null pointers */
  CS_ELAUNCH = 2,      /* a HIP launch or runtime call failed */
  CS_EUNSUPPORTED = 3, /* valid arguments outside a kernel's supported range */
  CS_ECAPACITY = 4     /* not enough free slots (CacheCapacityError) */
};

/* A strided device tensor of up to 6 dimensions; strides are in elements.
 * A view whose data pointer is NULL is "absent". */
typedef struct cs_view {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[6];
  int64_t stride[6];
} cs_view;

const char* cs_version(void);
const char* cs_last_error(void);

/* ------------------------------------------------------------------------ *
 * Flag bits written by the attention / validation kernels (int32 word).
 * ------------------------------------------------------------------------ */
enum cs_flag {
  CS_FLAG_Q_NONFINITE = 1 << 0,       /* position.py:117-124 (_rows "query") */
  CS_FLAG_K_NONFINITE = 1 << 1,       /* _rows "key" */
  CS_FLAG_V_NONFINITE = 1 << 2,       /* _rows "value" */
  CS_FLAG_QPOS_NEGATIVE = 1 << 3,     /* position.py:127-137 */
  CS_FLAG_QPOS_DUPLICATE = 1 << 4,
  CS_FLAG_KPOS_NEGATIVE = 1 << 5,
  CS_FLAG_KPOS_DUPLICATE = 1 << 6,
  CS_FLAG_KPOS_UNSORTED = 1 << 7,     /* position.py:178-179 */
  CS_FLAG_LOGIT_NONFINITE = 1 << 8,   /* position.py:162-163 */
  CS_FLAG_POS_INVALID = 1 << 9,       /* position.py:323-334 (bias positions) */
  CS_FLAG_SCORE_NONFINITE = 1 << 10,  /* position.py:519-520 */
  CS_FLAG_E_NONFINITE = 1 << 11,
  CS_FLAG_POS_NONFINITE = 1 << 12,    /* validate: positions not finite */
  CS_FLAG_BLOCK_INVALID = 1 << 13,    /* a block-table entry or slot outside the cache */
  CS_FLAG_NO_KEY = 1 << 14,           /* decode: a context length < 1 (position.py:149-150
                                         "attention requires at least one key") */
  CS_FLAG_CONTEXT_RANGE = 1 << 15,    /* decode: a context length above the max_nk the
                                         workspace was sized for */
  /* strict contextual-path checks, position.py:99-114, in the reference's order */
  CS_FLAG_PATH_NEGATIVE = 1 << 16,
  CS_FLAG_PATH_AVAILABLE = 1 << 17,
  CS_FLAG_PATH_INCREASING = 1 << 18,
  CS_FLAG_PATH_GAP = 1 << 19,
  /* selective-prefill row bookkeeping, runtime.py:408-456 */
  CS_FLAG_ROW_LOST = 1 << 20,         /* an active token in neither the previous rows nor the snapshot */
  CS_FLAG_ROWS_UNSORTED = 1 << 21,    /* a token list is not ascending and distinct */
  CS_FLAG_ROW_INDEX = 1 << 22,        /* a gather index outside the source rows */
  /* cs_ccpe_prefill_policy_bf16: the call needs cs_ccpe_attention instead
     (more dynamic keys beside fixed keys than the path checker holds); its
     results are to be discarded */
  CS_FLAG_POLICY_GENERIC = 1 << 23
};

/* ------------------------------------------------------------------------ *
 * Input checks (position.py:117-137, 178-179).  Writes CS_FLAG_* bits.
 * ------------------------------------------------------------------------ */

/* Nonfinite scan of a floating view; ORs `bit` into *flags. */
int cs_check_finite(const cs_view* x, int32_t bit, int32_t* flags, void* stream);

/* The coordinate checks of cope_attention (position.py:127-137, 178-179):
 * int64 positions [n]: negative, duplicate and (keys only) not strictly
 * increasing.  The quadratic duplicate scan runs only when the order check
 * found a descent.  Bits are the query or key variants selected by `is_key`;
 * bit 24 is used internally for query order. */
int cs_check_positions(const int64_t* pos, int64_t n, int32_t is_key,
                       int32_t* flags, void* stream);

/* Positions tensor [H, q, k] used as CoPE coordinates: ORs CS_FLAG_POS_INVALID
 * when an entry is nonfinite, < 0 or > max_positions-1 (position.py:323-334,
 * 504-516), and CS_FLAG_POS_NONFINITE when an entry is nonfinite. */
int cs_check_bias_positions(const cs_view* positions, int64_t max_positions,
                            int32_t* flags, void* stream);

/* ------------------------------------------------------------------------ *
 * CCPE attention, generic path (any float dtype, any head dims, masks,
 * fixed positions, lowered policies, position output).
 * Replaces position.py:404-560 cope_attention (and with out == NULL the
 * contextual-position computation of position.py:295-307).
 *
 *   q [nq, Hq, D], k [nk, Hkv, D], v [nk, Hkv, Dv]   same float dtype
 *   e [D, P]                                         CoPE table (any float)
 *   qpos [nq], kpos [nk]                             int64 device
 *   attn_mask, vis_mask [Hm, nq, nk] uint8 (Hm = 1 or Hq; stride 0 broadcast)
 *   sel_rows [nq], fixed_keys [nk] uint8 : SelectedAssociationPolicy lowering
 *       visible = !sel_rows[r] || !fixed_keys[j] || qpos[r] == kpos[j]
 *   fixed_pos [Hq, nq, nk]                           replaces contextual positions
 *   canonical [Hq, F, F] with q_ord [nq], k_ord [nk] (int64, -1 = not fixed):
 *       CanonicalPositionPolicy lowering; strict != 0 runs the path checks and
 *       ORs CS_FLAG_PATH_* into chunk_flags[r / chunk_rows], plus bit 30 for a
 *       chunk holding a fixed query row (the policy validates only those) and
 *       bit 29 for a chunk holding a fixed row with q_ord == -2 (an ordinal
 *       the profile has no trace for: CCPEProfile.lookup raises, position.py:
 *       733-738) and bit 28 for a chunk with a substituted canonical value
 *       outside [0, P-1] (the transform bounds check, position.py:500-515;
 *       not reported as CS_FLAG_POS_INVALID).
 *   out [nq, Hq, Dv] (dtype of v) or NULL;  pos_out [Hq, nq, nk] or NULL.
 * ------------------------------------------------------------------------ */
typedef struct cs_ccpe_args {
  cs_view q, k, v, e;
  const int64_t* qpos;
  const int64_t* kpos;
  cs_view attn_mask, vis_mask;
  const uint8_t* sel_rows;
  const uint8_t* fixed_keys;
  cs_view fixed_pos;
  cs_view canonical;
  const int64_t* q_ord;
  const int64_t* k_ord;
  int32_t strict;
  int32_t chunk_rows;
  int32_t* chunk_flags;
  cs_view out;
  cs_view pos_out;
  int32_t* flags;
} cs_ccpe_args;

int cs_ccpe_attention(const cs_ccpe_args* args, void* stream);

/* cope_attention with the two runtime policies on bf16 MFMA: the reuse call of
 * runtime.py:576-609 (CanonicalPositionPolicy, attention.py:18-57, and/or
 * SelectedAssociationPolicy, attention.py:60-72, in updated_and_self mode)
 * over dense K/V: the selective calls, the calibration-layer call (a profile
 * and no selection yet, runtime.py:448-454) and selected_attention "all".
 * Same lowered data as cs_ccpe_attention; supported when q/k/v/out are bf16
 * with head dim 128, e is fp32 [128, P <= 128], kpos is NULL (key coordinates
 * 0..nk-1), the GQA group divides 32, there are no masks, fixed positions or
 * position output, and either sel_rows/fixed_keys are given (canonical
 * optional) or both are NULL and canonical is given (the fixed keys are then
 * those with a profile ordinal); canonical is fp32; otherwise CS_EUNSUPPORTED.
 *
 * A selected fixed row sees no fixed key but its own, so the kernel reads one
 * canonical cell per (head, row) and skips tiles of fixed keys once a row's
 * positions have saturated.  A fixed row that is not selected sees every
 * fixed key at canonical[h][q_ord][k_ord]: the kernel reads those cells tile
 * by tile, 16 bytes per run of 4 keys where the profile allows.  The
 * transform's bounds check (every fixed key) and, with strict != 0, the path
 * checks of the substituted row (over fixed keys and the dynamic keys beside
 * them; contextual cells always pass) run in a checker launch over the
 * canonical rows and set the same chunk bits as cs_ccpe_attention.  When the
 * plan has more boundary keys than the checker holds, the call sets
 * CS_FLAG_POLICY_GENERIC in *flags and the caller runs cs_ccpe_attention
 * instead.  workspace: at least
 * cs_ccpe_prefill_policy_workspace_bytes(nq, Hq, nk) bytes, 256-byte aligned,
 * any contents.  The checker runs on a helper stream of the device, forked
 * from and joined back into `stream`, so that it overlaps the attention. */
int64_t cs_ccpe_prefill_policy_workspace_bytes(int32_t nq, int32_t hq, int64_t nk);
int cs_ccpe_prefill_policy_bf16(const cs_ccpe_args* args, void* workspace, int64_t workspace_bytes,
                                void* stream);

/* No counterpart in the reference (an implementation helper).  Creates, for
 * the current device, the helper stream of cs_ccpe_prefill_policy_bf16, which
 * is otherwise created at that entry point's first call.  The HIP runtime
 * gives a new stream a hardware queue of its own only while the device has
 * fewer queues than GPU_MAX_HW_QUEUES (4 by default) and then shares them;
 * a helper stream that shares the caller's queue runs the checker and the
 * attention one after the other.  Calling this once per device before the
 * process creates other streams (the Python package does so at its first use
 * of a device) keeps them apart.  Idempotent. */
int cs_prepare_device(void);

/* CoPE.contextual_positions (position.py:295-307) on explicit logits [H,q,k]
 * and a gate mask allowed [Hm,q,k] uint8: sigmoid gates, fp64 reverse cumulative
 * sum rounded once to out's dtype, clamp(0, P-1).  ORs CS_FLAG_LOGIT_NONFINITE
 * when an allowed logit is nonfinite. */
int cs_contextual_positions(const cs_view* logits, const cs_view* allowed,
                            int64_t max_positions, cs_view* out, int32_t* flags, void* stream);

/* Logits matrix (position.py:157-164): out[h,r,j] = q[r,h] . k[j, h/G] / sqrt(D)
 * for every (query, key) pair, causal or not (CoPE.position_trace). */
int cs_ccpe_logits(const cs_view* q, const cs_view* k, cs_view* out, int32_t* flags,
                   void* stream);

/* CoPE.positional_bias (position.py:309-344): bias[h,r,j] from positions
 * [Hq, nq, nk] and query rows q [nq, Hq, D]; out dtype = accumulation dtype. */
int cs_cope_positional_bias(const cs_view* q, const cs_view* e, const cs_view* positions,
                            cs_view* out, int32_t* flags, void* stream);

/* validate_contextual_path (position.py:28-114) on a positions tensor [H,q,k];
 * attn_mask optional [Hm,q,k] uint8.  ORs CS_FLAG_PATH_* into *flags. */
int cs_validate_contextual_path(const cs_view* positions, const int64_t* qpos,
                                const int64_t* kpos, const cs_view* attn_mask,
                                double atol, int32_t* flags, void* stream);

/* SelectedAssociationPolicy.__call__ (attention.py:65-72): bool mask [nq, nk]
 * in out[0 .. nq*nk); out must have nq*nk + nq + nk bytes (the tail holds the
 * row/column membership flags).  fixed and selected are sorted ascending. */
int cs_selected_visibility(const int64_t* queries, int64_t nq, const int64_t* keys,
                           int64_t nk, const int64_t* fixed, int64_t nfixed,
                           const int64_t* selected, int64_t nselected, uint8_t* out,
                           void* stream);

/* out[i] = values[i] is in set[0..m) (the torch.isin of
 * SelectedAssociationPolicy, attention.py:60-72); set sorted ascending. */
int cs_isin(const int64_t* values, int64_t n, const int64_t* set, int64_t m, uint8_t* out,
            void* stream);

/* CanonicalPositionPolicy substitution (attention.py:46-50):
 * result[h, rows[i], cols[c]] = canonical[h, q_ord_rows[i], k_ord_cols[c]]. */
int cs_canonical_substitute(cs_view* result, const cs_view* canonical,
                            const int64_t* rows, const int64_t* row_ordinals, int64_t nrows,
                            const int64_t* cols, const int64_t* col_ordinals, int64_t ncols,
                            void* stream);

/* ------------------------------------------------------------------------ *
 * CCPE fast paths: bf16, D = Dv = 128, key positions 0..nk-1, no masks.
 * K/V of key j of request b are read from one of three sources:
 *   dense  (block_table == NULL, slots == NULL): k, v [B][nk, Hkv, 128];
 *   blocks (block_table != NULL): the paged cache [blocks, Hkv, block_size, 256]
 *          (K = [..., :128], V = [..., 128:]) at block block_table[b, j / bs],
 *          offset j % bs -- the canonical slot of paged.py:146-151;
 *   slots  (slots != NULL): the per-token slot map of a SLIDE arena,
 *          s = slots[b * slots_stride + j] (the slot NativePagedKV.gather reads
 *          for token j, paged.py:433-472 over slide.py:264-270).  A slot below
 *          num_blocks * block_size is native (block s / bs, offset s % bs); slot
 *          num_blocks * block_size + i is sidecar row i of side_k / side_v
 *          [side_rows, Hkv, 128] (paged.py:205-240), which holds selected rows
 *          displaced by decode hole reuse (paged.py:474-524, slide.py:401-459).
 *          A slot outside both sets CS_FLAG_BLOCK_INVALID and reads zeros.
 * ------------------------------------------------------------------------ */
typedef struct cs_kv_source {
  /* paged forms */
  const void* cache;          /* bf16 base of [blocks, Hkv, block_size, 2*128] */
  int64_t s_block, s_head, s_offset; /* element strides; dim stride must be 1 */
  int32_t block_size;
  int64_t num_blocks;
  const int32_t* block_table; /* [B, max_blocks] */
  int64_t bt_stride;          /* elements between rows of block_table */
  int64_t bt_cols;            /* max_blocks: keys beyond it flag CS_FLAG_BLOCK_INVALID */
  /* dense form (block_table == NULL): k,v [B][nk, Hkv, 128] */
  const void* k;
  const void* v;
  int64_t k_s_batch, k_s_tok, k_s_head;
  int64_t v_s_batch, v_s_tok, v_s_head;
  /* slot form (slots != NULL; cache, strides, block_size and num_blocks as above, the
   * block table is not read): int64 slots [B, slots_cols] */
  const int64_t* slots;
  int64_t slots_stride;       /* elements between requests of slots */
  const void* side_k;         /* bf16 [side_rows, Hkv, 128] or NULL */
  const void* side_v;
  int64_t side_s_row, side_s_head; /* element strides shared by side_k and side_v */
  int64_t side_rows;
  int64_t slots_cols;         /* entries per slots row (> 0 with slots): keys at or past it
                               * read zeros and set CS_FLAG_BLOCK_INVALID */
} cs_kv_source;

/* Prefill (position.py:404-560 for q >> 1) on MFMA.
 *   q [B, nq, Hq, 128] bf16 (strides q_s_batch/q_s_tok/q_s_head, dim stride 1)
 *   qpos [B, nq] int64 (any order, each < nk_b is not required: keys 0..min(qpos,nk-1))
 *   nk [B] int32 key counts; e [128, P] fp32 contiguous (P <= 128: the QE table
 *   of a workgroup lives in LDS; larger tables take cs_ccpe_attention)
 *   out [B, nq, Hq, 128] bf16 contiguous */
int cs_ccpe_prefill_bf16(const void* q, int64_t q_s_batch, int64_t q_s_tok, int64_t q_s_head,
                         const int64_t* qpos, int64_t qpos_s_batch, int32_t batch, int32_t nq,
                         int32_t hq, int32_t hkv, const int32_t* nk, const cs_kv_source* kv,
                         const float* e, int32_t max_positions, void* out, int32_t* flags,
                         void* stream);

/* cope_attention for one query row per request (position.py:404-560 as the
 * decode step calls it, runtime.py:489-508 over the paged.py:433-472 gather).
 * Decode (q = 1 row per request at position nk[b]-1) with speculative
 * split-K: splits are aligned to the last key, split 0 is exact and every
 * other split assumes the gate mass to its right has reached P-1, recording
 * its own gate total (decode_main_kernel).  A second launch, one workgroup
 * per (request, KV head), forms the splits' true carries from the right,
 * recomputes exactly the splits whose carry is below P-1 and merges the
 * splits' (max, sum, accumulator) states into the output rows
 * (decode_finish_kernel).  workspace must hold
 * cs_ccpe_decode_workspace_bytes(batch, hq, max_nk, split) bytes, with any
 * contents; the call refuses a smaller workspace_bytes.  Calls that share a
 * workspace must be ordered (one stream).  A request with nk[b] < 1 sets
 * CS_FLAG_NO_KEY and one with nk[b] > max_nk sets CS_FLAG_CONTEXT_RANGE; the
 * output rows of such requests are not valid.
 *   q [B, Hq, 128] bf16 (q_s_batch, q_s_head), out [B, Hq, 128] bf16. */
int64_t cs_ccpe_decode_workspace_bytes(int32_t batch, int32_t hq, int32_t max_nk,
                                       int32_t split);
/* the decode step itself: cope_attention at one query row (position.py:404-560) */
int cs_ccpe_decode_bf16(const void* q, int64_t q_s_batch, int64_t q_s_head, int32_t batch,
                        int32_t hq, int32_t hkv, const int32_t* nk, int32_t max_nk,
                        const cs_kv_source* kv, const float* e, int32_t max_positions,
                        int32_t split, void* workspace, int64_t workspace_bytes, void* out,
                        int32_t* flags, void* stream);

/* The decode step of cs_ccpe_decode_bf16 over a paged cache whose requests
 * share runs of blocks (reused chunks that several requests' contexts hold,
 * in any order), with the same result: cope_attention at one query row
 * (position.py:404-560, the decode call of runtime.py:489-508).
 *   The keys of request b are split into a head, read from the shared runs,
 * and a tail of its own blocks (the keys nearest the query, and the request's
 * newer tokens).  Head: run i (head_table row i, head_nk[i] keys) is read
 * once for every request; request b attends to its keys up to head_qpos[i, b]
 * (int64, -1: none), with every position taken as P-1.  Tail (tail_table
 * row b, tail_nk[b] keys, query at tail_qpos[b] = tail_nk[b] - 1): exact
 * contextual positions.  The head and tail softmax states are merged per
 * (request, head).  The head's positions are P-1 exactly when the tail's gate
 * mass reaches P-1; where it does not, for any request and head, the call
 * runs cs_ccpe_decode_bf16 over the full block table (kv) instead, so the
 * result is always that call's.
 *   The caller states that each request's head keys and tail keys are
 * together its nk[b] keys, each once, the tail's in key order; the shared
 * blocks' keys carry no position (saturated keys need none), the tail's do.
 * workspace: cs_ccpe_decode_shared_workspace_bytes(batch, hq, head_items,
 * max_nk, split) bytes, 256-byte aligned.  No counterpart in the reference:
 * its decode gathers each request's keys (paged.py:433-472). */
typedef struct cs_decode_shared_args {
  const void* q;              /* [B, Hq, 128] bf16 */
  int64_t q_s_batch, q_s_head;
  int32_t batch, hq, hkv;
  const int32_t* nk;          /* [B] key counts; the query is key nk[b] - 1 */
  int32_t max_nk;
  const cs_kv_source* kv;     /* the cache and every request's full block table */
  const float* e;             /* [128, P] fp32 */
  int32_t max_positions, split;
  const int32_t* head_table;  /* [head_items, head_blocks] */
  int32_t head_items, head_blocks;
  const int32_t* head_nk;     /* [head_items] */
  const int64_t* head_qpos;   /* [head_items, B] */
  const int32_t* tail_table;  /* [B, tail_cols], rows tail_stride apart */
  int64_t tail_stride;
  int32_t tail_cols;
  const int32_t* tail_nk;     /* [B] */
  const int64_t* tail_qpos;   /* [B] */
  void* out;                  /* [B, Hq, 128] bf16 */
  int32_t* flags;
} cs_decode_shared_args;
int64_t cs_ccpe_decode_shared_workspace_bytes(int32_t batch, int32_t hq, int32_t head_items, int32_t max_nk,
                                              int32_t split);
int cs_ccpe_decode_shared_bf16(const cs_decode_shared_args* a, void* workspace, int64_t workspace_bytes,
                               void* stream);

/* Bytes of the static device scratch behind cs_ccpe_decode_bf16_noalloc. */
#define CS_DECODE_SCRATCH_BYTES (64ll << 20)

/* cs_ccpe_decode_bf16 without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The workspace is a static device array of CS_DECODE_SCRATCH_BYTES per GPU,
 * held until the process ends; a call whose
 * cs_ccpe_decode_workspace_bytes(batch, hq, max_nk, split) exceeds it is
 * refused (CS_EINVAL).  Runs on the current device (the stream must belong
 * to it) and allocates nothing.  Every call on one GPU shares the array, so
 * calls that overlap on one GPU (different streams, or threads without
 * ordering) race; calls ordered on one stream do not. */
int cs_ccpe_decode_bf16_noalloc(const void* q, int64_t q_s_batch, int64_t q_s_head,
                                int32_t batch, int32_t hq, int32_t hkv, const int32_t* nk,
                                int32_t max_nk, const cs_kv_source* kv, const float* e,
                                int32_t max_positions, int32_t split, void* out, int32_t* flags,
                                void* stream);

/* ------------------------------------------------------------------------ *
 * SLIDE slot kernels (paged.py:205-240, 433-472; slide.py:103-112).
 * cache [blocks, H, bs, 2D] any dtype; side_k/side_v [S, H, D] (may be absent).
 * A slot s < blocks*bs is native (block s/bs, offset s%bs); s >= blocks*bs is
 * sidecar row s - blocks*bs.  slots [n] int64 device.
 * ------------------------------------------------------------------------ */
int cs_slot_scatter(const cs_view* cache, const cs_view* side_k, const cs_view* side_v,
                    const int64_t* slots, const int64_t* rows, int64_t n,
                    const cs_view* key, const cs_view* value, void* stream);
/* NativePagedKV.gather (paged.py:433-472): key/value rows of slots, in order. */
int cs_slot_gather(const cs_view* cache, const cs_view* side_k, const cs_view* side_v,
                   const int64_t* slots, const int64_t* rows, int64_t n,
                   cs_view* key, cs_view* value, void* stream);

/* The copy-on-write moves of LayerSlotMap.promote_selected over all layers
 * (slide.py:283-360).  Relocation on a stacked cache [L, blocks, H, bs, 2D]:
 * copy whole token records (all layers, heads, K and V) from src_slots[i] to
 * dst_slots[i].
 * Source and destination sets must be disjoint. */
int cs_slot_copy(const cs_view* cache, const int64_t* src_slots, const int64_t* dst_slots,
                 int64_t n, void* stream);
/* Whole-page copy on a stacked cache [L, blocks, H, bs, 2D] (the same moves
 * when a chunk covers whole blocks, slide.py:283-360). */
int cs_page_copy(const cs_view* cache, const int64_t* src_blocks, const int64_t* dst_blocks,
                 int64_t n, void* stream);

/* Token -> slot maps (int64), LayerSlotMap's lookups and updates in bulk
 * (slide.py:54-520): map[tokens[i]] = slots[i]; out[i] = map[tokens[i]]. */
int cs_mapping_scatter(int64_t* map, int64_t map_len, const int64_t* tokens,
                       const int64_t* slots, int64_t n, void* stream);
/* the lookup half, out[i] = map[tokens[i]]: pinned_mapping and the source
 * slots of promote_selected (slide.py:175-192, 264-270) */
int cs_mapping_gather(const int64_t* map, int64_t map_len, const int64_t* tokens,
                      int64_t* out, int64_t n, void* stream);

/* LayerSlotMap's free-slot order (slide.py:103-112) as a bitmap.
 * Free-slot bitmap (bit set = free), nbits slots in ceil(nbits/32) words.
 * release: set bits of slots[0..n).  acquire: take the `count` lowest free
 * slots in ascending order (LayerSlotMap._fresh_slot order), clear them and
 * write them to out; if fewer than count are free nothing changes and
 * *status_out = CS_ECAPACITY (device int32). */
int cs_freelist_release(uint32_t* bitmap, int64_t nbits, const int64_t* slots, int64_t n,
                        void* stream);
/* _fresh_slot, count at a time (slide.py:103-112) */
int cs_freelist_acquire(uint32_t* bitmap, int64_t nbits, int64_t count, int64_t* out,
                        int32_t* status_out, void* stream);

/* ------------------------------------------------------------------------ *
 * WCA (wca.py:55-304).  fp64 throughout; per-token sums are exact
 * (double-double accumulation of the fp64 squares, rounded once).
 * ------------------------------------------------------------------------ */

/* err[t] = sum_{h,d} (new - old)^2 and norm[t] = sum_{h,d} old^2 for rows
 * t of old [T, H, D] selected by old_rows (NULL = identity) and new [n, H, D].
 * ORs 1 into *flags when an input is nonfinite, 2 when err overflows and 16
 * when norm overflows. */
int cs_wca_score(const cs_view* old_rows_src, const int64_t* old_rows, const cs_view* fresh,
                 double* err, double* norm, int32_t* flags, void* stream);

/* adaptation_weight (wca.py:65-93): alpha = err / (norm + eps), optionally
 * clamped to [0, 1]; ORs 2 into *flags
 * when err or norm + eps is nonfinite and 4 when the quotient is nonfinite. */
int cs_wca_alpha(const double* err, const double* norm, int64_t n, double eps, int32_t clamp,
                 double* alpha, int32_t* flags, void* stream);

/* WCAState._promote (wca.py:202-215): available = candidate & ~selected &
 * ~removed; slots = max(0, budget - #selected).  Takes the min(slots,
 * #available) available tokens with the largest key[t] (ties: lower index
 * first), sets selected[t] = 1 and writes them in that order to promoted[0..k).
 * scratch holds 2n int64 and promoted n; *count_out (device) receives k.
 * When abort_flags (device, may be NULL) has a bit of abort_mask set, nothing
 * changes and k = 0: an update that failed its checks promotes nothing.
 * n <= 1<<24.  Two launches: a one-workgroup select/mark/compact pass and an
 * ordering pass over min(budget, n) / 256 workgroups. */
int cs_wca_promote(const double* key, const uint8_t* candidate, const uint8_t* removed,
                   uint8_t* selected, int64_t n, int64_t budget, int64_t* scratch,
                   int64_t* promoted, int64_t* count_out, const int32_t* abort_flags,
                   int32_t abort_mask, void* stream);

/* Ascending indices t with a[t] | b[t] (b may be NULL) -> out[0..*count)
 * (WCAState.active_indices / selected_indices, wca.py:193-200). */
int cs_mask_nonzero(const uint8_t* a, const uint8_t* b, int64_t n, int64_t* out, int64_t* count,
                    void* stream);

/* ORs bit into *flags when a[i] != b[i] for some i < n: the device-side
 * `computed_indices` equality check of WCAState.update (wca.py:241-247). */
int cs_wca_same_rows(const int64_t* a, const int64_t* b, int64_t n, int32_t bit, int32_t* flags,
                     void* stream);

/* The blend of WCAState.update (wca.py:266-276):
 * fused = w * new + (1 - w) * old in fp64 (no contraction), stored in the
 * cache dtype (fp64 -> fp32 -> 16-bit, as torch converts); w = 1 where
 * mandatory[i].  rows [a] index old (NULL = identity); fused_k/v [a,H,D].
 * ORs 8 into *flags when a fused value is nonfinite in the cache dtype. */
int cs_wca_blend(const cs_view* old_k, const cs_view* old_v, const int64_t* rows,
                 const cs_view* new_k, const cs_view* new_v, const double* weight,
                 const uint8_t* mandatory, cs_view* fused_k, cs_view* fused_v,
                 int32_t* flags, void* stream);

/* mean_head_cosine (wca.py:96-112) of a [n, H, D] and rows b_rows of b
 * (NULL = identity) -> out [n]. */
int cs_wca_head_cosine(const cs_view* a, const cs_view* b, const int64_t* b_rows, double eps,
                       double* out, void* stream);

/* WCAState.initialize masks (wca.py:161-171): candidate = reused & (err > 0);
 * counts[0] = #reused, counts[1] = #candidates (device int64); ORs 32 into
 * *flags when a token is neither reused nor mandatory. */
int cs_wca_init_masks(const double* err, const uint8_t* reused, const uint8_t* mandatory,
                      int64_t n, uint8_t* candidate, int64_t* counts, int32_t* flags,
                      void* stream);

/* Weight actually used per active row (wca.py:257-265):
 * used[i] = 1 if mandatory[rows[i]] else (previous_layer ? alpha[rows[i]] : next[i]). */
int cs_wca_used_alpha(const double* alpha, const double* next, const int64_t* rows,
                      const uint8_t* mandatory, int64_t a, int32_t previous_layer,
                      double* used, void* stream);

/* Gate removal (wca.py:277-287): ascending rows[i] with selected[rows[i]] and
 * metric < threshold (metric = cosine, or 1 - cosine when distance_mode). */
int cs_wca_gate(const double* cosine, const int64_t* rows, const uint8_t* selected, int64_t a,
                int32_t distance_mode, double threshold, int64_t* removed, int64_t* count,
                void* stream);

/* Commit (wca.py:289-293): alpha[rows[i]] = next[i]; the *nrem (device int64,
 * NULL = none) tokens of removed[] -- a subset of rows -- are cleared from
 * selected and candidate and set in removed_mask.  When abort_flags (device,
 * may be NULL) has a bit of abort_mask set nothing is written, so the
 * transactional commit of wca.py:289-295 needs no host round trip. */
int cs_wca_commit(double* alpha, const double* next, const int64_t* rows, int64_t a,
                  const int64_t* removed, const int64_t* nrem, uint8_t* selected,
                  uint8_t* candidate, uint8_t* removed_mask, const int32_t* abort_flags,
                  int32_t abort_mask, void* stream);

/* One WCAState.update (wca.py:217-304) in a single call, for callers that
 * have already made the host-side checks: the calls of the entry points above
 * in the order WCAState.update makes them, with the same flag bits --
 * cs_check_finite of cached K (1<<20) and V (1<<22), cs_wca_same_rows of
 * computed (64, skipped when NULL), cs_check_finite of recomputed K (1<<21)
 * and V (1<<23), cs_wca_score, cs_wca_alpha, cs_wca_used_alpha, cs_wca_blend
 * (2, 4, 16, 8), then on gate layers cs_wca_head_cosine and cs_wca_gate, then
 * cs_wca_commit, cs_wca_promote and cs_mask_nonzero of selected | mandatory.
 * The commit and the promotion do nothing when a bit of abort_mask fired.
 * counts: removed (gate), promoted, active.  When the four K/V views are
 * contiguous and 16-byte aligned, their finite checks and the row-list
 * equality run as one launch with the same bits.  The first failing call's
 * status is returned; no call after it is made. */
typedef struct cs_wca_update_args {
  cs_view cached_k, cached_v, recomputed_k, recomputed_v, fused_k, fused_v;
  const int64_t* rows;      /* active rows, ascending [a] */
  const int64_t* computed;  /* the caller's rows [a], or NULL */
  int64_t a, n, budget;
  double* alpha;            /* committed weights [n] */
  const double* deviation;  /* initial deviation [n], the promotion key */
  uint8_t* selected;
  uint8_t* candidate;
  uint8_t* removed_mask;
  const uint8_t* mandatory;
  double* err;              /* work [a] */
  double* norm;             /* work [a] */
  double* next_alpha;       /* work [a] */
  double* cosine;           /* work [a], gate layers */
  double* used;             /* out [a] */
  int64_t* removed;         /* out [a], gate layers */
  int64_t* promoted;        /* out [n] */
  int64_t* scratch;         /* work [2n] */
  int64_t* active;          /* out [n] */
  int32_t* flags;           /* status word */
  int64_t* counts;          /* [3] */
  double epsilon, threshold;
  int32_t clamp, previous_layer, gate, distance_mode, abort_mask;
  int32_t clear_status;     /* bit 0: the call zeroes flags and counts[3] first;
                               bit 1 (needs report): once the report is written the
                               call zeroes them again, so a caller that keeps one
                               block for consecutive calls sets bit 0 only on its
                               first call and after a call that returned an error */
  int64_t* report;          /* NULL, or host-visible int64[4] that receives the flags
                               word and counts[0..2] from the call's last kernel
                               (read it after synchronizing the stream) */
} cs_wca_update_args;

int cs_wca_update(const cs_wca_update_args* u, void* stream);

/* WCAState.initialize (wca.py:151-199, with _promote at wca.py:202-215) in a
 * single call, for callers that have already made the host-side checks
 * (floating [n, H, D] K views of equal shape, dtype and device; bool masks
 * [n]): cs_check_finite of cached K (1<<20) and recomputed K (1<<21) --
 * for bf16 rows with contiguous heads on the score's own loads --,
 * cs_wca_score (2), cs_wca_init_masks (32; counts[0] = reused tokens,
 * counts[1] = candidates), cs_wca_alpha (2|16, 4), then the budget
 * min(ceil(fraction * counts[0]), counts[1]) into counts[2] on the device,
 * the promotion (counts[3], order in promoted[]) and cs_mask_nonzero of
 * selected | mandatory (counts[4]).  The promotion does nothing when any of
 * those bits fired.  Its last kernel copies flags and counts[5] into report
 * (host-visible int64[6]: flags word, then counts[0..4]; read it after
 * synchronizing the stream) and then zeroes them, so a block kept from call
 * to call needs clearing (clear_status bit 0: zeroed by the call first) only
 * when new or after a call that returned an error. */
typedef struct cs_wca_initialize_args {
  cs_view cached_k, recomputed_k;
  const uint8_t* reused;     /* [n] */
  const uint8_t* mandatory;  /* [n] */
  int64_t n;
  double epsilon, fraction;
  int32_t clamp;
  int32_t clear_status;      /* bit 0: zero flags and counts first */
  double* err;               /* out [n] */
  double* norm;              /* out [n] */
  double* alpha;             /* out [n] */
  uint8_t* candidate;        /* out [n] */
  uint8_t* selected;         /* [n], zero on entry */
  const uint8_t* removed;    /* [n], zero */
  int64_t* scratch;          /* work [2n] */
  int64_t* promoted;         /* out [n] */
  int64_t* active;           /* out [n] */
  int32_t* flags;            /* status word */
  int64_t* counts;           /* [5] */
  int64_t* report;           /* host-visible int64[6] */
} cs_wca_initialize_args;

int cs_wca_initialize(const cs_wca_initialize_args* a, void* stream);

/* ------------------------------------------------------------------------ *
 * Row bookkeeping of the selective prefill (runtime.py:408-456).  Row views
 * are [rows, H] with contiguous H; rows move bit for bit (any dtype).  Token
 * lists named "ascending" must be ascending and distinct (else
 * CS_FLAG_ROWS_UNSORTED).
 * ------------------------------------------------------------------------ */

/* Next layer's rows (runtime.py:408-432, replaces the lookup tables and masked
 * copies of CacheSlideRuntime._prefill): out row i takes token active[i]; it
 * continues from in row r with previous[r] == active[i] (previous ascending),
 * else it is restored from snapshot row o with fixed[o] == active[i] (fixed
 * ascending) and *restored (device int64) is incremented; a token in neither
 * list raises CS_FLAG_ROW_LOST (ReuseFailure "a mandatory dynamic row was
 * lost") and its out rows are zeros.  The residual views are optional
 * together; the snapshot views may be absent when no row is restored. */
int cs_rows_remap(const cs_view* hidden_in, const cs_view* residual_in, const cs_view* snap_hidden,
                  const cs_view* snap_residual, cs_view* hidden_out, cs_view* residual_out,
                  const int64_t* previous, int64_t n_prev, const int64_t* active, int64_t n_active,
                  const int64_t* fixed, int64_t n_fixed, int64_t* restored, int32_t* flags,
                  void* stream);

/* *count (device int64) += number of active tokens not in previous (ascending):
 * the rows cs_rows_remap restores (runtime.py:415-418 `continuing`). */
int cs_rows_missing(const int64_t* previous, int64_t n_prev, const int64_t* active,
                    int64_t n_active, int64_t* count, void* stream);

/* out[j] = rows[k] for tokens[k] == j (tokens ascending), zeros for every other
 * row of out (runtime.py:454-456: output = zeros; output[previous] = hidden);
 * a token outside [0, rows of out) raises CS_FLAG_ROW_INDEX. */
int cs_rows_scatter(const cs_view* rows, const int64_t* tokens, int64_t m, cs_view* out,
                    int32_t* flags, void* stream);

/* out[i] = src[idx[i]] (the hidden[fixed] / residual[fixed] snapshots of
 * runtime.py:420-431); an index outside src raises CS_FLAG_ROW_INDEX. */
int cs_rows_gather(const cs_view* src, const int64_t* idx, int64_t m, cs_view* out,
                   int32_t* flags, void* stream);

/* ------------------------------------------------------------------------ *
 * Layer snapshots between host memory and HBM (runtime.py:192-256).
 * ------------------------------------------------------------------------ */
enum cs_copy_kind { CS_COPY_H2D = 0, CS_COPY_D2H = 1, CS_COPY_D2D = 2 };

/* hipMemcpyAsync of `bytes` on `stream`.  Replaces the host<->device moves of a
 * snapshot: `tensor.to(device=..., dtype=...)` after safetensors decoding in
 * `_read` (runtime.py:227-229) and `tensor.detach().contiguous().cpu()` in
 * `_put` (runtime.py:238-243).  The host side should be pinned memory for an
 * asynchronous DMA. */
int cs_copy_async(void* dst, const void* src, int64_t bytes, int32_t kind, void* stream);

/* The finite check and dtype conversion of a decoded snapshot tensor
 * (runtime.py:224-229: `torch.isfinite(tensor).all()` then
 * `tensor.to(dtype=dtype)`): raises `bit` in flags when src holds a non-finite
 * value and writes dst = src converted with torch's rounding.  dst absent (or
 * equal to src) checks only.  Both views contiguous, floating point. */
int cs_snapshot_convert(const cs_view* src, const cs_view* dst, int32_t bit, int32_t* flags,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CACHESLIDE_HIP_H */
