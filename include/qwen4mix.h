/* qwen4mix: the qwen4exp token-mixing path (QSA + Gated DeltaNet) on MI355X.
 *
 * C ABI of libqwen4mix.so. Every entry point takes raw device pointers, plain
 * sizes, a dtype enum and the caller's HIP stream; the caller owns all memory
 * (kernels never allocate), state is updated in place, and the return value is
 * QM_OK or a negative QM_ERR_* code whose message qm_last_error() returns
 * (thread-local). There is no fallback path: an unsupported shape is an error.
 *
 * The reference has no C ABI; its plugin surface for this path is the Python
 * module interface of src/ttrunner_qwen38_flash_next/reference/. Each entry
 * point below cites the reference function(s) whose arithmetic it replaces.
 *
 * Layouts (b = sequence, h = head, d = head_dim, P = page_size):
 *   DeltaNet recurrent state  float32 [B, Hv, d_k, d_v]   (reference/cache.py:24)
 *   DeltaNet conv ring        act     [B, conv_dim, K]    slot p % K holds the
 *                              input of the token at position p
 *   QSA K pool                bf16    [n_pages, Hkv, P * d]  each page of a
 *                              kv head in MFMA lane order: 16-token x
 *                              32-channel tiles of 1 KB
 *   QSA V pool                bf16    [n_pages, Hkv, P * d]  32-token x
 *                              16-channel tiles of 1 KB, tokens of a group in
 *                              the PV MFMA's order (qm_v_slot)
 *                              (qm_qsa_page_index() maps (row, channel) of a
 *                              page to its element offset in either pool)
 *   page table                int32   [B, max_pages]  logical page -> physical
 *   indexer raw keys          act     [B, max_ctx, idx_dim]
 *   indexer block cache       float32 [B, max_blocks, idx_dim]  pooled, normed,
 *                              roped keys of complete blocks, each row permuted:
 *                              element d at (d % 16) * 8 + d / 16
 *   rope tables               float32 [n_pos, rope_dim]  (cos, sin)
 */
#ifndef QWEN4MIX_H
#define QWEN4MIX_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QM_OK 0
#define QM_ERR_ARG (-1)
#define QM_ERR_DTYPE (-2)
#define QM_ERR_LAUNCH (-3)
#define QM_ERR_WORKSPACE (-4)
#define QM_ERR_UNSUPPORTED (-5)

#define QM_ACT_F32 0
#define QM_ACT_BF16 1

#define QM_GEMV_MAX_SEG 8

/* Last error message of the calling thread ("" after success). */
const char* qm_last_error(void);
/* ABI version of this library. */
int qm_version(void);

/* ------------------------------------------------------------------------ */
/* Gated DeltaNet                                                           */
/* ------------------------------------------------------------------------ */

typedef struct qm_dn_geom {
  int batch;        /* sequences in the call                           */
  int n_v_heads;    /* Hv (32)                                          */
  int n_k_heads;    /* Hk (16); v-head j reads q/k head j % Hk          */
  int head_dim;     /* d_k = d_v (128)                                   */
  int conv_kernel;  /* K (4)                                             */
  int act_dtype;    /* QM_ACT_F32 or QM_ACT_BF16                         */
  float eps;        /* rms_norm_eps of the gated output norm             */
} qm_dn_geom;

/* Bytes of workspace qm_dn_decode needs; zero it once before first use (the
 * kernel leaves it ready for the next call). */
size_t qm_dn_decode_workspace(int batch, int n_v_heads, int head_dim);

/* One decode step of the DeltaNet mixer core, fused into one launch.
 * Replaces the seq == 1 body of Qwen4ExpModel._linear_attention between its
 * projections and ssm_out (reference/model.py:189-243): causal_conv1d_step
 * (reference/layers.py:141-147), the gates (reference/model.py:212-217), the
 * tiled q/k expansion (:230-233), recurrent_gated_delta_rule
 * (reference/layers.py:155-192) and rms_norm_gated (reference/layers.py:46-61).
 *   qkv [B, conv_dim], z [B, Hv*d], a, b [B, Hv]: projection outputs (act)
 *   a_neg, dt_bias [Hv] f32 (ssm_a, ssm_dt.bias); conv_w [conv_dim, K] act;
 *   norm_w [d] f32; positions [B] int32 position of this token;
 *   conv_ring, state: in/out; out [B, Hv*d] act (input of ssm_out). */
int qm_dn_decode(const qm_dn_geom* g, const void* qkv, const void* z, const void* a, const void* b,
                 const float* a_neg, const float* dt_bias, const void* conv_w, const float* norm_w,
                 const int* positions, void* conv_ring, float* state, void* out, void* workspace,
                 size_t workspace_bytes, hipStream_t stream);

/* Hand-off health of qm_dn_decode's workspace: *giveups = the number of
 * waits for the other workgroups of a head that gave up since the last reset
 * (a correct launch never gives up; the output of such a head is NaN). Waits
 * for the stream. reset != 0 then zeroes the workspace, the state of a fresh
 * one. No counterpart in the reference: its device ops return no such state. */
int qm_dn_decode_check(int batch, int n_v_heads, int head_dim, void* workspace, size_t workspace_bytes, int reset,
                       unsigned* giveups, hipStream_t stream);

/* Depthwise causal conv1d over (B, C, T), the free functions causal_conv1d
 * (reference/layers.py:133-138, state == NULL: zero history) and
 * causal_conv1d_step (reference/layers.py:141-147, with the rolling state):
 *   full = [state | x] (K-1 + T columns), out[b,c,t] = silu?(sum_j w[c,j]
 *   full[b,c,t+j]) with tap 0 the oldest; new_state = full[:, :, T:].
 *   x, out [B, C, T]; state, new_state [B, C, K-1] (either may be NULL;
 *   new_state may be state itself); weight [C, K]; all act_dtype, contiguous;
 *   out must not alias x or state. 1 <= K <= 8. */
int qm_causal_conv1d(int act_dtype, int batch, int channels, int seq, int taps, const void* x, const void* state,
                     const void* weight, int activation, void* out, void* new_state, hipStream_t stream);

/* The gated delta rule over T tokens on split, expanded inputs:
 * recurrent_gated_delta_rule (reference/layers.py:155-192).
 *   q, k [B, T, H, d], v [B, T, H, d] act; g, beta [B, T, H] f32;
 *   state [B, H, d, d] f32 in/out; out [B, T, H, d] act. */
int qm_dn_recurrent(int act_dtype, int batch, int seq, int heads, int head_dim, const void* q, const void* k,
                    const void* v, const float* g, const float* beta, float* state, void* out,
                    hipStream_t stream);

/* Bytes of workspace qm_dn_chunked needs: one fp32 record of 147712 bytes per
 * (sequence, head, 64-token chunk). 0 for an unsupported head_dim. */
size_t qm_dn_chunked_workspace(int batch, int seq, int heads, int head_dim);

/* The same rule in the chunked WY/UT form, 64-token chunks:
 * chunk_gated_delta_rule (reference/layers.py:195-275). Same arguments and
 * result (to float32 rounding) as qm_dn_recurrent, plus a workspace of
 * qm_dn_chunked_workspace() bytes (no initial contents needed). */
int qm_dn_chunked(int act_dtype, int batch, int seq, int heads, int head_dim, const void* q, const void* k,
                  const void* v, const float* g, const float* beta, float* state, void* out, void* workspace,
                  size_t workspace_bytes, hipStream_t stream);

/* Bytes of workspace qm_dn_prefill needs for a chunk of `seq` tokens. */
size_t qm_dn_prefill_workspace(const qm_dn_geom* g, int seq);

/* The DeltaNet mixer core over a chunk of `seq` tokens (prefill): the seq > 1
 * body of Qwen4ExpModel._linear_attention (reference/model.py:198-201,
 * 205-243): causal conv over [history | chunk] (reference/layers.py:133-138)
 * with the last K-1 inputs left in the ring, the gates, the delta rule
 * (chunk_gated_delta_rule, reference/layers.py:195-275; token loop for short
 * chunks) and rms_norm_gated. positions[b] = position of the chunk's first
 * token. Shapes as qm_dn_decode with a [B, S, ...] token axis. */
int qm_dn_prefill(const qm_dn_geom* g, int seq, const void* qkv, const void* z, const void* a, const void* b,
                  const float* a_neg, const float* dt_bias, const void* conv_w, const float* norm_w,
                  const int* positions, void* conv_ring, float* state, void* out, void* workspace,
                  size_t workspace_bytes, hipStream_t stream);

/* qm_dn_prefill without a workspace argument: the same kernels, with the
 * library's own scratch, one array of qm_dn_prefill_noalloc_max_bytes()
 * (32 MiB) per device, held until the process ends. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid hipMalloc); it calls no hipMalloc/hipFree.
 * A chunk whose qm_dn_prefill_workspace() exceeds the scratch (about 256
 * tokens at batch 1 and 32 value heads) is refused with QM_ERR_UNSUPPORTED.
 * Every call on one device shares that device's array: calls that overlap on
 * one GPU (other streams, other threads) race. */
int qm_dn_prefill_noalloc(const qm_dn_geom* g, int seq, const void* qkv, const void* z, const void* a, const void* b,
                          const float* a_neg, const float* dt_bias, const void* conv_w, const float* norm_w,
                          const int* positions, void* conv_ring, float* state, void* out, hipStream_t stream);
/* Bytes of the built-in scratch of qm_dn_prefill_noalloc. */
size_t qm_dn_prefill_noalloc_max_bytes(void);

/* ------------------------------------------------------------------------ */
/* QSA (Qwen Sparse Attention)                                              */
/* ------------------------------------------------------------------------ */

typedef struct qm_qsa_geom {
  int batch;        /* sequences                                          */
  int n_heads;      /* Hq (16)                                            */
  int n_kv_heads;   /* Hkv (2); q-head h reads kv-head h / (Hq/Hkv)       */
  int head_dim;     /* 256                                                */
  int rope_dim;     /* rotated leading channels (64)                      */
  int idx_heads;    /* indexer query heads (4)                            */
  int idx_dim;      /* indexer head dim (128)                             */
  int ratio;        /* indexer compress ratio = block size (64)           */
  int budget;       /* indexer budget in tokens (2048): top budget/ratio  */
  int page_size;    /* KV page size (64)                                  */
  int max_pages;    /* page-table row length                              */
  int max_ctx;      /* raw-key cache rows per sequence                    */
  int max_blocks;   /* block-cache rows per sequence                      */
  int act_dtype;    /* QM_ACT_F32 or QM_ACT_BF16                          */
  float eps;        /* rms_norm_eps                                       */
} qm_qsa_geom;

/* Position of page row `row` among the 32 token slots of its V tile group. */
int qm_v_slot(int row);
/* Element offsets, within one page of one kv head, of (row, channel) in the
 * K pool (k_index) and the V pool (v_index), for every row < page_size and
 * channel < head_dim (row-major [page_size, head_dim] int arrays). Host only;
 * for export, import and inspection of the pools. */
int qm_qsa_page_index(int page_size, int head_dim, int* k_index, int* v_index);

/* Per-token preparation for a decode step (or the S rows of a prefill chunk):
 * q/k RMS norm and partial rope, q|gate split (reference/model.py:345-356);
 * the current K/V appended at their page slots (reference/model.py:358-363;
 * paging as tt/model.py:625-666); the indexer query rope(rms_norm(.))
 * (reference/model.py:270-272); the raw indexer key appended
 * (reference/model.py:274-279); and, for every block the new tokens complete,
 * its pooled, normed, roped key written to the block cache
 * (reference/model.py:289-294; block cache as tt/model.py:1043-1115).
 *   seq: rows per sequence in this call (1 for decode)
 *   qg [B, S, Hq, 2*d]; k_new, v_new [B, S, Hkv, d]; iq [B, S, idx_heads*idx_dim];
 *   ik [B, S, idx_dim] (act); *_norm f32 weights; cos/sin [n_pos, rope_dim] f32;
 *   positions [B] int32 = position of the first row; page_table [B, max_pages].
 *   Outputs: q_out, B*S*2*Hq*d bf16: the normed, roped query as hi and lo
 *   parts (hi = bf16(q), lo = bf16(q - hi)), in the operand order of the
 *   attention MFMA: element (row, part, head h, channel c) at
 *   ((((((row*Hkv + h/8)*2 + part)*8 + c/32)*4 + (c%32)/8)*8 + h%8)*8 + c%8;
 *   iq_out [B, S, idx_heads, idx_dim] f32; pools, raw keys and block cache
 *   updated in place.
 *   qg may be NULL (no attention query: q_norm, q_out unused) and k_new/v_new
 *   may both be NULL (no K/V append), which leaves the indexer part alone. */
int qm_qsa_prep(const qm_qsa_geom* g, int seq, const void* qg, const void* k_new, const void* v_new,
                const void* iq, const void* ik, const float* q_norm, const float* k_norm,
                const float* iq_norm, const float* ik_norm, const float* cos, const float* sin,
                const int* positions, const int* page_table, void* k_pool, void* v_pool, void* raw_keys,
                float* block_keys, void* q_out, float* iq_out, hipStream_t stream);

/* Pooled keys of blocks first_block .. first_block+n_blocks-1 recomputed from
 * the raw-key cache (reference/model.py:289-294), for a history imported into
 * the caches rather than appended through qm_qsa_prep (tt/model.py:1043-1115
 * keeps the same block cache). raw_keys [B, max_ctx, idx_dim] act;
 * block_keys [B, max_blocks, idx_dim] f32. */
int qm_qsa_pool_blocks(const qm_qsa_geom* g, const void* raw_keys, const float* k_norm, const float* cos,
                       const float* sin, int first_block, int n_blocks, float* block_keys, hipStream_t stream);

/* int2 entries per query row of the attention item table (see qm_qsa_select). */
int qm_qsa_items_stride(const qm_qsa_geom* g);

/* Block scoring and top-k selection for each query row: scores
 * sum_h relu(q_h . block_j) / sqrt(idx_dim) (reference/model.py:297-298) over
 * the eligible blocks j*ratio + ratio - 1 <= p, top min(budget/ratio, eligible)
 * with ties to the lower index (reference/model.py:300-313; the lower-index
 * rule is this library's; torch leaves tie order unspecified).
 *   iq [B, S, idx_heads, idx_dim] f32; block_keys as above; positions [B] first
 *   row's position; ids [B, S, budget/ratio] int32 in rank order; n_sel [B, S];
 *   scores_out [B, S, max_blocks] f32 or NULL (ineligible entries -inf). Given
 *   scores_out, the scores are computed by a launch of their own spread over
 *   the blocks (the way to select among many blocks: a long-context decode
 *   row), and the ranking launch reads them back.
 *   items [B, S, qm_qsa_items_stride(g)] int2 or NULL: the attention work list
 *   of each row -- entry 0 holds the count, then one entry per 32-token group
 *   of the selected blocks (rank order) and of the row's tail block: physical
 *   pool row of the group's first token (page_table lookup, paging as
 *   tt/model.py:1252-1323) and its visible rows [lo, hi) as lo | hi << 8.
 *   page_table [B, max_pages] is needed when items is given. */
int qm_qsa_select(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys, const int* positions,
                  const int* page_table, int* ids, int* n_sel, void* items, float* scores_out,
                  hipStream_t stream);

/* The decode (one token per sequence) front end in one launch: qm_qsa_prep's
 * work for the query and key/value heads, plus, per sequence, the raw indexer
 * key append, the indexer query, the pooled key of the block this token
 * completes (if any) and qm_qsa_select -- the same results as qm_qsa_prep
 * followed by qm_qsa_select with seq = 1 (reference/model.py:248-363). */
int qm_qsa_decode_front(const qm_qsa_geom* g, const void* qg, const void* k_new, const void* v_new, const void* iq,
                        const void* ik, const float* q_norm, const float* k_norm, const float* iq_norm,
                        const float* ik_norm, const float* cos, const float* sin, const int* positions,
                        const int* page_table, void* k_pool, void* v_pool, void* raw_keys, float* block_keys,
                        void* q_out, float* iq_out, int* ids, int* n_sel, void* items, hipStream_t stream);

/* Workgroups per kv head of qm_qsa_decode for queries up to max_position: the
 * largest number of 32-token attention items of any position in the last
 * `ratio` positions up to it (at most 1024). */
int qm_qsa_decode_splits(const qm_qsa_geom* g, int max_position);
/* Bytes of workspace qm_qsa_decode needs; zero it once before first use and
 * keep it for that geometry: it holds, per (sequence, kv head), a generation
 * word, a give-up counter (its second word; nonzero only if a wait for the
 * other workgroups' partials ever gave up, which a correct launch never does),
 * the workgroups' flags and their partials. Calls that overlap on one
 * workspace race. */
size_t qm_qsa_decode_workspace(const qm_qsa_geom* g, int splits);

/* Workgroups of one (sequence, kv head) group of qm_qsa_decode for `splits`:
 * max(splits, 64) (short contexts widen the grid so every output slice has its
 * own merging workgroup). */
int qm_qsa_decode_group(int splits);
/* Resident capacity of the qm_qsa_decode kernel that `splits` selects on the
 * current device: workgroups that fit at once (occupancy per compute unit x
 * compute units), or a negative QM_ERR_* code (no device). */
int qm_qsa_decode_resident(int act_dtype, int splits);
/* QM_OK if a group of qm_qsa_decode_group(splits) workgroups fits `resident`
 * resident workgroups (every workgroup of a group waits for the others, so the
 * whole group must be on the device at once), else QM_ERR_UNSUPPORTED or
 * QM_ERR_ARG. qm_qsa_decode applies it with qm_qsa_decode_resident. */
int qm_qsa_decode_fits(int splits, int resident);
/* Hand-off health of qm_qsa_decode's workspace since the last reset:
 * counts[0] = waits for a group's partials that gave up, counts[1] = launches
 * whose position had more attention items than `splits` (a plan sized for
 * smaller positions). Either leaves NaN in the affected output; a correct
 * plan keeps both zero. Waits for the stream. reset != 0 then zeroes the
 * generation words and flags, the state of a fresh workspace. No counterpart in
 * the reference: its device ops return no such state. */
int qm_qsa_decode_check(const qm_qsa_geom* g, int splits, void* workspace, size_t workspace_bytes, int reset,
                        unsigned* counts, hipStream_t stream);

/* One QSA decode step (one token per sequence) in a single launch: everything
 * qm_qsa_decode_front + qm_qsa_attend compute -- token prep and K/V append,
 * raw indexer key append and block pooling, indexer query, block scores and
 * top-k, paged GQA attention over the selected blocks and the tail, sigmoid
 * gate (reference/model.py:248-382). Every working workgroup recomputes the
 * selection it needs and attends one 32-token item; the partials cross to the
 * workgroups that merge them inside the same launch.
 * Requires max_blocks, max_pages <= 2048, budget/ratio <= 256, ratio <= 64,
 * 1 <= splits <= 1024 (qm_qsa_decode_splits) and a group that fits the device
 * (qm_qsa_decode_fits); positions whose items exceed `splits` are counted and
 * poisoned (qm_qsa_decode_check).
 *   out [B, Hq*d] act; ids [B, budget/ratio], n_sel [B], items, iq_out
 *   [B, idx_heads, idx_dim] are optional inspection outputs (may be NULL);
 *   ids lists the selected blocks in block order when at most 128 blocks are
 *   eligible, in rank order otherwise (the items follow the same order). */
int qm_qsa_decode(const qm_qsa_geom* g, const void* qg, const void* k_new, const void* v_new, const void* iq,
                  const void* ik, const float* q_norm, const float* k_norm, const float* iq_norm,
                  const float* ik_norm, const float* cos, const float* sin, const int* positions,
                  const int* page_table, void* k_pool, void* v_pool, void* raw_keys, float* block_keys, void* out,
                  int splits, void* workspace, size_t workspace_bytes, int* ids, int* n_sel, void* items,
                  float* iq_out, hipStream_t stream);

/* Bytes of workspace qm_qsa_attend needs for `seq` query rows and `splits`. */
size_t qm_qsa_attend_workspace(const qm_qsa_geom* g, int seq, int splits);
/* Split count (workgroups per row and kv head) covering every query row at
 * positions first_position .. last_position. */
int qm_qsa_attend_splits(const qm_qsa_geom* g, int first_position, int last_position);

/* Paged GQA attention of `seq` query rows per sequence over each row's item
 * list (its selected blocks plus its tail block), then the sigmoid output gate
 * (reference/model.py:365-382 with the mask of :306-326): fp32 softmax of
 * q.k/sqrt(d) over the visible keys, times v, cast to act, times
 * sigmoid(gate). K/V of every row must already be in the pages (qm_qsa_prep).
 *   q: qm_qsa_prep's q_out (hi/lo, operand order); qg [B, S, Hq, 2*d] act (the gate is
 *   the second half of each head); items from qm_qsa_select;
 *   out [B, S, Hq*d] act. */
int qm_qsa_attend(const qm_qsa_geom* g, int seq, const void* q, const void* qg, const void* k_pool,
                  const void* v_pool, const void* items, void* out, int splits, void* workspace,
                  size_t workspace_bytes, hipStream_t stream);

/* Bytes of workspace qm_qsa_attend_chunk needs for `seq` query rows. */
size_t qm_qsa_attend_chunk_workspace(const qm_qsa_geom* g, int seq);

/* The same attention as qm_qsa_attend for a chunk of `seq` consecutive query
 * rows per sequence (the prefill form of reference/model.py:365-382 with the
 * mask of :306-326), organised by key block instead of by row: the rows'
 * selected-block entries are filed under their blocks on the device, each
 * block's keys and values are read once and scored for every row that attends
 * it (a tail block only up to the row's own position), and a row's partials
 * are merged with the gate. Indexer ratio 32 or 64, at most 4096 blocks.
 *   q (qm_qsa_prep's q_out) and qg [B, S, Hq, 2*d] act as qm_qsa_attend;
 *   positions [B] = position of row 0; ids [B, S, budget/ratio] and n_sel
 *   [B, S] from qm_qsa_select; out [B, S, Hq*d] act.
 * The workspace holds a slot table per (block, row), filed on the way in and
 * cleared by the merge, so every call leaves it zero: zero-fill it before its
 * first use, keep it for one (batch, max_blocks) geometry (a workspace sized
 * for a longer chunk serves a shorter one), and do not let two calls on it
 * overlap. */
int qm_qsa_attend_chunk(const qm_qsa_geom* g, int seq, const void* q, const void* qg, const void* k_pool,
                        const void* v_pool, const int* positions, const int* page_table, const int* ids,
                        const int* n_sel, void* out, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* qm_qsa_select for a chunk of `seq` rows that also files every row's
 * selection into a qm_qsa_attend_chunk workspace (the step qm_qsa_attend_chunk
 * otherwise runs as a kernel of its own), for qm_qsa_attend_chunk_filed. Same
 * ids and n_sel as qm_qsa_select; the conditions and the workspace rules of
 * qm_qsa_attend_chunk. No counterpart in the reference: it composes the
 * selection (reference/model.py:248-327) with the chunk attention's own
 * bookkeeping, to save a launch per chunk. */
int qm_qsa_select_chunk(const qm_qsa_geom* g, int seq, const float* iq, const float* block_keys,
                        const int* positions, int* ids, int* n_sel, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* qm_qsa_attend_chunk over a workspace that qm_qsa_select_chunk has just
 * filed (the same call's rows and geometry): the attention and the merge
 * only. No counterpart in the reference (see qm_qsa_select_chunk). */
int qm_qsa_attend_chunk_filed(const qm_qsa_geom* g, int seq, const void* q, const void* qg, const void* k_pool,
                              const void* v_pool, const int* positions, const int* page_table, void* out,
                              void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The layer projections at small M (the F.linear calls of
 * reference/model.py:184-187, 244, 270, 274, 345-352, 383 for decode):
 * y[m][n] = sum_k w[n][k] x[m][k] for m < M <= 4, one stream over w.
 *   w [n, k] and x [m, k] in act_dtype (row-major); k = 2048 or 4096 (bf16),
 *   1024, 2048 or 4096 (f32). The n rows split into n_seg <= 8 consecutive
 *   segments of seg_rows[s] rows: segment s is written to seg_out[s] as
 *   [m, seg_rows[s]] (act_dtype). seg_rows and seg_out are host arrays.
 *   Products accumulate in f32 and are rounded once to act_dtype. */
int qm_gemv(int act_dtype, int m, int n, int k, const void* w, const void* x, int n_seg, const int* seg_rows,
            void* const* seg_out, hipStream_t stream);

/* A branch's output projection with the hyper-connection reinjection as its
 * epilogue: the output projection of reference/model.py:244 (ssm_out) or :383
 * (attn_output) followed by Qwen4ExpModel._reinject (reference/model.py:79-81).
 * y = w x as qm_gemv computes it (one segment of n rows, rounded to act), then
 * hyper[m][s * n + j] = round(hyper[m][s * n + j] + round(y[m][j] * inject[m][s]))
 * for every stream s < streams, in place. hyper [m, streams * n],
 * inject [m, streams] act; m, k as qm_gemv. */
int qm_gemv_reinject(int act_dtype, int m, int n, int k, const void* w, const void* x, int streams,
                     const void* inject, void* hyper, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Hyper-connections around each branch                                     */
/* ------------------------------------------------------------------------ */

typedef struct qm_hc_geom {
  int rows;         /* M: token rows (batch * seq)                         */
  int streams;      /* hc_count (4): copies of the hidden vector            */
  int hidden;       /* hidden_size: width of one stream                     */
  int rank;         /* hc_lowrank (320): width of the down/up products      */
  int act_dtype;    /* QM_ACT_F32 or QM_ACT_BF16                            */
  float eps;        /* rms_norm_eps of the stream norm                      */
} qm_hc_geom;

/* Bytes of workspace qm_hc_mix needs (normalised rows and the down product);
 * 0 if the geometry is unsupported. */
size_t qm_hc_mix_workspace(const qm_hc_geom* g);

/* The hyper-connection read gate, Qwen4ExpModel._gated_residual
 * (reference/model.py:53-77): per-stream rms_norm of hyper, the down and
 * inject products, silu / 2 sigmoid of their outputs over `streams`, the up
 * product, sigmoid, and the mean over streams of gate * normed.
 *   hyper [M, streams * hidden] act; norm_w [streams * hidden] f32;
 *   down_inject_w [rank + (with_inject ? streams : 0), streams * hidden] act:
 *   the down rows, then the inject rows; up_w [streams * hidden, rank] act.
 *   mixed [M, hidden] act (the branch input); inject [M, streams] act when
 *   with_inject (the layer mixers), unused otherwise (the final mixer).
 *   streams * hidden must be 1, 2, 4, 5, 8 or 10 times 2048 (bf16) or 1024
 *   (f32); hidden a multiple of 8; rank a multiple of 8 (4 for f32), <= 512.
 * Two launches; every pointer except inject and mixed 16-byte aligned. */
int qm_hc_mix(const qm_hc_geom* g, const void* hyper, const float* norm_w, const void* down_inject_w,
              int with_inject, const void* up_w, void* mixed, void* inject, void* workspace,
              size_t workspace_bytes, hipStream_t stream);

/* Qwen4ExpModel._reinject (reference/model.py:79-81):
 * out[m][s * hidden + h] = hyper[m][s * hidden + h] + branch[m][h] * inject[m][s],
 * each product and sum rounded to act. hyper/out [M, streams * hidden],
 * branch [M, hidden], inject [M, streams]; out may be hyper. Reads rows,
 * streams, hidden and act_dtype of g (hidden a multiple of 8). */
int qm_hc_reinject(const qm_hc_geom* g, const void* hyper, const void* branch, const void* inject, void* out,
                   hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN4MIX_H */
