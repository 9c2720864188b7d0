/*
 * pfa_hip.h -- C ABI of libpfa_hip.so, the MI355X (gfx950) kernels behind the
 * ASPA (Adaptive Sparse Proto Attention) forward path.
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and a hipStream_t passed as void*;
 *   - enqueues work on that stream and returns without synchronising;
 *   - allocates nothing: scratch memory is passed in as a caller-owned
 *     workspace whose size is obtained from the matching *_workspace_size();
 *   - returns 0 on success, a positive hipError_t value when a HIP call
 *     failed, or a negative PFA_E_* code for an argument error.  The message
 *     of the most recent failure on the calling thread is available from
 *     pfa_last_error_string().
 *
 * Index conventions: token indices, packed row offsets and candidate lists
 * are int32 on the device.  Tensors the reference exposes as int64 are
 * widened by the Python layer only where its public API returns them.
 *
 * Each declaration names the reference function (file:line, relative to the
 * Proteus-Flux-Attention source tree) whose behaviour it replaces.
 */
#ifndef PFA_HIP_H
#define PFA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------- */
#define PFA_OK 0
#define PFA_E_INVALID (-1)      /* bad size / flag / pointer combination   */
#define PFA_E_UNSUPPORTED (-2)  /* valid request this build does not cover */
#define PFA_E_WORKSPACE (-3)    /* workspace smaller than required         */

/* ---- element type tags ---------------------------------------------- */
#define PFA_F32 0
#define PFA_BF16 1
#define PFA_F16 2
#define PFA_I8 3   /* symmetric int8 with a float scale per head */

/* Library version (major*10000 + minor*100 + patch). */
int pfa_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* pfa_last_error_string(void);

/* ====================================================================
 * Router: SwitchRouter logits+softmax, prototype prior, blend, usage boost,
 * renormalisation, importance and head top-k in one pass over x.
 * Replaces SwitchRouter.forward (src/proteus_attention/models/aspa.py:149-157),
 * AdaptiveSparseAttention._route_tokens (aspa.py:628-690), the importance
 * blend (aspa.py:1521-1530), gate->head aggregation (aspa.py:1540-1542) and
 * torch.topk over heads (aspa.py:1590-1591).  Ties in the head top-k go to
 * the lowest head index.
 *
 *   x            (n_tok, C) in x_dtype (PFA_F32 / PFA_BF16 / PFA_F16)
 *   w_packed     (C, 2*Gp) f32 with Gp = pfa_router_gate_pad(G), channel-
 *                interleaved: w_packed[c][g] = head_router.linear.weight[g][c]
 *                (its x_dtype value) and w_packed[c][Gp+g] = the L2-
 *                normalised prototype P[g][c]; padding gates are zero.  With
 *                use_proto == 0 only the first Gp columns are read.
 *   conf_weight  (G) f32 = routing_confidence + 1e-6, or NULL
 *   usage_bias   (G) f32 = softmax(-(usage+1e-6)), or NULL (boost off)
 *   gate_to_head (G) int32, values in [0, H)
 *   outputs (NULL allowed for any of the optional ones):
 *     gate_probs (n_tok, G) f32, sim (n_tok) f32, blend (n_tok) f32,
 *     importance (n_tok) f32 (required), head_idx (n_tok, topk) int32
 *     (required, each row ranked best first), head_score (n_tok, topk) f32,
 *     stats_partial (n_blocks, 8) f32: per workgroup the sums of router
 *     entropy, max prototype similarity, blend, count(blend > 0) and top-k
 *     head scores (telemetry of aspa.py:1857-1916); n_blocks from
 *     pfa_router_block_count().
 *   ema_partial (n_blocks, G, C+1) f32 or NULL: the prototype EMA statistics
 *     of aspa.py:703-707 fused into the same pass -- per workgroup of 64
 *     tokens, sum_t gate[t,g]*x[t,c] (columns 0..C-1) and sum_t gate[t,g]
 *     (column C) over the final gate probabilities; reduce them with
 *     pfa_proto_partial_reduce(ema_partial, n_blocks, ...).  Column C and
 *     the other shapes sum in token order; bf16 x with G <= 8 sums the
 *     columns 0..C-1 on MFMA from exact products (each gate split into
 *     three bf16 parts), in a fixed order.  Deterministic either way; equal
 *     to pfa_proto_accumulate's sums up to f32 rounding.
 * ==================================================================== */
int pfa_router_gate_pad(int G);
/* Sum of the router's per-workgroup telemetry partials (stats_partial
 * (n_blocks, 8) of pfa_router_topk) column by column in float64, into out[8]
 * (fixed summation order).  No counterpart in the reference, which reduces
 * these statistics with tensor ops; a single 64-byte result keeps the
 * device-to-host telemetry copy small. */
int pfa_router_stats_reduce(const float* stats_partial, int n_blocks, double* out, void* stream);

int pfa_router_block_count(int64_t n_tok, int* n_blocks);

/* Per-forward router inputs in one launch (replaces the tensor ops of
 * aspa.py:636-663 that feed the router): w_packed (C, 2*Gp) f32 from
 * head_router.linear.weight (G, C) in w_dtype (rounded to x_dtype) and the
 * L2-normalised prototypes (G, C) (F.normalize, eps 1e-6; protos NULL: proto
 * columns zero); conf_weight (G) f32 = confidence + 1e-6 rounded to buf_dtype
 * (confidence NULL: not written); usage_bias (G) f32 = softmax(-(usage +
 * 1e-6)) in buf_dtype (usage NULL: not written).  protos, confidence and
 * usage share buf_dtype. */
int pfa_router_prepare(const void* w_router, int w_dtype, const void* protos,
                       const void* confidence, const void* usage, int buf_dtype,
                       int G, int C, int x_dtype, float* w_packed,
                       float* conf_weight, float* usage_bias, void* stream);
int pfa_router_topk(const void* x, int x_dtype, int64_t n_tok, int C, int G,
                    const float* w_packed, int use_proto,
                    const float* conf_weight, const float* usage_bias,
                    const int32_t* gate_to_head, int H, int topk,
                    float proto_temp, float proto_threshold, float proto_blend,
                    float usage_boost, float* gate_probs, float* sim,
                    float* blend, float* importance, int32_t* head_idx,
                    float* head_score, float* stats_partial, float* ema_partial,
                    void* stream);

/* pfa_router_topk with its inputs built inside the router's workgroups
 * instead of by pfa_router_prepare (the same arithmetic, thread map and
 * reduction order, so the same bits): w_router (G, C) and the buffers
 * protos (G, C) (NULL: no prototype prior), confidence and usage (G)
 * (NULL: unused) as they are.  One launch fewer at the head of the router
 * chain (aspa.py:636-663 + 628-690).  Supported when
 * pfa_router_raw_supported(...) returns 1 and G <= 16: bf16 x, weights and
 * buffers, C a multiple of 128 up to 768 (G <= 8) or 512; otherwise
 * PFA_E_UNSUPPORTED.
 * pfa_router_topk_raw_ws serves every shape pfa_router_raw_supported
 * accepts, G up to 64: with G <= 16 it is pfa_router_topk_raw (the
 * workspace unused); with 17-64 gates it runs the 16-gate MFMA tables once
 * per block of 16 gates, writing each token's logits, prototype dots and
 * sum of squares to the workspace ((2G + 1) * n_tok f32, 16-byte aligned:
 * pfa_router_raw_workspace_size), then the same epilogue and prototype EMA
 * statistics in a second launch.  Same outputs as pfa_router_topk (the
 * prototype dots in another f32 summation order). */
int pfa_router_raw_supported(int x_dtype, int w_dtype, int buf_dtype, int G,
                             int C, int use_proto);
int pfa_router_topk_raw(const void* x, int x_dtype, int64_t n_tok, int C,
                        int G, const void* w_router, int w_dtype,
                        const void* protos, const void* confidence,
                        const void* usage, int buf_dtype,
                        const int32_t* gate_to_head, int H, int topk,
                        float proto_temp, float proto_threshold,
                        float proto_blend, float usage_boost,
                        float* gate_probs, float* sim, float* blend,
                        float* importance, int32_t* head_idx,
                        float* head_score, float* stats_partial,
                        float* ema_partial, void* stream);
int pfa_router_raw_workspace_size(int64_t n_tok, int G, size_t* bytes);
int pfa_router_topk_raw_ws(const void* x, int x_dtype, int64_t n_tok, int C,
                           int G, const void* w_router, int w_dtype,
                           const void* protos, const void* confidence,
                           const void* usage, int buf_dtype,
                           const int32_t* gate_to_head, int H, int topk,
                           float proto_temp, float proto_threshold,
                           float proto_blend, float usage_boost,
                           float* gate_probs, float* sim, float* blend,
                           float* importance, int32_t* head_idx,
                           float* head_score, float* stats_partial,
                           float* ema_partial, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ====================================================================
 * Prototype EMA statistics (aspa.py:692-718): per slice of tokens the
 * partial sums  sum_t gate[t,g]*x[t,c]  (columns 0..C-1) and
 * sum_t gate[t,g]  (column C), laid out (n_parts, G, C+1) f32, then summed
 * in a fixed order into (G, C+1).  Replaces the (G,BT)@(BT,C) product of
 * aspa.py:703-707 without materialising x in f32.  The reduction works in
 * place: `partial` is scratch and holds no useful values afterwards.
 * ==================================================================== */
int pfa_proto_partial_count(int64_t n_tok, int* n_parts);
int pfa_proto_accumulate(const void* x, int x_dtype, int64_t n_tok, int C,
                         int G, const float* gate_probs, float* partial,
                         int n_parts, void* stream);
int pfa_proto_partial_reduce(float* partial, int n_parts, int G, int C,
                             float* out, void* stream);

/* EMA step of aspa.py:700-716 from the reduced (G, C+1) sums: for gates with
 * count > 1e-6, protos = decay*protos + (1-decay)*mean; usage = decay*usage
 * (+ (1-decay)*count); confidence = decay*confidence (+ (1-decay)); every
 * op rounded to the buffers' dtype (PFA_F32 / PFA_BF16 / PFA_F16). */
int pfa_proto_ema_update(const float* sums, int G, int C, float decay,
                         void* protos, void* usage, void* confidence,
                         int dtype, void* stream);

/* ====================================================================
 * Token top-k: per batch row keep the `need` highest importance tokens
 * (ties -> lowest index), need = clamp(max(keep_count, #(imp >= threshold),
 * guard), 1, T); the first `guard` tokens are always kept.
 * Replaces AdaptiveSparseAttention._select_active_tokens
 * (aspa.py:790-842).  importance (B, T) f32 -> mask (B, T) uint8.
 * A radix select over the whole GPU (about 5 launches); workspace from
 * pfa_token_topk_workspace_size (about 4*B*T bytes + 10 KB per row).
 * ==================================================================== */
int pfa_token_topk_workspace_size(int B, int64_t T, size_t* bytes);
int pfa_token_topk(const float* importance, int B, int64_t T, int64_t keep_count,
                   int guard, float threshold, uint8_t* mask_out,
                   void* workspace, size_t ws_bytes, void* stream);

/* ====================================================================
 * Row packing.  Builds the (B*H, T) activity mask from the head top-k
 * indices and an optional token mask, compacts active (batch, head) pairs
 * and packs active (head, token) rows in row-major order (ascending token
 * within a head).
 * Replaces the mask build (aspa.py:1593-1606), active-head compaction
 * (aspa.py:1704-1726) and _pack_active_rows
 * (src/proteus_attention/kernels/sparse_attn.py:924-947).
 *
 *   head_idx    (B*T, topk) int32 (router output)
 *   token_mask  (B, T) uint8 or NULL
 *   mask_out    (B*H, T) uint8, required
 *   active_heads_out (B*H) int32  : compact id -> b*H+h (first P valid)
 *   row_offsets_out  (B*H + 1) int32 : exclusive scan over active heads
 *   token_idx_out    (B*H*T) int32 capacity : token of each packed row
 *   row_head_out     (B*H*T) int32 capacity : compact head of each row
 *   row_of_out       (B*H, T) int32 or NULL : packed row of (b*H+h, t), -1
 *                    when inactive (used by the residue-class anchor pass)
 *   summary_out (4) int32 : {P, N, max_rows, 0}
 * The workspace holds per-(head, block) counts.
 * ==================================================================== */
int pfa_pack_workspace_size(int B, int H, int64_t T, size_t* bytes);
int pfa_pack_rows(const int32_t* head_idx, int topk, const uint8_t* token_mask,
                  int B, int H, int64_t T, uint8_t* mask_out,
                  int32_t* active_heads_out, int32_t* row_offsets_out,
                  int32_t* token_idx_out, int32_t* row_head_out,
                  int32_t* row_of_out, int32_t* summary_out, void* workspace,
                  size_t ws_bytes, void* stream);

/* pfa_pack_rows without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as pfa_pack_rows; the per-(head, block) counts live in a static
 * device array of PFA_PACK_STATIC_SCRATCH_BYTES per GPU instead of a
 * workspace, so B*H*ceil(T/1024) is limited to about 2^18 (PFA_E_INVALID
 * beyond that).  It calls no allocator.  The array is looked up on the first
 * call on each device, which must then be the current device.  All calls on
 * one GPU share that array: calls that overlap on one GPU (two streams, two
 * threads) race and must be serialised by the caller. */
#define PFA_PACK_STATIC_SCRATCH_BYTES ((size_t)1 << 20)
int pfa_pack_rows_static(const int32_t* head_idx, int topk, const uint8_t* token_mask,
                         int B, int H, int64_t T, uint8_t* mask_out,
                         int32_t* active_heads_out, int32_t* row_offsets_out,
                         int32_t* token_idx_out, int32_t* row_head_out,
                         int32_t* row_of_out, int32_t* summary_out, void* stream);

/* Same packing from an arbitrary (P, T) uint8 mask (the operator-level
 * entry point aspa_sparse_attention packs its own active_mask). Heads are
 * NOT compacted: compact id == mask row. */
int pfa_pack_mask(const uint8_t* mask, int P, int64_t T, int32_t* row_offsets_out,
                  int32_t* token_idx_out, int32_t* row_head_out,
                  int32_t* summary_out, void* workspace, size_t ws_bytes,
                  void* stream);

/* ====================================================================
 * Prototype candidates: for every token t of every batch row b, the
 * indices of the min(t+1, K) largest proto_scores[b, 0..t] (ties -> lowest
 * index).  Replaces the (rows, T) masked topk of
 * _shortlist_prepare_proto_candidates (sparse_attn.py:260-300) by a
 * superblock scan plus a rank-based parallel resolution of each 64-token
 * block.  1 <= K <= 2048.
 *
 * pfa_proto_prefix_blocks writes the compact form:
 *   blocks_out (B, ceil(T/64), K) int32: row j = the set of token 64j-1
 *     (the prefix before block j), best score first, padded with INT32_MAX;
 *   evict_out (B, T) int32: the first token at which position p is no
 *     longer in the set (p if it never enters, INT32_MAX if it stays), so
 *     that p is in the set of token t exactly when p <= t < evict[p], and
 *     set(t) = { p in blocks[t/64] U {64*(t/64) .. t} : evict[p] > t }.
 * pfa_proto_prefix_topk writes every token's set, sorted by index, into
 * sets_out (B, T, K) int32 (entries past min(t+1, K) hold t); evict_out is
 * optional there.  Both take the workspace sized by
 * pfa_proto_prefix_workspace_size.
 * ==================================================================== */
int pfa_proto_prefix_workspace_size(int B, int64_t T, int K, size_t* bytes);
int pfa_proto_prefix_blocks(const float* proto_scores, int B, int64_t T,
                            int64_t score_stride, int K, int32_t* blocks_out,
                            int32_t* evict_out, void* workspace,
                            size_t ws_bytes, void* stream);
int pfa_proto_prefix_topk(const float* proto_scores, int B, int64_t T,
                          int64_t score_stride, int K, int32_t* sets_out,
                          int32_t* evict_out, void* workspace, size_t ws_bytes,
                          void* stream);

/* ====================================================================
 * Shortlist candidate builder (packed rows).
 * Replaces build_packed_shortlist_candidates (sparse_attn.py:457-596) and
 * build_shortlist_candidates (sparse_attn.py:376-454): per row the union of
 * the local window, strided anchors, prototype top-k and optional extra
 * candidates, clamped to [0, min(row, seq_len-1)], the row itself appended,
 * sorted ascending, de-duplicated, truncated to the smallest L values and
 * padded with the row index; lengths = max(count, 1).
 *
 *   rows (N) int32 (tokens, each in [0, seq_len)), row_batch (N) int32 or
 *     NULL (batch 0)
 *   n_rows_dev: NULL, or a device int32 holding the row count: then only
 *     rows [0, min(N, *n_rows_dev)) are built and N is a capacity (the
 *     packing summary's N, read on the device by a caller that does not
 *     wait for it)
 *   local_w: effective window min(linear_window, L, local_cap), 0 = no
 *     local piece;  anchor_slots: min(anchor_cap, L, max(1, seq_len)),
 *     0 = no anchors (sparse_attn.py:413-429)
 *   proto_sets (B, proto_len, proto_k) int32 from pfa_proto_prefix_topk, or
 *     NULL; row t uses set min(t, proto_len-1)
 *   extra (N, extra_width) int32 + extra_len (N) int32, or NULL
 *   cand_out (N, L) int32 or int64 (cand_is_i64), len_out (N) int32/int64
 * ==================================================================== */
int pfa_shortlist_build(const int32_t* rows, const int32_t* row_batch, int64_t N,
                        const int32_t* n_rows_dev, int64_t seq_len, int L, int local_w, int anchor_stride,
                        int anchor_slots, const int32_t* proto_sets,
                        int proto_k, int64_t proto_len, const int32_t* extra,
                        const int32_t* extra_len, int extra_width,
                        void* cand_out, int cand_is_i64, void* len_out,
                        int len_is_i64, void* stream);

/* ====================================================================
 * Packed sparse attention (online softmax), fused gather and scatter.
 * Replaces the Triton _shortlist_attention_kernel (sparse_attn.py:597-921)
 * and the PyTorch fallback _fallback_sparse_attention
 * (sparse_attn.py:950-1046) behind aspa_sparse_attention
 * (sparse_attn.py:1373-1646).
 *
 * Tensors q/k/v/out are addressed as [b][h][t][d] through element strides
 * so that (B*H, T, D) head-major buffers and the (B, T, 3, H, D) output of
 * the QKV projection are both read in place:
 *   addr(bh, t, d) = base + (bh / H) * s_b + (bh % H) * s_h + t * s_t + d
 * Row r (packed) belongs to compact head row_head[r] whose global index is
 * head_map[row_head[r]] (head_map NULL: identity) and queries token
 * token_idx[r].  n_rows_dev (NULL, or a device int32 row count) bounds the
 * rows to [0, min(N, *n_rows_dev)), as for pfa_shortlist_build.
 *
 * Key set of row r:
 *   cand != NULL : cand[r, 0 .. len[r])                (candidate branch)
 *   cand == NULL, mask == NULL : keys 0 .. token_idx[r] (implicit causal)
 *   cand == NULL, mask != NULL : keys 0 .. head_max_token[head] with the
 *       additive (T, T) mask row token_idx[r] added (mask_dtype).
 * With a mask in the candidate branch, mask[token, cand] is added.
 * Scores are scaled by `scale`; for PFA_I8 inputs element values are
 * multiplied by the per-global-head scales q_scale/k_scale/v_scale.
 * A row with no finite score produces NaN, as softmax over all -inf does.
 * ==================================================================== */
typedef struct pfa_tensor4 {
  void* ptr;
  int64_t s_b, s_h, s_t; /* element strides; d is contiguous */
} pfa_tensor4;

int pfa_sparse_attn_fwd(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v,
                        int in_dtype, pfa_tensor4 out, int out_dtype, int H,
                        int64_t T, int D, const int32_t* token_idx,
                        const int32_t* row_head, const int32_t* head_map,
                        int64_t N, const int32_t* n_rows_dev,
                        const int32_t* cand, int64_t cand_stride,
                        const int32_t* cand_len, const void* mask,
                        int mask_dtype, const int32_t* head_max_token,
                        float scale, const float* q_scale, const float* k_scale,
                        const float* v_scale, void* stream);

/* ====================================================================
 * Shortlist attention without materialised candidates (bf16, D = 16, 32,
 * 64 or 128; q_rope_cos / q_rope_sin need D <= 64 and the fused variant's
 * fuse bits D = 64).
 * Same result as pfa_shortlist_build followed by pfa_sparse_attn_fwd for the
 * module's packed rows when no row is truncated (local_w + anchors below the
 * window + proto_k + 1 <= L, checked by the caller): each row attends to its
 * window [t - min(t+1, local_w) + 1, t], its strided anchors below the window
 * and its prototype prefix set below the window (proto_blocks (B,
 * ceil(T/64), proto_k) and proto_evict (B, T) from pfa_proto_prefix_blocks
 * over the T tokens; proto_k <= 1024), with the zero anchor, all on bf16
 * MFMA.
 * Replaces sparse_attn.py:457-596 + 597-921 on the module path
 * (aspa.py:1269-1302).
 *   row_of (B*H, T) from pfa_pack_rows; summary from pfa_pack_rows ({P,...});
 *   head_map (P_cap) compact -> b*H+h; partials (N, pfa_shortlist_attn_part_
 *   floats_for(D)) f32 scratch for the anchor pass (pfa_shortlist_attn_part_
 *   floats() is the width for D <= 64); lengths (N) int32 or NULL
 *   receives each row's candidate count (the builder's lengths).
 *   q_rope_cos / q_rope_sin: NULL, or the bf16 (T, D) RoPE tables (D <= 64) of
 *   pfa_rope_qk_inplace; q rows are then rotated as they are loaded (the
 *   caller rotated only k, with pfa_rope_k_inplace), giving the same q bits
 *   as rotating the q tensor first.
 *   passes: 3 runs both launches; 1 only the anchor pass (writes partials),
 *   2 only the main pass (reads them).  Splitting lets the anchor pass run
 *   on another stream while the prototype tables are built; the caller
 *   orders pass 1 before pass 2 and keeps partials alive between them.
 *   q, k, v, out: 16-byte aligned with strides multiple of 8 elements; the
 *   k and v token strides positive and below 2^31 (PFA_E_INVALID otherwise).
 *   Results are deterministic: the same inputs give the same bits.
 *   q_scale / k_scale / v_scale: NULL, or per global head (b*H + h) f32
 *   scales of the per-head int8 quantisation (aspa.py:1258-1267,
 *   1312-1363; pfa_quantize_heads_int8 with bf16 output): q, k, v then
 *   hold the int8 values as exact bf16 integers, the scores are
 *   scale*q_scale*k_scale*(q8.k8) (exact integer dots on MFMA) and the
 *   outputs v_scale*(P.v8)/l -- the dequantisation of sparse_attn.py:
 *   1538-1541 applied inside the tile.  All three or none.
 * ==================================================================== */
int pfa_shortlist_attn_part_floats(void);
int pfa_shortlist_attn_part_floats_for(int head_dim);
int pfa_shortlist_attn_fwd(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v,
                           pfa_tensor4 out, int dtype, int H, int64_t T, int D,
                           const int32_t* token_idx, const int32_t* row_head,
                           const int32_t* head_map, int64_t N, int P_cap,
                           const int32_t* summary, const int32_t* row_of,
                           int local_w, int anchor_stride, int anchor_slots,
                           const int32_t* proto_blocks, int proto_k,
                           const int32_t* proto_evict, float scale,
                           float* partials, int32_t* lengths,
                           const void* q_rope_cos, const void* q_rope_sin,
                           const float* q_scale, const float* k_scale,
                           const float* v_scale, int passes, void* stream);

/* pfa_shortlist_attn_fwd (without the int8 scales) whose anchor pass also
 * does work the module path otherwise launches separately before it:
 *   PFA_FUSE_K_ROPE: rotates k in place, row by row, for the active heads
 *     (head_map[0..P)) with the q_rope tables -- the bits of
 *     pfa_rope_k_inplace on those heads (aspa.py:606-618, 1648-1649 for
 *     k); q is rotated on load as with pfa_shortlist_attn_fwd.  k of the
 *     other heads is left as it is (no kernel reads it).
 *   PFA_FUSE_ZERO: writes zeros to out[b][h][t][:] for every (head, token)
 *     pair without a packed row (row_of == -1, and every token of the
 *     heads missing from head_map[0..P)), so out needs no zero fill first
 *     (the x.new_zeros of aspa.py:1707 that the index_copy_ of
 *     aspa.py:1762-1806 fills).
 * Both ride on the anchor pass: anchors on and passes 1 or 3; head_map
 * ascending (as pfa_pack_rows writes it) with P_cap = B*H; N may be 0 (the
 * zero fill still runs).  The main pass then reads the rotated k.
 * Replaces pfa_rope_k_inplace + pfa_zero_fill (aspa.py:1648-1649, 1707) on
 * the structured module path. */
#define PFA_FUSE_K_ROPE 1
#define PFA_FUSE_ZERO 2
int pfa_shortlist_attn_fwd_fused(pfa_tensor4 q, pfa_tensor4 k, pfa_tensor4 v,
                                 pfa_tensor4 out, int dtype, int H, int64_t T,
                                 int D, const int32_t* token_idx,
                                 const int32_t* row_head,
                                 const int32_t* head_map, int64_t N, int P_cap,
                                 const int32_t* summary, const int32_t* row_of,
                                 int local_w, int anchor_stride,
                                 int anchor_slots, const int32_t* proto_blocks,
                                 int proto_k, const int32_t* proto_evict,
                                 float scale, float* partials, int32_t* lengths,
                                 const void* q_rope_cos, const void* q_rope_sin,
                                 int passes, int fuse, void* stream);

/* ====================================================================
 * Per-head symmetric int8 quantisation of the active heads of q, k or v.
 * Replaces AdaptiveSparseAttention._quantize_per_head_int8
 * (aspa.py:1312-1363) and its call sites (aspa.py:1258-1267): per compact
 * head p < P (P = summary[0], or P_cap when summary is NULL) of global head
 * bh = head_map[p] (identity when NULL), over its T x D elements of x
 * ([b][h][t][d] through pfa_tensor4 strides, dtype PFA_F32/BF16/F16):
 *   base  = max |x|                                      mode 0 ("max")
 *         = torch.quantile(|x|, percentile) (linear interpolation; the
 *           absmax when that is 0, or when percentile == 0)  mode 1
 *         = as mode 1, then ema[p] = decay*e + (1-decay)*base with e =
 *           ema[p] (ema_valid) or the absmax; base = ema[p]   mode 2
 *   scales[bh] = max(base / 127, 1e-6)
 *   dst[bh][t][d] = clamp(round_half_even(x / scale), -127, 127)
 * each step an f32 operation rounded as the reference's tensor ops round.
 * dst_dtype PFA_I8 writes int8; PFA_BF16 writes the same integers as bf16
 * (exact), and dst may then be x itself (in place) -- the input of
 * pfa_shortlist_attn_fwd's int8 mode.  ema: (P) f32, read and written in
 * mode 2 only.  The workspace is sized by pfa_quantize_heads_workspace_size
 * for the same P_cap, T, D and mode.
 * Size limit of the reference (modes 1 and 2): the reference takes
 * torch.quantile over the whole (P, T*D) tensor at once, which raises
 * "quantile() input tensor is too large" above 2^24 elements (P*T*D >
 * 16,777,216, e.g. 8 active heads x T = 65,536 x D = 64).  This entry point
 * returns values there; they have no reference counterpart, and the oracle
 * and golden cases stay below that size.
 * ==================================================================== */
int pfa_quantize_heads_workspace_size(int P_cap, int64_t T, int D, int mode,
                                      size_t* bytes);
int pfa_quantize_heads_int8(pfa_tensor4 x, int dtype, int H, int64_t T, int D,
                            const int32_t* head_map, int P_cap,
                            const int32_t* summary, int mode, float percentile,
                            double ema_decay, float* ema, int ema_valid,
                            pfa_tensor4 dst, int dst_dtype, float* scales,
                            void* workspace, size_t ws_bytes, void* stream);

/* Per compact head, the largest token among its packed rows (needed by the
 * explicit-mask branch: sparse_attn.py:1010-1015). */
int pfa_head_max_token(const int32_t* token_idx, const int32_t* row_offsets,
                       int P, int32_t* out, void* stream);

/* ====================================================================
 * RoPE on the q and k thirds of a (B, T, 3C) QKV projection, in place.
 * Replaces _apply_rope_embedding (aspa.py:606-618): interleaved (even,
 * odd) pairs rotated with cos/sin tables (T, D) in the same dtype, each
 * product and the sum rounded to that dtype as the reference's
 * elementwise ops do.
 * ==================================================================== */
int pfa_rope_qk_inplace(void* qkv, int dtype, int B, int64_t T, int H, int D,
                        const void* cos_tab, const void* sin_tab, void* stream);

/* The k third only (same arithmetic), for callers that rotate q elsewhere
 * (pfa_shortlist_attn_fwd with q_rope_cos / q_rope_sin). */
int pfa_rope_k_inplace(void* qkv, int dtype, int B, int64_t T, int H, int D,
                       const void* cos_tab, const void* sin_tab, void* stream);

/* pfa_rope_k_inplace that also writes zeros to zero_out, the (B, T, H*D)
 * attention output of the same dtype (16-byte aligned), in the same pass:
 * the module's zero-initialised output (aspa.py:1707, the tensor the
 * attention fills only at active (head, token) rows) without a separate
 * fill over it.  The RoPE bits are those of pfa_rope_k_inplace; shapes
 * other than D = 64 rotate first and then fill. */
int pfa_rope_k_zero_inplace(void* qkv, int dtype, int B, int64_t T, int H,
                            int D, const void* cos_tab, const void* sin_tab,
                            void* zero_out, void* stream);

/* ====================================================================
 * Fill: write zeros into `bytes` of device memory with a vector-store
 * kernel (usable where memset nodes are not wanted).
 * ==================================================================== */
int pfa_zero_fill(void* ptr, size_t bytes, void* stream);

/* ====================================================================
 * Chunk salience top-k.  Replaces _select_top_tokens + _nucleus_select
 * (src/proteus_attention/tools/chunked_shortlist.py:140-208): scores
 * (n) f32 with positions whose keep_mask byte is 0 (keep_mask may be NULL)
 * set to -inf; non-finite scores rank as -1e9; the first
 * keep = min(budget, n) positions in the order (score desc, position asc)
 * are taken, or with top_p < 1 the nucleus count
 * #(cumulative softmax mass < top_p) + 1 (clamped to [1, min(budget, n)]);
 * with drop_nonfinite, entries whose (masked) score is not finite are then
 * dropped (the filter of _select_top_tokens).  Writes, in
 * selection order, values_out (budget) f32 and indices_out (budget) int64
 * (position + index_offset), and count_out (1) int32 (0 when no score is
 * finite: the reference's "None").  Ties: lowest position first.
 * ==================================================================== */
int pfa_chunk_topk_workspace_size(int64_t n, int budget, size_t* bytes);
int pfa_chunk_topk(const float* scores, const uint8_t* keep_mask, int64_t n,
                   int budget, float top_p, int64_t index_offset,
                   int drop_nonfinite, float* values_out, int64_t* indices_out,
                   int32_t* count_out, void* workspace, size_t ws_bytes,
                   void* stream);

/* ====================================================================
 * Global shortlist merge.  Replaces _finalise_indices
 * (chunked_shortlist.py:211-254): the n candidates (scores f32, indices
 * int64 in [-2^31, 2^31)) ordered by score descending (ties: lower
 * candidate position first), one survivor per index -- its last entry in
 * that order -- then the first max_tokens survivors, returned sorted by
 * index: keep_indices_out (max_tokens) int64, keep_scores_out (max_tokens)
 * f32, count_out (1) int32 = number written.
 * ==================================================================== */
int pfa_shortlist_finalise_workspace_size(int64_t n, size_t* bytes);
int pfa_shortlist_finalise(const float* scores, const int64_t* indices, int64_t n,
                           int64_t max_tokens, int64_t* keep_indices_out,
                           float* keep_scores_out, int32_t* count_out,
                           void* workspace, size_t ws_bytes, void* stream);

/* ====================================================================
 * Per-(head, row) symmetric int8 quantisation of the shortlisted K or V
 * rows of the chunked pipeline's final pass.  The per-head scheme of
 * AdaptiveSparseAttention._quantize_per_head_int8 (aspa.py:1312-1363,
 * "max" mode) applied to each (head, row) of D elements:
 * scale = max(absmax / 127, 1e-6), q = clamp(round_half_even(x / scale),
 * -127, 127).  src row r, head h at src + r*row_stride + h*D (dtype
 * PFA_F32 / PFA_BF16 / PFA_F16); dst (H, n_rows, D) int8, scales
 * (H, n_rows) f32.
 * ==================================================================== */
int pfa_quantize_rows_int8(const void* src, int dtype, int64_t n_rows,
                           int64_t row_stride, int H, int D, int8_t* dst,
                           float* scales, void* stream);

/* ====================================================================
 * RoPE in place on arbitrary rows: H heads of D elements at
 * x + r*row_stride, rotated with table row positions[r] (positions NULL:
 * pos_offset + r).  Same arithmetic and rounding as pfa_rope_qk_inplace
 * (_apply_rope_embedding, aspa.py:606-618); used for query slices of a
 * streamed chunk and for shortlisted keys at their original positions.
 * ==================================================================== */
int pfa_rope_rows_inplace(void* x, int dtype, int64_t n_rows, int64_t row_stride,
                          int H, int D, const void* cos_tab, const void* sin_tab,
                          const int32_t* positions, int64_t pos_offset,
                          void* stream);

/* ====================================================================
 * All-query attention over an int8 shortlist (bf16, D = 64): the chunked
 * pipeline's final pass in its all-query form.  The reference attends the
 * reduced sequence to itself (chunked_shortlist.py:710-739); this entry
 * point lets every one of T query tokens attend to the S shortlisted keys,
 * causal by original position when `causal` (key j visible to query t iff
 * key_pos[j] <= t; key_pos ascending).  K/V are int8 (H, S, D) with
 * per-(head, row) scales (H, S) from pfa_quantize_rows_int8 (k8/v8
 * 16-byte aligned), dequantised once per call to bf16 (x8 * scale, round
 * to nearest even) into the workspace, which therefore holds 4*H*S*D
 * bytes plus the query tiles' key ranges.  q/out are bf16 [h][t][d]
 * through pfa_tensor4 strides (s_b unused: one sequence).  A query with
 * no visible key gets a zero row.  S >= 1.
 * ==================================================================== */
int pfa_int8_kv_attn_workspace_size(int64_t T, int H, int S, size_t* bytes);
int pfa_int8_kv_attn_fwd(pfa_tensor4 q, pfa_tensor4 out, int64_t T, int H, int D,
                         const int8_t* k8, const int8_t* v8, const float* k_scale,
                         const float* v_scale, const int32_t* key_pos, int S,
                         int causal, float scale, void* workspace,
                         size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PFA_HIP_H */
