/*
 * sps_attn.h - C ABI of the MI355X (gfx950) SPS attention hot path.
 *
 * One shared library (libsps_attn.so) exports the three kernel families of the SPS Transformer's
 * attention path. All entry points are stateless, take plain device pointers, element strides and
 * sizes, enqueue asynchronously on the caller's HIP stream (passed as void*, a hipStream_t), never
 * synchronise the host and never allocate device memory: scratch space is a caller-provided
 * workspace whose size the *_workspace_bytes functions report. They return SPS_OK or an error
 * code; sps_last_error() returns the message of the calling thread's last failure.
 *
 * Tensor conventions. A [B, H, N, D] tensor is described by its base pointer and the element
 * strides {b, h, n}; the D axis must be contiguous, the base 16-byte aligned and every stride a
 * multiple of 8 elements (16 bytes). Document ids are a [B, N] int32 or int64 array with unit
 * stride along N. Positions of the SPS families index the interleaved input/<predict> sequence
 * (token t owns positions 2t and 2t+1), so N must be even there.
 *
 * Reference interfaces replaced (lil-lab/sps, paths under src/modeling/models/):
 *   sps_attn_fwd / sps_attn_bwd   <- _sps_sliding_attention.forward/backward
 *                                    (attention/triton_sps_flash_attention.py:491-722),
 *                                    _reverse_sps_sliding_attention.forward/backward
 *                                    (attention/triton_reverse_sps_flash_attention.py:602-824),
 *                                    _full_attention.forward/backward
 *                                    (attention/triton_full_flash_attention.py:463-676)
 *   sps_decode                    <- triton_segmented_q1_attention (utils/decode_attention.py:393-480),
 *                                    triton_segmented_q2_attention (utils/decode_attention.py:483-594)
 *   sps_kv_update                 <- fused_sps_kv_update (utils/decode_attention_fast.py:139-221)
 *   sps_decode_kv_update          <- the decode step's attention over the caches followed by
 *                                    fused_sps_kv_update (reverse_sps/inference.py:169-238, 322-362)
 *   sps_rope_qkv                  <- apply_rotary_emb (model.py:201-230) + the transposes and casts
 *                                    before the attention call (sps/core.py:45-55)
 *   sps_prefill_to_decode         <- _materialize_prefill_layer_state
 *                                    (reverse_sps/inference.py:568-613)
 *   sps_document_ids              <- generate_left_padded_document_idx (model.py:70-99) + the
 *                                    repeat_interleave(2) of reverse_sps/core.py:226
 *   sps_attn_mask                 <- the mask block of _attn_fwd_inner_sps
 *                                    (attention/triton_sps_flash_attention.py:70-111); a
 *                                    verification entry point that materialises the mask the
 *                                    kernels evaluate.
 */
#ifndef SPS_ATTN_H
#define SPS_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define SPS_OK 0
#define SPS_E_INVALID 1     /* malformed argument (null pointer, bad shape, misaligned stride) */
#define SPS_E_UNSUPPORTED 2 /* well-formed but outside this build (head dim, dtype) */
#define SPS_E_WORKSPACE 3   /* workspace smaller than *_workspace_bytes reports */
#define SPS_E_HIP 4         /* HIP runtime error while enqueueing */

/* Element types. */
#define SPS_DTYPE_BF16 0
#define SPS_DTYPE_F16 1
#define SPS_DTYPE_F32 2
#define SPS_DTYPE_I32 3
#define SPS_DTYPE_I64 4
#define SPS_DTYPE_U8 5 /* bool / uint8 flags (nonzero = true) */

/* Attention families (mask semantics). */
#define SPS_FAMILY_FULL 0        /* causal + document mask (full_attention) */
#define SPS_FAMILY_SPS 1         /* persistent keys at even positions (sps_sliding_attention) */
#define SPS_FAMILY_REVERSE_SPS 2 /* persistent keys at odd positions (reverse_sps_sliding_attention,
                                    also used by the delayed-state model) */

/* Version string of the library. */
const char* sps_version(void);

/* Copies the calling thread's last error message into buf (NUL-terminated, truncated to len)
 * and returns the full message length. */
int sps_last_error(char* buf, size_t len);

/* Workspace needed by sps_attn_fwd (backward = 0), sps_attn_bwd (backward = 1) or
 * sps_attn_mask (backward = 0). */
size_t sps_attn_workspace_bytes(int family, int B, int H, int N, int has_docs, int backward);

/*
 * Forward attention. q, k, v, o: [B, H, N, D] of dtype (bf16 or f16), D in {16, 32, 64, 128, 256}.
 * lse: [B, H, N] fp32 contiguous, receives the log2-domain log-sum-exp of the scaled scores
 * (m + log2 l), consumed by sps_attn_bwd. docs may be NULL (no document mask).
 * window: temporary-key window in tokens (SPS families). has_pkw/pkw: optional persistent-key
 * window (the reference's persistent_key_window; has_pkw = 0 means None). sm_scale may be any finite
 * value (zero and negative ones too; NaN or infinity: SPS_E_INVALID): the kernels form
 * S * sm_scale * log2(e) in fp32 from the unscaled 16-bit inputs, as the reference scales its fp32
 * scores. fp32 inputs are not taken (SPS_E_UNSUPPORTED): the path runs on bf16/f16 MFMA only.
 */
int sps_attn_fwd(int family, int B, int H, int N, int D, int dtype,
                 const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides,
                 const void* v, const int64_t* v_strides,
                 void* o, const int64_t* o_strides,
                 float* lse,
                 const void* docs, int docs_dtype, int64_t docs_stride_b,
                 float sm_scale, int window, int has_pkw, int pkw,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward attention: given dO, writes dq, dk, dv (same dtype as q). o and lse are the forward
 * outputs. The workspace also holds, per query, -lse and -Delta (Delta = rowsum(o * dO)).
 */
int sps_attn_bwd(int family, int B, int H, int N, int D, int dtype,
                 const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides,
                 const void* v, const int64_t* v_strides,
                 const void* o, const int64_t* o_strides,
                 const void* dout, const int64_t* dout_strides,
                 const float* lse,
                 void* dq, const int64_t* dq_strides,
                 void* dk, const int64_t* dk_strides,
                 void* dv, const int64_t* dv_strides,
                 const void* docs, int docs_dtype, int64_t docs_stride_b,
                 float sm_scale, int window, int has_pkw, int pkw,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Passes of the backward (sps_attn_bwd runs SPS_BWD_DQ, then SPS_BWD_DKDV, on one stream). */
#define SPS_BWD_DQ 1   /* Delta = rowsum(o * dO), and -lse, -Delta per query into the workspace, and dq
                          (reference: _attn_bwd_preprocess + _sps_bwd_dq_kernel,
                          triton_reverse_sps_flash_attention.py:334-348, triton_sps_flash_attention.py:385-488) */
#define SPS_BWD_DKDV 2 /* dk, dv from the -lse / -Delta and document ranges the SPS_BWD_DQ pass left in the workspace
                          (reference: _sps_bwd_dkdv_kernel, triton_sps_flash_attention.py:272-382) */

#define SPS_BWD_REUSE_LAYOUT 4 /* with SPS_BWD_DQ: the workspace already holds the document row layout
                                  that sps_attn_fwd wrote for the same docs, family, N, window and pkw
                                  (the forward was given a workspace of the backward's size), so the
                                  pass skips recomputing it */

/*
 * Passes of sps_attn_bwd, same arguments plus `pass`: SPS_BWD_DQ, SPS_BWD_DKDV or both, optionally
 * with SPS_BWD_REUSE_LAYOUT. An SPS_BWD_DKDV pass alone must follow an SPS_BWD_DQ pass with the same
 * workspace on the same stream; arguments a pass does not touch (dk, dv for SPS_BWD_DQ; dq for
 * SPS_BWD_DKDV) are still validated. Lets a caller time or schedule the two kernels separately, as the
 * reference launches them separately (triton_sps_flash_attention.py:651-707), and reuse the forward's
 * document layout.
 */
int sps_attn_bwd_pass(int pass, int family, int B, int H, int N, int D, int dtype,
                      const void* q, const int64_t* q_strides,
                      const void* k, const int64_t* k_strides,
                      const void* v, const int64_t* v_strides,
                      const void* o, const int64_t* o_strides,
                      const void* dout, const int64_t* dout_strides,
                      const float* lse,
                      void* dq, const int64_t* dq_strides,
                      void* dk, const int64_t* dk_strides,
                      void* dv, const int64_t* dv_strides,
                      const void* docs, int docs_dtype, int64_t docs_stride_b,
                      float sm_scale, int window, int has_pkw, int pkw,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * Writes into mask ([B, N, N] uint8, zero-filled by the caller) a 1 for every (query, key) pair
 * that the attention kernels treat as visible, following the block schedule of the
 * query-stationary kernels (schedule = 0: forward and dQ) or of the key-stationary dK/dV kernel
 * (schedule = 1). Used to prove the kernels' masks bit-exact against the reference predicate.
 */
int sps_attn_mask(int family, int B, int N,
                  const void* docs, int docs_dtype, int64_t docs_stride_b,
                  int window, int has_pkw, int pkw, int schedule, uint8_t* mask,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Workspace needed by sps_decode for the given segment scan lengths. */
size_t sps_decode_workspace_bytes(int B, int H, int D, int nq, int kv_dtype, int n_seg,
                                  const int64_t* seg_scan);

/*
 * Segmented decode attention, nq in {1, 2} queries per (batch, head).
 * q: [B, nq, H, D] of q_dtype (SPS_DTYPE_BF16, F16 or F32; values already in the attention dtype),
 * strides {b, slot, h}.
 * Segments (n_seg <= 3): K and V [B, H, storage, D] of kv_dtype (bf16, f16 or f32) with strides
 * {b, h, t}; live lengths seg_len[s] ([B] if seg_len_per_head[s] == 0, else [B, H]) of dtype
 * SPS_DTYPE_I32 or SPS_DTYPE_I64; key t of segment s is attended iff
 * t < min(max(len, 0), seg_scan[s]).
 * Extras (n_extra <= 2): [B, H, D] keys/values of extra_dtype sharing strides {b, h}; extra e is
 * attended by query slot j iff bit j of extra_query_mask[e] is set (q=1: 1; q=2: current input 3,
 * current <predict> 2). out: fp32 [B, nq, H, D], strides {b, slot, h}; 0 where nothing is attended.
 * D in {16, 32, 64, 128, 256}. Two launches: per-chunk partials into the workspace, then a merge.
 */
int sps_decode(int B, int H, int D, int nq,
               const void* q, int q_dtype, const int64_t* q_strides,
               int kv_dtype, int n_seg,
               const void* const* seg_k, const int64_t* seg_k_strides,
               const void* const* seg_v, const int64_t* seg_v_strides,
               const void* const* seg_len, const int* seg_len_dtype, const int* seg_len_per_head,
               const int64_t* seg_scan,
               int n_extra, const void* const* extra_k, const void* const* extra_v, int extra_dtype,
               const int64_t* extra_strides, const int* extra_query_mask,
               float sm_scale, float* out, const int64_t* out_strides,
               void* workspace, size_t workspace_bytes, void* stream);

/*
 * sps_decode without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The per-chunk partial records go to a scratch array of 16 MiB that the library holds
 * on each GPU it runs on (a file-scope device array, resolved per device on that device's first
 * call); the call allocates nothing. Returns SPS_E_UNSUPPORTED when the records would need more than
 * 16 MiB (sps_decode_workspace_bytes for the same arguments). Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (different streams, no ordering between them) race;
 * calls ordered on one stream are safe. The array keeps the last call's records, and no call reads
 * records it did not write. Arguments otherwise as sps_decode.
 */
int sps_decode_static(int B, int H, int D, int nq,
                      const void* q, int q_dtype, const int64_t* q_strides,
                      int kv_dtype, int n_seg,
                      const void* const* seg_k, const int64_t* seg_k_strides,
                      const void* const* seg_v, const int64_t* seg_v_strides,
                      const void* const* seg_len, const int* seg_len_dtype, const int* seg_len_per_head,
                      const int64_t* seg_scan,
                      int n_extra, const void* const* extra_k, const void* const* extra_v, int extra_dtype,
                      const int64_t* extra_strides, const int* extra_query_mask,
                      float sm_scale, float* out, const int64_t* out_strides, void* stream);

/*
 * Decode KV-cache update of one layer, one launch (replaces fused_sps_kv_update,
 * utils/decode_attention_fast.py:139-221; semantics of the un-fused path it replaces,
 * _update_normal_memory_unfused / _update_predict_memory_unfused, reverse_sps/inference.py:137-168
 * and 240-268). For every sequence b with active[b * active_stride] != 0:
 *   ring (window_tokens > 0): slot = ring_len[b] >= window_tokens ? ring_pos[b] : ring_len[b];
 *     ring K/V[b, h, slot, :] = k_window / v_window[b, h, :] for every head; then ring_len[b] += 1
 *     if the ring was not full, else ring_pos[b] = (ring_pos[b] + 1) % window_tokens.
 *   retained: if 0 <= ret_len[b, h] < ret_storage: retained K/V[b, h, ret_len[b, h], :] =
 *     k_retained / v_retained[b, h, :] and ret_len[b, h] += 1 (otherwise nothing is written).
 * Inactive sequences are untouched. Caches: [B, H, storage, D] of kv_dtype (bf16, f16, f32) with
 * element strides ring_strides = {k_b, k_h, k_t, v_b, v_h, v_t} (likewise ret_strides), D axis
 * contiguous. ring_len / ring_pos: [B] with strides ring_len_strides = {len_b, pos_b}; ret_len:
 * [B, H] with strides {b, h}; all of len_dtype (int32/int64). New K/V: [B, H, D] of new_dtype,
 * strides new_strides = {kw_b, kw_h, vw_b, vw_h, kr_b, kr_h, vr_b, vr_h}, converted to kv_dtype
 * with round-to-nearest-even. active: [B] of SPS_DTYPE_U8 (bool), I32 or I64. The ring pointers may
 * be null when window_tokens <= 0. window_tokens must not exceed ring_storage.
 */
int sps_kv_update(int B, int H, int D, int kv_dtype, void* ring_k, void* ring_v, const int64_t* ring_strides,
                  int ring_storage, int window_tokens, void* ring_len, void* ring_pos,
                  const int64_t* ring_len_strides, void* ret_k, void* ret_v, const int64_t* ret_strides,
                  int ret_storage, void* ret_len, const int64_t* ret_len_strides, int len_dtype, int new_dtype,
                  const void* k_window, const void* v_window, const void* k_retained, const void* v_retained,
                  const int64_t* new_strides, const void* active, int active_dtype, int64_t active_stride,
                  void* stream);

/* Workspace needed by sps_decode_kv_update: sps_decode's partial records plus a length snapshot. */
size_t sps_decode_kv_update_workspace_bytes(int B, int H, int D, int nq, int kv_dtype, int n_seg,
                                            const int64_t* seg_scan);

/*
 * One decode step of one layer: sps_decode, then sps_kv_update, as one entry point with the update
 * folded into the attention's launches (replaces the reference's decode step pair, the segmented
 * attention over the caches followed by fused_sps_kv_update: reverse_sps/inference.py:322-362 with
 * :169-238, utils/decode_attention_fast.py:139-221). The attention reads the caches as they were
 * before the update. Arguments: sps_decode's from B to out_strides, then sps_kv_update's from
 * ring_k to active_stride (the caches in kv_dtype, the decode's K/V dtype), then the workspace
 * (sps_decode_kv_update_workspace_bytes) and the stream. When the update copies new rows of the
 * cache dtype with 16-byte aligned rows and strides (and the segments hold at least one chunk), it
 * runs inside the attention's merge launch: the partial kernel snapshots the lengths, and the merge
 * writes the rows and advances the lengths from the snapshot; otherwise the update is a launch of
 * its own after the attention. Results are those of the two calls in that order.
 */
int sps_decode_kv_update(int B, int H, int D, int nq,
                         const void* q, int q_dtype, const int64_t* q_strides,
                         int kv_dtype, int n_seg,
                         const void* const* seg_k, const int64_t* seg_k_strides,
                         const void* const* seg_v, const int64_t* seg_v_strides,
                         const void* const* seg_len, const int* seg_len_dtype, const int* seg_len_per_head,
                         const int64_t* seg_scan,
                         int n_extra, const void* const* extra_k, const void* const* extra_v, int extra_dtype,
                         const int64_t* extra_strides, const int* extra_query_mask,
                         float sm_scale, float* out, const int64_t* out_strides,
                         void* ring_k, void* ring_v, const int64_t* ring_strides, int ring_storage,
                         int window_tokens, void* ring_len, void* ring_pos, const int64_t* ring_len_strides,
                         void* ret_k, void* ret_v, const int64_t* ret_strides, int ret_storage, void* ret_len,
                         const int64_t* ret_len_strides, int len_dtype, int new_dtype,
                         const void* k_window, const void* v_window, const void* k_retained,
                         const void* v_retained, const int64_t* new_strides,
                         const void* active, int active_dtype, int64_t active_stride,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Pre-attention rotary embedding and cast, one pass (replaces apply_rotary_emb, model.py:201-230,
 * and the transposes / .to(bfloat16) of the attention callers, sps/core.py:45-55,
 * reverse_sps/core.py:60-75). For every (b, n, h) row and pair i < D/2:
 *   out[2i]   = x[2i] * f.re - x[2i+1] * f.im,   out[2i+1] = x[2i] * f.im + x[2i+1] * f.re
 * in fp32 with f = freqs[b, n, i] (complex, stored as (re, im) float pairs; freqs_strides =
 * {b, n} in floats, b = 0 when all sequences share the positions), applied to Q and K; V (may be
 * null) is copied. Results are rounded once to out_dtype (round to nearest even). Inputs
 * [B, N, H, D] of in_dtype with element strides {b, n, h}; outputs likewise (any layout with a
 * contiguous D axis: [B, N, H, D] memory is what the attention entry points take as [B, H, N, D]
 * views). Every row start must be 16-byte aligned; D a multiple of 8.
 */
int sps_rope_qkv(int B, int N, int H, int D, int in_dtype, const void* q, const int64_t* q_strides, const void* k,
                 const int64_t* k_strides, const void* v, const int64_t* v_strides, const float* freqs,
                 const int64_t* freqs_strides, int out_dtype, void* q_out, const int64_t* q_out_strides,
                 void* k_out, const int64_t* k_out_strides, void* v_out, const int64_t* v_out_strides,
                 void* stream);

/*
 * Prefill -> decode caches of one layer, one launch for the batch (replaces the per-row loop of
 * _materialize_prefill_layer_state, reverse_sps/inference.py:568-613). k, v: [B, 2T, H, D] of
 * in_dtype (strides {b, n, h}), the interleaved input/<predict> rows after RoPE; doc_mask: [B, T]
 * bytes (nonzero: token t belongs to the row's current document; row stride doc_mask_stride).
 * For every b whose document has n > 0 tokens d_0 < ... < d_{n-1}:
 *   retained K/V[b, h, j, :] = K/V[b, 2 d_j + retained_slot, h, :] for j < n, ret_len[b, h] = n;
 *   ring (window_tokens > 0): w = min(n, window_tokens), ring K/V[b, h, i, :] =
 *     K/V[b, 2 d_{n-w+i} + window_slot, h, :] for i < w, ring_len[b] = w, ring_pos[b] = 0;
 * other cache rows are untouched, and rows with n == 0 are untouched entirely. Values are converted
 * to kv_dtype (round to nearest even). Caches and length arrays are described as for sps_kv_update;
 * rows past ret_storage are not written (the caller sizes the retained buffer for the prompt).
 * Every row start must be 16-byte aligned; D a multiple of 8.
 */
int sps_prefill_to_decode(int B, int T, int H, int D, int in_dtype, const void* k, const int64_t* k_strides,
                          const void* v, const int64_t* v_strides, int window_slot, int retained_slot,
                          const uint8_t* doc_mask, int64_t doc_mask_stride, int kv_dtype, void* ring_k,
                          void* ring_v, const int64_t* ring_strides, int ring_storage, int window_tokens,
                          void* ring_len, void* ring_pos, const int64_t* ring_len_strides, void* ret_k,
                          void* ret_v, const int64_t* ret_strides, int ret_storage, void* ret_len,
                          const int64_t* ret_len_strides, int len_dtype, void* stream);

/*
 * Document ids of token rows, one launch for the batch (replaces generate_left_padded_document_idx,
 * model.py:70-99, and the repeat_interleave(2) of the SPS callers, reverse_sps/core.py:218-227).
 * tokens: [B, T] int32/int64 with row stride tokens_stride_b. A token is real when it differs from
 * pad_token_id. A real token's id is the row's pad count plus the number of real EOS tokens
 * (eos_token_id) strictly before it; the i-th pad token's id is i. Each id is written `repeat` (1 or
 * 2) times: out[b, t * repeat + r], int32/int64 with row stride out_stride_b (repeat = 2 gives the
 * [B, 2T] ids of the interleaved input/<predict> sequence). Rows must be left padded: bad_rows
 * (int32 [B], may be null) receives 1 for a row with a pad token after a real token (its ids follow
 * the same formula; the reference raises ValueError for such input) and 0 otherwise.
 */
int sps_document_ids(int B, int T, const void* tokens, int tokens_dtype, int64_t tokens_stride_b,
                     int64_t eos_token_id, int64_t pad_token_id, int repeat, void* out, int out_dtype,
                     int64_t out_stride_b, int* bad_rows, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPS_ATTN_H */
