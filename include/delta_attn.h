/*
 * delta_attn.h -- C ABI of the MI355X (gfx950) Delta Attention prefill path.
 *
 * Three kernels make up one delta-attention layer prefill:
 *   (1) key-sparse attention: causal sliding window + sink tokens, with the
 *       window anchored at the last row of each q_block-row query block;
 *   (2) query-sparse / key-dense attention: a chosen set of query rows, each
 *       attending every key up to its own inclusive limit, optionally fused
 *       with the delta epilogue (delta = dense - sparse at anchor rows,
 *       dense rows scattered straight into the layer output);
 *   (3) delta broadcast-add: every row gets the delta of the nearest
 *       anchor at or before it.
 *
 * Conventions shared by every entry point:
 *   - Tensors are device pointers. The last (head_dim) dimension is
 *     contiguous; every other dimension is described by an element stride
 *     (not a byte stride). Rows must be 16-byte aligned: base pointers
 *     16-byte aligned and every stride a multiple of 8 elements.
 *   - dtype is DA_BF16 or DA_FP16; compute is fp32 accumulate on MFMA.
 *   - Everything is asynchronous on `stream` (a hipStream_t; NULL = default
 *     stream). No entry point synchronises, allocates or frees; the caller
 *     owns all memory, including workspaces.
 *   - Return 0 on success or a negative DA_ERR_* code. No entry point keeps
 *     a pointer after it returns and, apart from the static scratch of
 *     da_decode_attn_fwd_dev_noalloc and the process-wide tile-shape choice
 *     of da_set_sparse_rows_per_wave (read when a launch is issued; results do
 *     not depend on it), there is no mutable global state, so calls are
 *     re-entrant.
 */
#ifndef DELTA_ATTN_H
#define DELTA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DA_OK 0
#define DA_ERR_INVALID_ARG (-1)      /* shape, stride, range or null-pointer error */
#define DA_ERR_HEAD_DIM (-2)         /* head_dim not supported (forward, decode and RoPE: 32, 64, 128, 256; backward: up to 128) */
#define DA_ERR_DTYPE (-3)            /* dtype not DA_BF16 / DA_FP16 */
#define DA_ERR_ALIGNMENT (-4)        /* pointer or stride breaks 16-byte row alignment */
#define DA_ERR_WORKSPACE (-5)        /* workspace missing or smaller than required */
#define DA_ERR_LAUNCH (-6)           /* hipGetLastError reported a launch failure */
#define DA_ERR_SCRATCH (-7)          /* sizes need more than the library's static scratch holds */

#define DA_BF16 0
#define DA_FP16 1

/* Epilogue modes of da_qsparse_attn_fwd. */
#define DA_EPI_OUTPUT 0    /* o[b, h, i, :] = attention row i (the plain kernel) */
#define DA_EPI_DELTA 1     /* rows i < n_anchor: delta[b, i, h, :] = dense - sparse[b, q_rows[i], h, :];
                              rows i >= n_anchor: out[b, q_rows[i], h, :] = dense */
#define DA_EPI_SCATTER 2   /* out[b, q_rows[i], h, :] = dense for every row (mode "recompute") */
#define DA_EPI_DENSE 3     /* rows i < n_anchor: delta[b, i, h, :] = dense (the dense anchor rows
                              da_sparse_attn_delta_fwd consumes); rows i >= n_anchor:
                              out[b, q_rows[i], h, :] = dense */

/*
 * Kernel (1): key-sparse attention (sink + block-anchored sliding window).
 * Replaces hip-attn `block_sparse_attention` as called from
 * delta_attention/llama.py:407-449 (LlamaAttention.hip_attention_interface,
 * "window" branch); visibility follows delta_attention/train/flex_delta.py:59-61:
 *   key k is visible to row r  iff  k <= r  and  (k < sink  or
 *   k + window > floor(r / q_block) * q_block + q_block - 1).
 * q [B, Hq, S, D] (strides q_str = {batch, head, seq}), k/v [B, Hkv, S, D],
 * out [B, S, Hq, D] layout given by o_str = {batch, head, seq}; Hq % Hkv == 0
 * (GQA: query head h reads key/value head h / (Hq / Hkv)).
 * sm_scale multiplies q.k before the softmax.
 */
int da_sparse_attn_fwd(const void* q, const void* k, const void* v, void* out,
                       int B, int Hq, int Hkv, int S, int D,
                       const int64_t q_str[3], const int64_t k_str[3],
                       const int64_t v_str[3], const int64_t o_str[3],
                       int window, int sink, int q_block, float sm_scale,
                       int dtype, void* stream);

/* da_sparse_attn_fwd for query rows row0 .. row0 + n_rows - 1 only (the
 * visibility of each row as in the full launch; out rows outside the range
 * untouched), so that a row range can run beside other work: the adaptive
 * stride's chunk decisions need only their chunk's rows of the key-sparse
 * output (llama.py:784-788). No counterpart in the reference, which runs the
 * key-sparse pass over all rows first. row0 + n_rows must not exceed S. */
int da_sparse_attn_fwd_rows(const void* q, const void* k, const void* v, void* out,
                            int B, int Hq, int Hkv, int S, int D,
                            const int64_t q_str[3], const int64_t k_str[3],
                            const int64_t v_str[3], const int64_t o_str[3],
                            int window, int sink, int q_block, float sm_scale,
                            int row0, int n_rows, int dtype, void* stream);

/*
 * Kernel (1) with kernel (3) fused into its epilogue: the uniform-stride
 * broadcast of delta_attention/llama.py:733-755 applied while the key-sparse
 * rows are still in registers, so the sparse output is written once and never
 * re-read. For rows r < s_p:
 *   delta[g] = rnd(dense_sel[b, g, h, :] - rnd(sparse[b, g * gamma, h, :]))
 *   out[b, r, h, :] = rnd(rnd(sparse[b, r, h, :]) + delta[r / gamma])
 * (the reference's bf16 composition, bit-identical to da_sparse_attn_fwd
 * followed by da_delta_add on the same inputs). Rows >= s_p of `out` are not
 * written (they hold the dense tail, written by da_qsparse_attn_fwd with
 * DA_EPI_DENSE, which also produces dense_sel [B, n_anchor, Hq, D] with ds_str
 * = {batch, head, anchor}). delta_out (NULL: not written) receives the deltas
 * in the same layout (dl_str). Requires s_p % gamma == 0 and gamma dividing
 * da_fused_delta_rows(Hq, Hkv); other arguments as for da_sparse_attn_fwd.
 * No counterpart in the reference beyond the composition it replaces.
 */
int da_sparse_attn_delta_fwd(const void* q, const void* k, const void* v, void* out,
                             int B, int Hq, int Hkv, int S, int D,
                             const int64_t q_str[3], const int64_t k_str[3],
                             const int64_t v_str[3], const int64_t o_str[3],
                             int window, int sink, int q_block, float sm_scale,
                             const void* dense_sel, const int64_t ds_str[3],
                             int gamma, int s_p,
                             void* delta_out, const int64_t dl_str[3],
                             int dtype, void* stream);

/*
 * Largest row-tile height the fused delta launch can use for this head
 * geometry (128; 0 for invalid head counts): gamma must divide it. The launch
 * packs two heads per 64-row tile when Hq / Hkv is even and gamma divides 64,
 * else one head per 128-row tile; the results do not depend on the packing.
 */
int da_fused_delta_rows(int Hq, int Hkv);

/*
 * Query rows per wave of the head_dim-128 key-sparse launches (kernel (1),
 * the fused delta launch and the adaptive layer's sparse passes): 32 (the
 * default; two 4-wave workgroups per CU) or 64 (one workgroup per CU, each
 * K/V fragment read from LDS feeding two MFMAs, O in AGPRs). Process-wide;
 * returns DA_ERR_INVALID_ARG for other values. The per-row rescale decisions
 * make every output bit independent of the choice. No counterpart in the
 * reference: a tile-shape knob of this implementation (the reference's
 * kernels pick their tiles internally).
 */
int da_set_sparse_rows_per_wave(int rows);
int da_sparse_rows_per_wave(void);

/*
 * Workspace (bytes) that da_qsparse_attn_fwd needs for these sizes; 0 is a
 * valid answer. n = number of selected query rows, Skv = number of keys.
 */
size_t da_qsparse_workspace_bytes(int B, int Hq, int Hkv, int n, int Skv, int D);

/*
 * Kernel (2): query-sparse / key-dense attention with split-KV.
 * Replaces the Triton `_attn_fwd` behind delta_attention/delta_kernel.py:262-329
 * (`attention(q, k, v, mask, sm_scale)`), called at llama.py:720 / :786 / :814.
 * Row i of the selection reads query row q_rows[i] (q_rows == NULL: row i) of q
 * and attends keys 0 .. row_last[b * rl_bstride + i] inclusive (limits need not
 * be sorted; rl_bstride 0 shares one limit vector over the batch). Limits are
 * clamped to Skv - 1; a negative limit gives an all-zero row; q_rows values
 * are clamped into [0, Sq).
 * q [B, Hq, Sq, D]; k/v [B, Hkv, Skv, D].
 *   epi == DA_EPI_OUTPUT : o [B, Hq, n, D] with o_str = {batch, head, row}.
 *   epi == DA_EPI_DELTA  : `o` is the layer output [B, S, Hq, D] (o_str =
 *       {batch, head, seq}) holding the sparse rows; `delta` is
 *       [B, n_anchor, Hq, D] in `dtype` with d_str = {batch, head, anchor}.
 *       Rounding follows the reference's bf16 composition
 *       (delta_attention/llama.py:740): delta = rnd(rnd(dense) - sparse).
 *   epi == DA_EPI_SCATTER: `o` as for DA_EPI_DELTA, every row written.
 *   epi == DA_EPI_DENSE  : as DA_EPI_DELTA, but `delta` receives rnd(dense) for
 *       rows i < n_anchor (`o` is not read).
 * workspace must hold da_qsparse_workspace_bytes(...) bytes.
 */
int da_qsparse_attn_fwd(const void* q, const void* k, const void* v,
                        const int64_t* q_rows, const int64_t* row_last, int64_t rl_bstride,
                        int n, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                        const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
                        void* o, const int64_t o_str[3],
                        int epi, int n_anchor, void* delta, const int64_t d_str[3],
                        float sm_scale, void* workspace, size_t workspace_bytes,
                        int dtype, void* stream);

/* da_qsparse_attn_fwd (DA_EPI_OUTPUT) for a row list of n slots of which
 * about n_live hold keys: the split items per row tile follow the plan of
 * n_live rows and the grid covers all n, so a padded list keeps the
 * parallelism of its live rows. n_dev: NULL, or a device int, read on the
 * device, saying that only the first *n_dev rows (clamped to [0, n]) are
 * live; their row tiles' items come first in the grid, the others exit at
 * once, and output rows in row tiles wholly past *n_dev are not written.
 * For the adaptive stride's chunk lists, whose length is decided on the
 * device (n = the chunk's anchor slots at the finest stride). No counterpart
 * in the reference, whose chunk lists have host-known lengths.
 * workspace must hold da_qsparse_workspace_bytes_live(...) bytes. */
size_t da_qsparse_workspace_bytes_live(int B, int Hq, int Hkv, int n, int n_live, int Skv, int D);
int da_qsparse_attn_fwd_live(const void* q, const void* k, const void* v,
                             const int64_t* q_rows, const int64_t* row_last, int64_t rl_bstride,
                             int n, int n_live, const int* n_dev,
                             int B, int Hq, int Hkv, int Sq, int Skv, int D,
                             const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
                             void* o, const int64_t o_str[3], float sm_scale,
                             void* workspace, size_t workspace_bytes, int dtype, void* stream);

/*
 * Decode row: the query at the end of a KV cache of n_keys keys (position
 * n_keys - 1) attends keys [0, sink) and its last `window` keys
 * [n_keys - window, n_keys) (window == 0: every key). Replaces the decode
 * rows of delta_attention/llama.py:537-549 (`_decode_sparse_row`, sink + last
 * window keys; with window >= n_keys - sink that is every key) and the dense
 * anchor row of :598-600 (window 0), which delta_decode_forward composes.
 * q [B, Hq, 1, D] and out [B, Hq, 1, D] with strides {batch, head, row};
 * k/v [B, Hkv, n_keys, D] ({batch, head, seq}). Split-KV over the row's key
 * tiles, merged in a second kernel; workspace must hold
 * da_decode_workspace_bytes(...) bytes.
 */
size_t da_decode_workspace_bytes(int B, int Hq, int Hkv, int n_keys, int D, int window, int sink);
int da_decode_attn_fwd(const void* q, const void* k, const void* v, void* out,
                       int B, int Hq, int Hkv, int n_keys, int D,
                       const int64_t q_str[3], const int64_t k_str[3],
                       const int64_t v_str[3], const int64_t o_str[3],
                       int window, int sink, float sm_scale,
                       void* workspace, size_t workspace_bytes, int dtype, void* stream);

/*
 * The same decode row with the key count in device memory: *n_keys_dev
 * (int32, 4-byte aligned, clamped to [1, max_keys] when the kernels run) keys
 * of k/v buffers that hold max_keys rows. The launch shape and the workspace
 * (da_decode_workspace_bytes(..., max_keys, ...)) depend on max_keys only, so
 * one recorded call serves every length of a growing cache: this is the form
 * a decode step captured in a HIP graph uses (the key count advances on the
 * device between replays). Same row semantics as da_decode_attn_fwd
 * (delta_attention/llama.py:537-549, 598-600); the split-KV partition differs
 * with max_keys, so the two agree to rounding, not bit for bit.
 * addend (NULL: none) [B, Hq, 1, D] with add_str {batch, head, row}: out =
 * rnd(rnd(row) + addend), the cached-delta add of a delta decode step
 * (llama.py:612-620 `sparse_out + last_delta`) in the same launch.
 */
int da_decode_attn_fwd_dev(const void* q, const void* k, const void* v, void* out,
                           int B, int Hq, int Hkv, const int32_t* n_keys_dev, int max_keys, int D,
                           const int64_t q_str[3], const int64_t k_str[3],
                           const int64_t v_str[3], const int64_t o_str[3],
                           int window, int sink, float sm_scale,
                           const void* addend, const int64_t add_str[3],
                           void* workspace, size_t workspace_bytes, int dtype, void* stream);

/*
 * da_decode_attn_fwd_dev without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The split-KV partials go to a static device array of
 * DA_DECODE_SCRATCH_BYTES (16 MiB; each GPU the library runs on holds its own
 * copy until the process ends); sizes whose partials
 * (da_decode_workspace_bytes(B, Hq, Hkv, max_keys, D, window, sink)) exceed
 * it return DA_ERR_SCRATCH. Allocates nothing. Calls that overlap on one GPU
 * (e.g. on two streams at once) share the array and race. The current device
 * must be the device of `stream`. Results equal da_decode_attn_fwd_dev's on
 * the same arguments bit for bit.
 */
#define DA_DECODE_SCRATCH_BYTES (16u << 20)
size_t da_decode_scratch_bytes(void);
int da_decode_attn_fwd_dev_noalloc(const void* q, const void* k, const void* v, void* out,
                                   int B, int Hq, int Hkv, const int32_t* n_keys_dev,
                                   int max_keys, int D,
                                   const int64_t q_str[3], const int64_t k_str[3],
                                   const int64_t v_str[3], const int64_t o_str[3],
                                   int window, int sink, float sm_scale,
                                   const void* addend, const int64_t add_str[3],
                                   int dtype, void* stream);

/*
 * Kernel (3): delta broadcast-add over rows 0 .. s_p-1.
 * Replaces the torch broadcast at delta_attention/llama.py:740-755 (uniform
 * stride) and delta_attention/stride.py:26-40 (`apply_delta_variable`).
 * out[b, r, h, :] = sparse[b, r, h, :] + delta_of(owner(r))[b, h, :]
 * where owner(r) = r / gamma when anchors == NULL, else the index of the last
 * anchor <= r (rows before anchors[0] take the last anchor, matching the
 * reference's searchsorted(...) - 1 == -1 indexing).
 * The delta comes from `delta` ([B, n_anchor, H, D] in `dtype`, d_str) when it
 * is non-NULL, else it is formed as rnd(dense_sel[b, a, h, :] -
 * sparse[b, anchors[a], h, :]) (dense_sel [B, n_anchor, H, D] with ds_str;
 * requires anchors). Arithmetic is fp32 with one rounding to `dtype` per
 * operation, the same sequence as the reference's torch ops, so results are
 * bit-identical to them on the same inputs.
 * sparse/out are [B, >=s_p, H, D] (strides {batch, head, seq}). With a
 * precomputed `delta`, out may alias sparse (in-place); when the delta is
 * formed from dense_sel, out must not alias sparse. With anchors == NULL,
 * n_anchor must be at least ceil(s_p / gamma); with anchors, they must be
 * ascending (values outside [0, s_p) are clamped into it when the delta is
 * formed from dense_sel).
 */
int da_delta_add(const void* sparse, const int64_t sp_str[3],
                 void* out, const int64_t o_str[3],
                 const void* delta, const int64_t d_str[3],
                 const void* dense_sel, const int64_t ds_str[3],
                 const int64_t* anchors, int n_anchor, int gamma, int s_p,
                 int B, int H, int D, int dtype, void* stream);

/*
 * Decoder-layer residual add + RMSNorm over rows of n elements (n in {2048,
 * 4096, 5120, 8192}), replacing `residual + hidden_states` followed by
 * LlamaRMSNorm (delta_attention/llama.py:69-74, :968-979):
 *   residual == NULL: y = rnd(w * rnd(x * rsqrt(mean(x^2) + eps)))
 *   otherwise:        h = rnd(x + residual) is written to h, then y = norm(h).
 * One rounding to `dtype` per torch op; fp32 inside. Row strides in elements;
 * in-place use (h == x or h == residual, y == x) is allowed.
 */
int da_add_rmsnorm(const void* x, int64_t x_stride, const void* residual, int64_t r_stride,
                   void* h, int64_t h_stride, void* y, int64_t y_stride,
                   const void* weight, int64_t rows, int n, float eps,
                   int dtype, void* stream);

/*
 * SwiGLU gate of LlamaMLP (delta_attention/llama.py:212-213):
 * out = rnd(rnd(silu(gate)) * up), silu(g) = g / (1 + exp(-g)) in fp32, over
 * rows of n elements (n % 8 == 0; row strides in elements).
 */
int da_swiglu(const void* gate, int64_t g_stride, const void* up, int64_t u_stride,
              void* out, int64_t o_stride, int64_t rows, int n, int dtype, void* stream);

/*
 * Attention prologue, in place: optional per-head RMSNorm (weights q_norm_w /
 * k_norm_w of length D, NULL = no norm; Qwen3, delta_attention/qwen3.py:37-43 and
 * llama.py:60-74) followed by rotary position embedding (rotate_half
 * convention, delta_attention/llama.py:161-192) of q [B, S, Hq, D] (strides
 * q_str = {batch, seq, head}) and k [B, S, Hkv, D] (k_str); either may be NULL.
 * cos/sin are [Bc, S, D] tables in `dtype` with element strides
 * cs_str = {batch (0 = shared), seq}. Each tensor op of the reference is
 * rounded to `dtype` once, as torch does, so the RoPE result is bit-identical
 * to the reference's ops on the same inputs.
 */
int da_rope_qk(void* q, const int64_t q_str[3], int Hq,
               void* k, const int64_t k_str[3], int Hkv,
               int B, int S, int D,
               const void* cos, const void* sin, const int64_t cs_str[2],
               const void* q_norm_w, const void* k_norm_w, float eps,
               int dtype, void* stream);

/*
 * One-token decode step variant (S == 1) of da_rope_qk that also appends to
 * the KV cache, replacing the cache update that follows RoPE in a decode step
 * (the reference's DynamicCache.update after apply_rotary_pos_emb,
 * llama.py:851-862): the rotated k is written to k_cache at row *pos (k itself
 * is not modified) and v is copied to v_cache at row *pos; q is rotated in
 * place. pos is an int64 in device memory (a graph-recorded step reads the
 * current row at replay). Caches are [B, max_len, Hkv, D] with strides
 * kc_str / vc_str = {batch, row, head}; k and v [B, 1, Hkv, D] with k_str /
 * v_str = {batch, seq, head}. max_len (>= 1) is the caches' row count: a
 * *pos outside [0, max_len) when the kernel runs writes neither cache (q is
 * still rotated), so a runaway position cannot write past the caches.
 */
int da_rope_qk_append(void* q, const int64_t q_str[3], int Hq,
                      const void* k, const int64_t k_str[3], int Hkv,
                      const void* v, const int64_t v_str[3],
                      int B, int D,
                      const void* cos, const void* sin, const int64_t cs_str[2],
                      const void* q_norm_w, const void* k_norm_w, float eps,
                      void* k_cache, const int64_t kc_str[3],
                      void* v_cache, const int64_t vc_str[3], int64_t max_len,
                      const int64_t* pos, int dtype, void* stream);

/* Consecutive-anchor delta cosine (stride.py:43-52 interanchor_cos, the
 * adaptive stride's drift signal, llama.py:784-788; drift.py:23-49
 * drift_summary's cosines and histogram). For deltas d_0 .. d_{n-1} per
 * (batch, head), writes cos_out[b, i, h] (dense [B, n-1, H] fp32) =
 * <d_i, d_{i+1}> / (max(|d_i|, 1e-8) * max(|d_{i+1}|, 1e-8)), fp32 over D.
 *   a       [B, n, H, D] (strides batch, anchor, head): the deltas, or with
 *           `sparse` given the dense anchor rows; then d_i = rnd(a_i -
 *           sparse[b, rows[i], h]) (one rounding to the element type, as the
 *           reference's tensor subtraction).
 *   sparse  [B, n_rows, H, D] (strides batch, row, head) or NULL; rows: device
 *           int64 [n] anchor rows into it (clamped to [0, n_rows)), NULL for 0..n-1.
 *   hist    NULL, or a device int32 [bins] that each cosine in [lo, hi] adds
 *           one to (torch.histc's bin rule; the caller zeroes it).
 * n < 2 launches nothing. Element strides must be even (4-byte pair reads). */
int da_anchor_delta_cos(const void* a, const int64_t a_str[3],
                        const void* sparse, const int64_t s_str[3],
                        const int64_t* rows, int64_t n_rows,
                        int B, int n, int H, int D,
                        float* cos_out, int* hist, int bins, float lo, float hi,
                        int dtype, void* stream);

/* One chunk of the adaptive stride (llama.py:779-805: interanchor_cos of the
 * chunk's deltas, then stride.py:55-62 next_gamma or stride.py:65-86
 * next_gamma_relative) decided on the device, so that the host enqueues every
 * chunk of delta_adaptive_forward without reading a value back; the reference
 * reads each chunk's mean cosine on the host. Two launches on `stream`:
 *   1. the cosines of da_anchor_delta_cos over the chunk's first n deltas,
 *      rnd(dense_i - sparse[b, rows[i], h]), into cos_work (>= B*(max_n-1)*H
 *      floats), with n = state[1] read on the device;
 *   2. one workgroup: their mean (fp64) and min (n < 2: 1.0 and 1.0) into
 *      log_mean[chunk] / log_min[chunk], this chunk's stride and n into
 *      log_gamma[chunk] / log_n[chunk]; the next stride by the absolute rule
 *      (trigger 0: halve below threshold, double above threshold + margin) or
 *      the relative one (trigger 1: against mu -/+ k * sd of log_mean[0 ..
 *      chunk-1], population sd, once two chunks are logged), clamped to
 *      [gamma_min, gamma_max]; state = {next stride, next n}; and, when
 *      next_end > next_start, rows_next[j] = next_start + j * stride for
 *      j < next n, -1 for the remaining max_n slots (da_qsparse_attn_fwd
 *      gives a -1 row an all-zero output).
 *   dense   [B, max_n, H, D] (strides batch, anchor, head): the chunk's dense
 *           anchor rows; sparse [B, n_rows, H, D] (strides batch, row, head).
 *   rows    device int64 [max_n]: the chunk's anchor rows (-1 past n).
 *   state   device int32 [2]: {stride, n} of this chunk (the caller writes the
 *           first chunk's).
 * Element strides must be even. No counterpart entry point in the reference
 * (it runs these steps as host code). */
int da_adapt_chunk_step(const void* dense, const int64_t d_str[3],
                        const void* sparse, const int64_t s_str[3], int64_t n_rows,
                        const int64_t* rows, int B, int H, int D, int max_n,
                        int* state, float* cos_work, int chunk,
                        int next_start, int next_end, int64_t* rows_next,
                        int trigger, double threshold, double margin, double k,
                        int gamma_min, int gamma_max,
                        double* log_mean, float* log_min, int* log_gamma, int* log_n,
                        int dtype, void* stream);

/* The whole adaptive-stride layer, replacing the host loop of
 * LlamaAttention.delta_adaptive_forward (llama.py:759-824) from the key-sparse
 * pass to the concatenated output: the chunk loop is enqueued here, so the
 * host neither reads back nor waits per chunk. Chunks are the adapt_chunk-row
 * ranges [start, end) of rows [0, s_p) (stride.py:111-112); the first uses
 * stride gamma0, each next one the stride da_adapt_chunk_step picks (trigger,
 * threshold, margin, k_sd, gamma_min, gamma_max as there). Per chunk c:
 *   side_stream (when not NULL): kernel (1) over rows [start, end) into out;
 *   stream: kernel (2) over the chunk's anchor rows start + j * stride
 *     against keys < end; the chunk's delta cosines, logs and next stride
 *     (da_adapt_chunk_step, after the chunk's rows of kernel (1)); then rows
 *     [start, end) of out become rnd(out[r] + rnd(dense[g] - out[anchor g]))
 *     for r in anchor g's stride group, in place (stride.py:26-40).
 * Then rows [s_p, S) of out are the dense tail rows (all causal keys), and
 * `stream` waits for everything given to side_stream. With side_stream NULL,
 * rows [0, s_p) of out must already hold the key-sparse pass and everything
 * runs on `stream`.
 *   q [B, Hq, S, D], k/v [B, Hkv, S, D], out [B, S, Hq, D]: strides as for
 *           da_sparse_attn_fwd.
 *   logs    device arrays of n_log >= ceil(s_p / adapt_chunk) entries:
 *           log_mean (fp64) / log_min (fp32) of each chunk's delta cosines,
 *           log_gamma / log_n (int32) its stride and anchor count; chunk c's
 *           anchors are start + j * log_gamma[c] for j < log_n[c].
 *   workspace  >= da_adapt_layer_workspace_bytes(...) bytes, 256-byte aligned,
 *           any contents; the same sizes must be passed to both calls.
 * No counterpart entry point in the reference (it runs the loop as Python). */
size_t da_adapt_layer_workspace_bytes(int B, int Hq, int Hkv, int S, int D, int s_p,
                                      int adapt_chunk, int gamma0, int gamma_min);
int da_adapt_layer_fwd(const void* q, const void* k, const void* v, void* out,
                       int B, int Hq, int Hkv, int S, int D,
                       const int64_t q_str[3], const int64_t k_str[3],
                       const int64_t v_str[3], const int64_t o_str[3],
                       int window, int sink, int q_block, float sm_scale,
                       int s_p, int adapt_chunk, int gamma0, int gamma_min, int gamma_max,
                       int trigger, double threshold, double margin, double k_sd,
                       double* log_mean, float* log_min, int* log_gamma, int* log_n, int n_log,
                       void* workspace, size_t ws_bytes, int dtype, void* stream,
                       void* side_stream);

/*
 * Training path: forward with saved row statistics, and the backward.
 * Together they replace the autograd of delta_forward_train
 * (delta_attention/train/flex_delta.py:95-196): its flex_attention sparse
 * branch (:167-170), the masked-SDPA anchor/tail rows (:175-184) and the
 * composition (:186-196).
 *
 * lse: fp32 [B, Hq, rows] (contiguous), the log-sum-exp of each row's scaled
 * scores in the log2 domain (scores times sm_scale * log2(e)): lse = m + log2(l);
 * +inf for a row with no visible key.
 *
 * da_sparse_attn_fwd_lse: da_sparse_attn_fwd plus lse ([B, Hq, S]).
 */
int da_sparse_attn_fwd_lse(const void* q, const void* k, const void* v, void* out,
                           int B, int Hq, int Hkv, int S, int D,
                           const int64_t q_str[3], const int64_t k_str[3],
                           const int64_t v_str[3], const int64_t o_str[3],
                           int window, int sink, int q_block, float sm_scale,
                           float* lse, int dtype, void* stream);

/* da_qsparse_attn_fwd with epi == DA_EPI_OUTPUT, plus lse ([B, Hq, n]). */
int da_qsparse_attn_fwd_lse(const void* q, const void* k, const void* v,
                            const int64_t* q_rows, const int64_t* row_last, int64_t rl_bstride,
                            int n, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                            const int64_t q_str[3], const int64_t k_str[3],
                            const int64_t v_str[3], void* o, const int64_t o_str[3],
                            float* lse, float sm_scale, void* workspace, size_t workspace_bytes,
                            int dtype, void* stream);

/*
 * Gradients of key-sparse attention (the mask of da_sparse_attn_fwd; the
 * backward of flex_delta.py:167-170). o/dout: the forward output and its
 * gradient, [B, S, Hq, D] with o_str/do_str = {batch, head, row}; lse from
 * da_sparse_attn_fwd_lse. dq [B, Hq, S, D], dk/dv [B, Hkv, S, D] (strides
 * {batch, head, row}) receive the gradients (GQA: summed over each KV head's
 * query heads); accumulate != 0 adds them instead: x = rnd(x + rnd(grad)).
 * Workspace: da_sparse_attn_bwd_workspace_bytes.
 */
/*
 * Rows per dK/dV work item at most in the two backward entry points below
 * (a key block's rows are cut into equal chunks of at most this many; the
 * chunks' fp32 partials are summed by a reduce launch): a positive multiple
 * of 32 up to 2^20, or 0 for the default 8192. Process-wide, read when a
 * plan is made: set it before the workspace queries (the workspace follows
 * the chunk count). Results agree to the rounding of the partial sums. No
 * counterpart in the reference: a work-split knob of this implementation,
 * which the tests use to drive the multi-chunk paths at small sizes.
 */
int da_set_bwd_rows_per_chunk(int rows);

size_t da_sparse_attn_bwd_workspace_bytes(int B, int Hq, int Hkv, int S, int D,
                                          int window, int sink, int q_block);
int da_sparse_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                       const void* dout, const float* lse, void* dq, void* dk, void* dv,
                       int B, int Hq, int Hkv, int S, int D,
                       const int64_t q_str[3], const int64_t k_str[3],
                       const int64_t v_str[3], const int64_t o_str[3],
                       const int64_t do_str[3], const int64_t dq_str[3],
                       const int64_t dk_str[3], const int64_t dv_str[3],
                       int window, int sink, int q_block, float sm_scale, int accumulate,
                       void* workspace, size_t workspace_bytes, int dtype, void* stream);

/*
 * Gradients of selected rows attending their causal keys (the backward of the
 * masked SDPA at flex_delta.py:178-184). Row i is q row q_rows[i] (distinct
 * rows) and sees keys 0 .. row_last[i]; row_last must be ascending (the
 * anchor-then-tail order is). o/dout [B, n, Hq, D] with {batch, head, i}
 * strides, lse [B, Hq, n] from da_qsparse_attn_fwd_lse; dq is [B, Hq, Sq, D]
 * (rows q_rows[i] written or, with accumulate, added to), dk/dv as above.
 */
size_t da_qsparse_attn_bwd_workspace_bytes(int B, int Hq, int Hkv, int n, int Skv, int D);
int da_qsparse_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                        const void* dout, const float* lse,
                        const int64_t* q_rows, const int64_t* row_last, int n,
                        void* dq, void* dk, void* dv,
                        int B, int Hq, int Hkv, int Sq, int Skv, int D,
                        const int64_t q_str[3], const int64_t k_str[3],
                        const int64_t v_str[3], const int64_t o_str[3],
                        const int64_t do_str[3], const int64_t dq_str[3],
                        const int64_t dk_str[3], const int64_t dv_str[3],
                        float sm_scale, int accumulate, void* workspace,
                        size_t workspace_bytes, int dtype, void* stream);

/*
 * Backward of the composition (flex_delta.py:186-196, and the _ScaleGrad /
 * detach arms, flex_delta.py:79-92): upstream gradient grad [B, S, H, D] ->
 *   dsparse [B, S, H, D]: grad[r] for r < s_p, rnd(grad[r] - ddelta[r / gamma])
 *                         at anchor rows, 0 for r >= s_p;
 *   ddense [B, n_anchor + S - s_p, H, D]: ddelta[i] for the anchors, then
 *                         grad[s_p + t] for the tail rows;
 * with ddelta[i] = rnd(delta_grad_scale * rnd(sum_j grad[i gamma + j])) (the
 * scale multiply only when it is not 1), 0 when detach_delta. Strides
 * {batch, head, row}; requires s_p % gamma == 0.
 */
int da_delta_compose_bwd(const void* grad, const int64_t g_str[3],
                         void* dsparse, const int64_t sp_str[3],
                         void* ddense, const int64_t dd_str[3],
                         int B, int H, int S, int D, int gamma, int s_p,
                         float delta_grad_scale, int detach_delta, int dtype, void* stream);

/* Library identification: the gfx target the code objects were built for. */
const char* da_build_target(void);

#ifdef __cplusplus
}
#endif

#endif /* DELTA_ATTN_H */
