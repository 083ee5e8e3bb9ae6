/*
 * libvault_amd — C ABI of the MI355X (gfx950) kernels for the VAULT v3 decode/prefill hot path.
 *
 * Conventions (mirroring runtime/vault3.h:9-12, 35-49, 89, 153-161 of the reference):
 *   - Every entry point is stream-ordered on `stream` (a hipStream_t; NULL = default stream),
 *     takes device pointers and plain sizes, never allocates (vgx_host_alloc / vgx_host_free, the
 *     pinned host ring of the decode step, aside), never synchronises.
 *   - Return value: 0 = VGX_OK, negative = error (codes reuse the reference's V3_E_* numbers
 *     where the meaning matches).  Launch failures return VGX_E_HIP.
 *   - Dtype tags are the VLT3 tensor dtypes (tools/vlt3.py:29; runtime/vault3.h:51).
 *
 * Quantized weights live on the device in a packed "row-quad" layout produced by
 * vgx_qweight_pack from the VLT3 AoS blocks (34-byte Q8_0, 18-byte Q4_0; tools/vlt3.py:98-99):
 *   rows are padded to a multiple of 4 (padding rows have scale 0);
 *   quants: [rows/4][cols/32][4][QB]   QB = 32 (Q8_0 int8), 16 (Q4_0 nibble bytes), 128 (F32 floats)
 *   scales: [rows/4][cols/32][4] fp16, at byte offset vgx_qweight_scale_offset() (Q8_0/Q4_0 only)
 * The byte count per block is unchanged (34 / 18 B); the layout lets one lane fetch one 32-weight
 * block of four rows with aligned 128-bit loads.
 */
#ifndef VAULT_AMD_H
#define VAULT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VGX_ABI_VERSION 2

enum {
    VGX_OK = 0,
    VGX_E_SIZE = -1,   /* V3_E_SIZE: a size or count is out of range */
    VGX_E_DTYPE = -5,  /* V3_E_DTYPE: unsupported dtype for this entry point */
    VGX_E_SHAPE = -7,  /* V3_E_SHAPE: inconsistent shapes (e.g. cols not a multiple of 32) */
    VGX_E_ARENA = -8,  /* V3_E_ARENA: caller workspace too small or misaligned */
    VGX_E_LIMIT = -10, /* V3_E_LIMIT: exceeds a compiled limit */
    VGX_E_ALIGN = -11, /* V3_E_ALIGN: pointer not aligned as required */
    VGX_E_ARG = -31,   /* null pointer or invalid flag */
    VGX_E_HIP = -32,   /* a HIP launch failed */
    VGX_E_STATE = -33  /* not allowed in the caller's current state (see the entry point) */
};

enum { VGX_F32 = 0, VGX_F16 = 1, VGX_BF16 = 2, VGX_Q8_0 = 8, VGX_Q4_0 = 9 };

/* ---------------------------------------------------------------- version ---------------------- */

/* ABI version of this library (VGX_ABI_VERSION).  No counterpart in the reference. */
int vgx_abi_version(void);

/* ---------------------------------------------------------------- weights ---------------------- */

/* Bytes of the packed device layout for a [rows x cols] tensor of `dtype` (Q8_0, Q4_0 or F32);
 * negative on error.  Replaces the reference's in-place use of file blocks
 * (runtime/vault3.c:172-196 dtype_nbytes, 536-598 block walks). */
int64_t vgx_qweight_packed_bytes(int dtype, int64_t rows, int64_t cols);

/* Byte offset of the fp16 scale plane inside a packed Q8_0/Q4_0 tensor. */
int64_t vgx_qweight_scale_offset(int dtype, int64_t rows, int64_t cols);

/* VLT3 AoS blocks (device copy of the file payload) -> packed layout.  F32 takes row-major
 * floats.  Replaces the file-layout reads of runtime/vault3.c:499-602 / tools/vlt3.py:114-157. */
int vgx_qweight_pack(int dtype, const void *src_blocks, void *dst_packed, int64_t rows, int64_t cols,
                     void *stream);

/* Gate and up projections (same dtype, [rows x cols] each) packed into one tensor of 2*rows rows,
 * row-quad q holding gate rows 2q,2q+1 and up rows 2q,2q+1, for vgx_qlinear_swiglu.
 * Replaces the paired row walk of runtime/vault3.c:1942-1956 (mlp_gu_run). */
int vgx_qweight_pack_gateup(int dtype, const void *gate_blocks, const void *up_blocks, void *dst_packed,
                            int64_t rows, int64_t cols, void *stream);

/* Like vgx_qweight_pack with the rows of every head of head_dim rows among the first n_rope_rows
 * reordered so that packed row-quad j of a head holds rows 2j, 2j + head_dim/2, 2j + 1,
 * 2j + 1 + head_dim/2 (two RoPE rotation pairs); later rows keep their order.  The layout that
 * vgx_qkv_rope_step reads (q rows: n_rope_rows = rows; k|v rows: n_rope_rows = the k rows).
 * Same bytes as the reference tensor, reordered (tools/vlt3.py:98-99 blocks). */
int vgx_qweight_pack_rope(int dtype, const void *src_blocks, void *dst_packed, int64_t rows, int64_t cols,
                          int64_t head_dim, int64_t n_rope_rows, void *stream);

/* Packed layout -> VLT3 AoS blocks (inverse of vgx_qweight_pack; bit-exact round trip). */
int vgx_qweight_unpack(int dtype, const void *packed, void *dst_blocks, int64_t rows, int64_t cols,
                       void *stream);

/* Packed weights -> fp32 [rows x cols]: w = f32(d) * q (Q8_0), (n - 8) * f32(d) (Q4_0).
 * Bit-exact restatement of tools/vlt3.py:114-116, 152-157 (dequantize_q8_0 / dequantize_q4_0). */
int vgx_qweight_dequant(int dtype, const void *packed, float *out, int64_t rows, int64_t cols, void *stream);

/* Embedding lookup: out[i, :] = dequant(row ids[i]) for i < n_ids; ids outside [0, rows) read row
 * `pad_row` (runtime/vault3.c:2040 substitutes pad_id).  Replaces embed_row (runtime/vault3.c:626-654)
 * and nn.Embedding (src/vault_v3_model.py:1169, 2285). */
int vgx_embed_rows(int dtype, const void *packed, int64_t rows, int64_t cols, const int64_t *ids, int64_t n_ids,
                   int64_t pad_row, float *out, int64_t ldo, void *stream);

/* Adds to *count (device uint32, zeroed by the caller) the number of non-finite values in a VLT3
 * payload of n_elems elements: F32 / F16 / BF16 elements, or the fp16 block scales of Q8_0 / Q4_0
 * AoS blocks (data = the file's block bytes).  Replaces check_tensor_finite (runtime/vault3.c:215-271),
 * the loader's NaN / Inf rejection. */
int vgx_count_nonfinite(int dtype, const void *data, int64_t n_elems, uint32_t *count, void *stream);

/* ---------------------------------------------------------------- linear ----------------------- */

/* y[b, r] (+)= sum_c W[r, c] * x[b, c] (+ bias[r]) for b < batch, r < rows.
 * accumulate = 0 overwrites y, 1 adds into y (fused residual add).  bias may be NULL.
 * Replaces matvec/row_dot (runtime/vault3.c:499-624) and every nn.Linear / F.linear of the
 * decode and prefill paths (src/vault_v3_model.py:1036-1047, 1139, 1145-1150, 2150-2151). */
int vgx_qlinear(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                int64_t batch, const float *bias, float *y, int64_t ldy, int accumulate, void *stream);

/* GEMV epilogues of vgx_qlinear_ex. */
enum { VGX_EPI_STORE = 0, VGX_EPI_ACCUM = 1, VGX_EPI_SWIGLU = 2 };

/* Fused RMSNorm + GEMV: with u_b = norm_w * (x_b / sqrt(mean(x_b^2) + eps)) (or u_b = x_b when norm_w
 * is NULL), computes for b < batch
 *   VGX_EPI_STORE:  y[b, r]  = W[r] . u_b (+ bias[r])
 *   VGX_EPI_ACCUM:  y[b, r] += W[r] . u_b (+ bias[r])              (residual add)
 *   VGX_EPI_SWIGLU: y[b, r]  = silu(gate_r . u_b) * (up_r . u_b)   (vgx_qweight_pack_gateup tensor,
 *                                                                    `rows` = d_ff, bias must be NULL)
 * x and y must not overlap.  Replaces RMSNorm + nn.Linear pairs of the decode layer
 * (src/vault_v3_model.py:2289-2292, 1041-1047, 1145-1150, 2150-2151) and rmsnorm + matvec /
 * mlp_gu_run of runtime/vault3.c:2152-2160, 2193-2197, 2218-2219. */
int vgx_qlinear_ex(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                   int64_t batch, const float *norm_w, float eps, const float *bias, float *y, int64_t ldy,
                   int epilogue, void *stream);

/* vgx_qlinear_ex whose output address is read on the device when the launch runs: y = the float
 * pointer stored at *y_addr (an int64 device word, e.g. vgx_step_begin's out_ref).  A captured graph
 * then writes each replay's output to a buffer the host chose for that replay.  No counterpart in the
 * reference (its logits are a host array, runtime/vault3.c:2218-2222). */
int vgx_qlinear_indirect(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                         int64_t batch, const float *norm_w, float eps, const float *bias, const int64_t *y_addr,
                         int64_t ldy, int epilogue, void *stream);

/* Workspace bytes of vgx_qgemm for these sizes and epilogue (256-byte aligned buffer: a fixed 64 KiB
 * region of int32 output-tile counters first, then bf16 hi / lo splits of the activations, their
 * per-block sums, and K-split partial sums when the GEMM splits K to fill the GPU).  Decode batches
 * (at most 64 rows) whose splits the split workgroups sum themselves take tickets from the counters:
 * the workspace must be zero-filled before its first use, every call leaves the counters at zero (so a
 * captured graph needs no memset), and calls sharing one workspace must not overlap in time.  The
 * same workspace may serve vgx_qkv_rope_batch, which leaves the counter region untouched. */
int64_t vgx_qgemm_workspace_bytes(int64_t batch, int64_t rows, int64_t cols, int epilogue);

/* vgx_qlinear_ex for many activation rows on bf16 MFMA (Q8_0 / Q4_0 weights): same arguments and
 * epilogues, plus a caller workspace.  The activations (after the optional RMSNorm) enter as a bf16
 * hi + lo pair (2^-17 relative); weights, scales and the per-block fp32 accumulation are exact as in
 * the GEMV.  F32 weights run on fp32 MFMA (fp32 products and sums; no RMSNorm prologue on that path:
 * norm_w must be NULL; no workspace).  Replaces the chunk-prefill projections
 * (src/vault_v3_model.py:2051, 2095-2096 on [clen x d] blocks), batched decode projections, and the
 * segment scorer's fc1 over a chunk (:1224-1247). */
int vgx_qgemm(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx, int64_t batch,
              const float *norm_w, float eps, const float *bias, float *y, int64_t ldy, int epilogue, void *workspace,
              int64_t workspace_bytes, void *stream);

/* h[b, r] = silu(gate_r . x_b) * (up_r . x_b) over a vgx_qweight_pack_gateup tensor; `rows` is
 * the number of output rows (d_ff).  Replaces mlp_gu_run (runtime/vault3.c:1942-1956) and
 * F.silu(gate_proj(x)) * up_proj(x) (src/vault_v3_model.py:1149-1150). */
int vgx_qlinear_swiglu(int dtype, const void *w_gateup_packed, int64_t rows, int64_t cols, const float *x,
                       int64_t ldx, int64_t batch, float *h, int64_t ldh, void *stream);

/* ---------------------------------------------------------------- attention -------------------- */

/* Decode step descriptor: a small int32 device array that the host rewrites before every step, so
 * that one captured HIP graph of the decode step replays at every position of a chunk.  No
 * counterpart in the reference (its step reads pos from the host state, runtime/vault3.c:2034-2143). */
enum {
    VGX_STEP_SLOT = 0,       /* ring slot c = pos % W written by this step */
    VGX_STEP_TABLE_ROW = 1,  /* RoPE table row of the query/key position */
    VGX_STEP_SINK_SLOT = 2,  /* sink slot to fill (pos while pos < sink capacity), -1 for none */
    VGX_STEP_N_CUR = 3,      /* keys of the current chunk visible to this step (c + 1) */
    VGX_STEP_WORDS = 4
};

/* One contiguous run of key/value rows per (batch, kv group): row t of (b, g) is at element offset
 * b*batch_stride + g*group_stride + t*head_dim of k (and of v).  Element type is the KV dtype.
 * dyn_len (may be NULL): device int32; when set, only the first min(len, *dyn_len) rows are keys
 * (the current-chunk span of a graph-captured decode step points at step[VGX_STEP_N_CUR]). */
typedef struct {
    const void *k;
    const void *v;
    int64_t len;
    int64_t batch_stride;
    int64_t group_stride;
    const int32_t *dyn_len;
} vgx_kv_span;

/* Workspace bytes vgx_attn_decode needs for these sizes (0 when one split suffices): a fixed 16 KiB
 * region of int32 split tickets (one per (batch entry, kv group) for the first 4096 pairs; its size
 * and place do not depend on the call), then the per-split softmax partials (m, l, acc) that the
 * workgroup finishing a pair last combines (or a merge launch, for pairs beyond the ticket region or
 * more than 32 splits).  256-byte aligned.  The workspace must be zero-filled before its first use
 * and written by nothing else: every call leaves the tickets at zero (so a captured graph needs no
 * memset), and calls of any batch / group counts may share one workspace.  Calls sharing one
 * workspace must not overlap in time. */
int64_t vgx_attn_decode_workspace_bytes(int64_t B, int64_t H, int64_t G, int64_t D, int64_t n_keys);

/* Decode attention: out[b, h, :] = softmax_j(q[b,h].k_j * scale + bias[h, j]) v_j over the keys of
 * all spans concatenated in order, kv group g = h / (H/G).  q: fp32, head h of batch entry b at
 * b*ldq + h*D (post-RoPE); out: [B][H][D] fp32.  kv_dtype: VGX_F32 or VGX_BF16.  n_spans <= 4.
 * bias (may be NULL) is fp32 [H][bias_hstride], added to the keys of span `bias_span` (the
 * segment-memory span).  causal_base >= 0 makes the last span causal: batch entry b sees only its
 * first causal_base + b + 1 keys (chunked prefill, one query per entry); -1 disables it.
 * D in {64, 128}.
 * Replaces VAULTv3Attention.step's SDPA / explicit biased softmax (src/vault_v3_model.py:1098-1136),
 * the chunk attention of _forward_chunk_recurrent (:2064-2093) and attn_run (runtime/vault3.c:1958-2032). */
int vgx_attn_decode(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                    const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out, int64_t B,
                    int64_t H, int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream);

/* vgx_attn_decode without a caller workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  Same arguments, results and kernels as vgx_attn_decode; the split partials and
 * tickets live in a fixed 2 MiB device array of the library, one per GPU, held until the process
 * ends (located, and its tickets cleared by a fill kernel, by the first call on each device; that first
 * call must not be made while the stream is being captured into a graph, which would record the fill
 * instead of running it: it then returns VGX_E_STATE and records nothing).  Calls that would need
 * more than 2 MiB of workspace (vgx_attn_decode_workspace_bytes) return VGX_E_LIMIT: at 12 / 2 heads
 * and D = 128 that admits every batch up to 64 at 3584 keys (1.6 MB at most).  Every call on one GPU uses that GPU's
 * array, so calls that overlap in time on one GPU (other streams, other threads) race; the array
 * keeps the last call's contents. */
int vgx_attn_decode_noalloc(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                            const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out,
                            int64_t B, int64_t H, int64_t G, int64_t D, float scale, void *stream);

/* A run of keys for prefill attention: key j of kv group g at element offset
 * g*group_stride + j*row_stride of k (and v); rows are head_dim contiguous elements of the KV dtype
 * (bf16 or fp32; every run of one call has the same dtype). */
typedef struct {
    const void *k;
    const void *v;
    int64_t len;
    int64_t row_stride;
    int64_t group_stride;
} vgx_kv_run;

/* One block of queries (a chunk) for vgx_attn_prefill: query t of head h at q + t*ldq + h*q_hstride
 * (D contiguous elements, fp32 or bf16), output at out + t*ldo + h*o_hstride (elements of the call's
 * output dtype); runs concatenated in
 * order; when causal_base >= 0 the last run is causal: query t sees its keys j <= causal_base + t. */
typedef struct {
    const void *q;
    int64_t ldq;
    int64_t q_hstride;
    void *out;
    int64_t ldo;
    int64_t o_hstride;
    int64_t n_q;
    int64_t causal_base;
    int n_runs;
    vgx_kv_run runs[4];
    /* Optional bias on run bias_run (bias == NULL: none): query t of head h adds
     * bias[t*bias_ldq + bias_head_row[h]*bias_rstride + j] to its score with key j of that run;
     * bias_head_row (H entries, device memory) < 0 leaves head h unbiased.  The chunk-level resonance
     * bias on the segment run (src/vault_v3_model.py:1718-1793, 2083-2090). */
    const float *bias;
    const int32_t *bias_head_row;
    int64_t bias_ldq;
    int64_t bias_rstride;
    int bias_run;
} vgx_attn_block;

/* Prefill attention on bf16 MFMA (kv_dtype VGX_BF16, or VGX_F32 whose K / V enter the MFMAs as bf16
 * hi + lo pairs; q_dtype VGX_F32 (hi + lo) or VGX_BF16; D = 128; H/G in {1, 2, 4, 6, 8}) for up to 8
 * query blocks in one launch: out = softmax(q k^T * scale) v per query head h over kv group h / (H/G),
 * key tiles wholly in a query tile's causal future skipped.  out_dtype VGX_F32, or VGX_BF16 (the fp32
 * result rounded to nearest even, for bf16 callers).
 * Replaces the SDPA calls of block_sliding_attention (src/vault_v3_model.py:812-863) and of the
 * chunk-recurrent prefill (:2064-2093). */
int vgx_attn_prefill(int kv_dtype, int q_dtype, int out_dtype, const vgx_attn_block *blocks, int n_blocks, int64_t H,
                     int64_t G, int64_t D, float scale, void *stream);

/* vgx_attn_prefill with a workspace (16-byte aligned, at least vgx_attn_prefill_workspace_bytes(H, G)
 * bytes): a launch of few query tiles (a chunk of the chunk-recurrent prefill) splits each tile's keys
 * into up to four ranges computed in parallel and combines them (a second launch); results within
 * the same bars, not bit-equal to the unsplit call (the sums run in another order).  No counterpart in
 * the reference: the same computation as vgx_attn_prefill. */
int64_t vgx_attn_prefill_workspace_bytes(int64_t H, int64_t G);
int vgx_attn_prefill_ws(int kv_dtype, int q_dtype, int out_dtype, const vgx_attn_block *blocks, int n_blocks, int64_t H,
                        int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- small fused ops -------------- */

/* RMSNorm rows: y[r, :] = w * (x[r, :] / sqrt(mean(x[r, :]^2) + eps)).
 * Replaces RMSNorm.forward (src/vault_v3_model.py:764-774) and rmsnorm (runtime/vault3.c:656-660). */
int vgx_rmsnorm(const float *x, int64_t ldx, const float *w, float *y, int64_t ldy, int64_t n_rows, int64_t dim,
                float eps, void *stream);

/* RoPE + KV-cache write for N tokens (decode: one token per sequence; prefill: a run of tokens).
 * q (token t, head h at t*ldq + h*D; fp32) is rotated in place (q may be NULL when H = 0);
 * k (t*ldk + g*D) is rotated into k_rot (if non-NULL) and copied raw into k_raw (if non-NULL);
 * v (t*ldv + g*D) is copied into v_dst.  Destination row of token t,
 * group g: t*dst_tstride + g*dst_gstride (elements, KV dtype).  The first n_sink tokens are also
 * copied raw into sink_k_raw / sink_v at t*sink_tstride + g*sink_gstride.  table: fp32 rows
 * [cos(D/2) | sin(D/2)]; token t uses row table + t*table_rstride.
 * Replaces the ring write + RoPE of src/vault_v3_model.py:1079-1094, 2049-2058 and
 * runtime/vault3.c:2162-2179. */
int vgx_rope_qkv_write(int kv_dtype, float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
                       int64_t N, int64_t H, int64_t G, int64_t D, const float *table, int64_t table_rstride,
                       void *k_rot, void *k_raw, void *v_dst,
                       int64_t dst_tstride, int64_t dst_gstride, void *sink_k_raw, void *sink_v, int64_t n_sink,
                       int64_t sink_tstride, int64_t sink_gstride, void *stream);

/* Decode-step form of vgx_rope_qkv_write for B sequences with one token each: the ring slot, the
 * RoPE table row and the sink slot are read from the device step descriptor `step`
 * (VGX_STEP_SLOT / _TABLE_ROW / _SINK_SLOT).  q [B][H][D] (row stride ldq) is rotated in place; k/v
 * [B][G][D]; row (b, g) of slot c lands at b*dst_bstride + g*dst_gstride + c*dst_rstride of
 * k_rot / k_raw / v_dst, and of sink_k_raw / sink_v with the sink strides when the sink slot is >= 0
 * (sink pointers may be NULL).  Replaces src/vault_v3_model.py:1079-1094 and
 * runtime/vault3.c:2162-2179 inside a captured step. */
int vgx_rope_qkv_write_step(int kv_dtype, float *q, int64_t ldq, const float *k, int64_t ldk, const float *v,
                            int64_t ldv, int64_t B, int64_t H, int64_t G, int64_t D, const float *table,
                            int64_t table_rstride, const int32_t *step, void *k_rot, void *k_raw, void *v_dst,
                            int64_t dst_bstride, int64_t dst_gstride, int64_t dst_rstride, void *sink_k_raw,
                            void *sink_v, int64_t sink_bstride, int64_t sink_gstride, int64_t sink_rstride,
                            void *stream);

/* One decode token (batch 1): RMSNorm + q / k / v projections + bias, RoPE of q and k, and the
 * ring / sink writes of vgx_rope_qkv_write_step, in one launch.  wq: [H*D x d_model] and wkv:
 * [2*G*D x d_model] (k rows then v rows) packed with vgx_qweight_pack_rope (n_rope_rows = H*D for q,
 * G*D for k|v); dtype pairs (q, k|v): (Q4_0, Q8_0) or equal Q8_0 / Q4_0 / F32.  bq [H*D] and bkv
 * [2*G*D] are the natural-order biases (may be NULL).  q_out [H][D] receives the rotated query;
 * k_rot / k_raw / v_dst and sink_k_raw / sink_v (both or neither) are state tensors of kv_dtype
 * addressed as in vgx_rope_qkv_write_step with batch 0; x_copy (may be NULL) receives a copy of x.
 * x, norm_w and x_copy must be 16-byte aligned.  Replaces src/vault_v3_model.py:2289-2290,
 * 1041-1047, 1079-1094 and runtime/vault3.c:2152-2179 for one token. */
int vgx_qkv_rope_step(int q_dtype, const void *wq, const float *bq, int kv_wdtype, const void *wkv, const float *bkv,
                      int64_t d_model, int64_t H, int64_t G, int64_t D, const float *x, const float *norm_w, float eps,
                      float *x_copy, const float *table, int64_t table_rstride, const int32_t *step, float *q_out,
                      int kv_dtype, void *k_rot, void *k_raw, void *v_dst, int64_t dst_gstride, int64_t dst_rstride,
                      void *sink_k_raw, void *sink_v, int64_t sink_gstride, int64_t sink_rstride, void *stream);

/* A decode batch (1 <= B <= 64 sequences, one token each): RMSNorm + q / k / v projections + bias,
 * RoPE of q and k, and the ring / sink writes of vgx_rope_qkv_write_step, with the K-split sums of
 * the projections taken by the RoPE launch (no reduce launch of their own).  Weights packed with
 * vgx_qweight_pack (Q8_0 / Q4_0): wq [H*D x d_model] and wkv [2*G*D x d_model] (k rows then v rows),
 * or wq NULL and wkv [(H+2*G)*D x d_model] holding q, k and v rows (then bq must be NULL and bkv is
 * the bias of all rows).  x [B][d_model] (row stride ldx, 16-byte aligned, ldx % 4 == 0); norm_w
 * (16-byte aligned) may be NULL for no RMSNorm.  q_out [B][H][D] (row stride ldq) receives the
 * rotated queries; the state tensors are addressed as in vgx_rope_qkv_write_step.  workspace: at
 * least vgx_qkv_rope_batch_workspace_bytes(B, d_model, H, G, D, wq != NULL) bytes, 256-byte aligned;
 * its first 64 KiB (vgx_qgemm's tile counters, when one workspace serves both) are not written.
 * Replaces src/vault_v3_model.py:1041-1047, 1079-1094 (the batched decode path) and
 * runtime/vault3.c:2152-2179 per sequence. */
int64_t vgx_qkv_rope_batch_workspace_bytes(int64_t B, int64_t d_model, int64_t H, int64_t G, int64_t D,
                                           int separate_q);
int vgx_qkv_rope_batch(int q_wdtype, const void *wq, const float *bq, int kv_wdtype, const void *wkv,
                       const float *bkv, int64_t d_model, int64_t H, int64_t G, int64_t D, const float *x, int64_t ldx,
                       int64_t B, const float *norm_w, float eps, const float *table, int64_t table_rstride,
                       const int32_t *step, float *q_out, int64_t ldq, int kv_dtype, void *k_rot, void *k_raw,
                       void *v_dst, int64_t dst_bstride, int64_t dst_gstride, int64_t dst_rstride, void *sink_k_raw,
                       void *sink_v, int64_t sink_bstride, int64_t sink_gstride, int64_t sink_rstride,
                       void *workspace, int64_t workspace_bytes, void *stream);

/* Rotate rows: dst[o, i, :] = R(src[o, i, :]) with angle row table + i*table_rstride, for o < n_outer,
 * i < n_rows (rows contiguous, D elements each; src may equal dst).  Replaces the chunk-boundary
 * re-base of k_prev by R_{-W} and the prefix re-rotation of segment/sink keys
 * (src/vault_v3_model.py:1842-1856, 1926-1927; runtime/vault3.c:859-896, 1930-1940). */
int vgx_rope_rotate(int kv_dtype, const void *src, void *dst, int64_t n_outer, int64_t src_ostride,
                    int64_t dst_ostride, int64_t n_rows, int64_t D, const float *table, int64_t table_rstride,
                    void *stream);

/* Row gather: dst[o, j, :] = src[o, idx[j], :] for j < n_idx, o < n_outer (D elements per row,
 * element size from dtype VGX_F32 / VGX_BF16); an index outside [0, src_rows) writes zeros.
 * src and dst must not overlap.  Replaces the segment-bank KV compaction
 * (src/vault_v3_model.py:1914-1920; runtime/vault3.c:1892-1913). */
int vgx_gather_rows(int dtype, const void *src, void *dst, const int32_t *idx, int64_t n_idx, int64_t src_rows,
                    int64_t n_outer, int64_t src_ostride, int64_t dst_ostride, int64_t D, void *stream);

/* ---------------------------------------------------------------- segment-memory bank ---------- */

/* Control words of a segment bank (int32, on the device): entries in the bank, running global
 * segment-id offset, segment id and length of the current chunk's open segment.  They mirror
 * mem_cnt, seg_id_offset, cur_seg_id and cur_seg_len of the reference state (runtime/vault3.h:93-161). */
enum { VGX_SEG_MEM_CNT = 0, VGX_SEG_ID_OFFSET = 1, VGX_SEG_CUR_ID = 2, VGX_SEG_LEN = 3, VGX_SEG_WORDS = 4 };

/* One decode step's bookkeeping: tok_cur[b * tok_ld + c] = ids[b] for b < B at the ring slot
 * c = step[VGX_STEP_SLOT]; with seg_cur (batch 1 with segment memory), seg_cur[c] = the open segment
 * id, then the segment closes after this token at c = window - 1, at seg_max tokens, or by the token's
 * break tier (tiers[id], a byte per vocabulary entry; NULL = all 0): tier 1 from seg_min tokens, tier
 * 2 from max(seg_min, 2 seg_max / 3), tier 3 from max(seg_min, seg_max - 8).  Replaces
 * runtime/vault3.c:2107-2124 and src/vault_v3_model.py:2256-2268. */
int vgx_seg_step(const int64_t *ids, int64_t B, const int32_t *step, int32_t *tok_cur, int64_t tok_ld,
                 int32_t *seg_cur, int32_t *ctrl, const uint8_t *tiers, int64_t vocab, int64_t seg_min,
                 int64_t seg_max, int64_t window, void *stream);

/* Host inputs of a graph-captured decode step with no host-to-device copy.  The host writes each step's
 * descriptor words, token ids, output address and (while a resonance mode is active) segment-bias
 * vectors into one slot of a ring of n_slots slots in pinned, device-coherent host memory
 * (vgx_host_alloc); the step's first kernel, vgx_step_begin, reads the slot that the device counter
 * *counter names (slot *counter mod n_slots), does what vgx_seg_step does with those ids and words
 * (ids are not written when the slot's ring position lies outside [0, window)),
 * stores the words where the step's captured kernels read them, and advances the counter.  The host
 * numbers its slots the same way (the counter starts at 0 and every launch takes one slot) and
 * rewrites a slot only after the launch that read it has completed.  No counterpart in the reference
 * (its step reads the host state directly, runtime/vault3.c:2034-2143).
 *
 * Slot layout (byte offsets; slot_bytes from vgx_step_slot_bytes, a multiple of 256): */
enum {
    VGX_SLOT_STEP = 0,        /* int32[VGX_STEP_WORDS]: the descriptor words */
    VGX_SLOT_FLAGS = 16,      /* int32: VGX_SLOTF_* */
    VGX_SLOT_IDS_ADDR = 24,   /* int64: device address of int64 ids[B] (VGX_SLOTF_DEVICE_IDS) */
    VGX_SLOT_OUT_ADDR = 32,   /* int64: stored to *out_ref (the output address of an indirect GEMV) */
    VGX_SLOT_IDS = 64         /* int64 ids[B] (host ids), then the bias part at vgx_step_slot_bias_off */
};
enum { VGX_SLOTF_DEVICE_IDS = 1, VGX_SLOTF_BIAS = 2 };

/* Bytes of one slot for B ids and (bias_cap > 0) the bias part: int8 row[2][n_heads] (the early
 * rows' vector per head, then the late rows'; -1 = a zero row), padded to 16 bytes, then float
 * vec[3][bias_cap].  vgx_step_slot_bias_off: the bias part's offset. */
int64_t vgx_step_slot_bytes(int64_t B, int64_t n_heads, int64_t bias_cap);
int64_t vgx_step_slot_bias_off(int64_t B);

/* Pinned host memory the device reads coherently at the same address (hipHostMalloc, coherent and
 * mapped), zero-filled; for the step ring.  The only allocating entry points of the library. */
int vgx_host_alloc(int64_t bytes, void **ptr);
int vgx_host_free(void *ptr);

/* The first kernel of a decode step (one workgroup).  Reads slot (*counter mod n_slots) of ring:
 * step[0..VGX_STEP_WORDS) = its words; ids[b] = its ids (host ids, or those at its device address);
 * out_ref (may be NULL) = its output address; then vgx_seg_step's ring and segmenter update with
 * these ids and words; with bias_early / bias_late (both or neither) and the slot's VGX_SLOTF_BIAS,
 * row h of bias_early (row stride bias_ld, bias_cap entries) = vec[row[0][h]] and of bias_late =
 * vec[row[1][h]] (zeros for -1); finally *counter = (*counter + 1) mod n_slots.  Replaces the step's host copies of the
 * descriptor, ids and bias rows (runtime/vault3.c:1976-1988 fills the bias rows on the host). */
int vgx_step_begin(const void *ring, int64_t n_slots, int64_t slot_bytes, int32_t *counter, int32_t *step, int64_t *ids,
                   int64_t B, int64_t *out_ref, int32_t *tok_cur, int64_t tok_ld, int32_t *seg_cur, int32_t *ctrl,
                   const uint8_t *tiers, int64_t vocab, int64_t seg_min, int64_t seg_max, int64_t window,
                   float *bias_early, float *bias_late, int64_t n_heads, int64_t bias_ld, int64_t bias_cap,
                   void *stream);

/* vgx_step_begin followed, in the same launch, by the embedding rows of the ids it wrote:
 * emb_out[b * emb_ldo + c] = row ids[b] of the packed embedding table emb_packed (emb_rows x emb_cols
 * of emb_dtype; out-of-range ids take row 0), as vgx_embed_rows with pad row 0.  One launch instead
 * of two at the start of a decode step.  emb_packed NULL: vgx_step_begin.  Replaces the step's
 * embedding lookup after its ids (embed_row, runtime/vault3.c:626-654; nn.Embedding,
 * src/vault_v3_model.py:2285). */
int vgx_step_begin_embed(const void *ring, int64_t n_slots, int64_t slot_bytes, int32_t *counter, int32_t *step,
                         int64_t *ids, int64_t B, int64_t *out_ref, int32_t *tok_cur, int64_t tok_ld, int32_t *seg_cur,
                         int32_t *ctrl, const uint8_t *tiers, int64_t vocab, int64_t seg_min, int64_t seg_max,
                         int64_t window, float *bias_early, float *bias_late, int64_t n_heads, int64_t bias_ld,
                         int64_t bias_cap, int emb_dtype, const void *emb_packed, int64_t emb_rows, int64_t emb_cols,
                         float *emb_out, int64_t emb_ldo, void *stream);

/* The segment-bank update at a chunk boundary, for the evicted chunk ev_chunk (its tokens' scores
 * sc_prev, local segment ids seg_prev, tokens tok_prev, window entries each): quarantine (a score
 * <= -1e29 sets its whole segment to -1e30, written back), per-segment maximum, candidates t >= t0
 * (t0 = the pinned count for chunk 0) scored max - 1e-6 (global segment id mod 16384), then the top
 * `budget` of bank + candidates by (score desc, position asc), kept in chronological order.  The bank
 * arrays (mem_pos int64, mem_score fp32, mem_tok / mem_seg int32, capacity >= budget) and the control
 * words are updated in place; idx_old[j] / idx_new[j] (budget entries each) give new slot j's source
 * row in the old bank / the evicted chunk, -1 otherwise (for vgx_gather_rows_masked).  window + budget
 * <= 4096.  One workgroup; replaces update_segment_bank (runtime/vault3.c:1833-1915, quarantine
 * :2079-2088) and src/vault_v3_model.py:1858-1921 with merge_segment_bank_indices (:918-949). */
int vgx_seg_evict(float *sc_prev, const int32_t *seg_prev, const int32_t *tok_prev, int64_t window, int64_t *mem_pos,
                  float *mem_score, int32_t *mem_tok, int32_t *mem_seg, int32_t *ctrl, int64_t ev_chunk,
                  int64_t t0, int64_t budget, int32_t *idx_old, int32_t *idx_new, void *stream);

/* vgx_gather_rows, except that rows whose index is negative (or beyond src_rows) are left as they are
 * (the two-source bank compaction: old bank rows, then the evicted chunk's). */
int vgx_gather_rows_masked(int dtype, const void *src, void *dst, const int32_t *idx, int64_t n_idx, int64_t src_rows,
                           int64_t n_outer, int64_t src_ostride, int64_t dst_ostride, int64_t D, void *stream);

/* vgx_rope_rotate with the table row of row i at (i + row_base - *dyn) (table = the row of position
 * 0; negative rows lie before it), rows i >= *dyn skipped when limit_rows != 0: the re-rotation of the
 * segment keys to [-M, 0) and of the sinks to [-(M + S), -M) with the bank count M on the device
 * (src/vault_v3_model.py:1842-1856; runtime/vault3.c:859-896). */
int vgx_rope_rotate_dyn(int kv_dtype, const void *src, void *dst, int64_t n_outer, int64_t src_ostride,
                        int64_t dst_ostride, int64_t n_rows, int64_t D, const float *table, int64_t table_rstride,
                        const int32_t *dyn, int64_t row_base, int limit_rows, void *stream);

/* ---------------------------------------------------------------- token selection -------------- */

/* out[b] = the index of the largest of the V logits of row b (row stride ld), the first one on ties;
 * NaN logits are never selected.  Replaces v3_argmax (runtime/vault3.c:3198-3202). */
int vgx_argmax(const float *logits, int64_t ld, int64_t B, int64_t V, int64_t *out, void *stream);

/* Top-k sampling per row (k <= 64): the k largest logits (ties: the smaller index first), weights
 * exp((l_j - l_max) / temp), one draw of the row's xorshift64 state rng[b] (updated in place; 0 is
 * replaced by 0x9E3779B97F4A7C15): r = ((x >> 40) & 0xFFFFFF) / 2^24 * sum, the first j whose running
 * sum reaches r.  temp <= 0 or k <= 1 gives the argmax.  workspace: vgx_sample_topk_workspace_bytes.
 * Replaces v3_sample_topk (runtime/vault3.c:3204-3230). */
int64_t vgx_sample_topk_workspace_bytes(int64_t B, int64_t V);
int vgx_sample_topk(const float *logits, int64_t ld, int64_t B, int64_t V, int64_t k, float temp, uint64_t *rng,
                    int64_t *out, void *workspace, int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- segment-memory scorer -------- */

/* Causal EMA habituation of scorer features over T tokens (rows t*ldf of f, fd features each):
 * hab[t] = f[t] - 0.65 e, then e = 0.985 e + 0.015 f[t]; e starts from ema (or f[0] when first != 0,
 * which also skips the first update) and is stored back into ema.
 * Replaces _score_chunk_habituated (src/vault_v3_model.py:1224-1247) and the EMA of step (:2299-2304). */
int vgx_ema_habituate(const float *f, int64_t ldf, float *hab, int64_t ldh, float *ema, int64_t T, int64_t fd,
                      int first, void *stream);

/* LayerNorm rows: y = (x - mean) / sqrt(var + eps) * w + b (biased variance).
 * Replaces the scorer LayerNorm (src/vault_v3_model.py:879-880; runtime/vault3.c:963-971). */
int vgx_layernorm(const float *x, int64_t ldx, const float *w, const float *b, float *y, int64_t ldy, int64_t n_rows,
                  int64_t dim, float eps, void *stream);

/* Scorer tail for T tokens: h holds 2T rows of fc1 outputs (rows 0..T-1 raw features, T..2T-1
 * habituated).  out[t] = raw_t + 0.35 max(0, hab_t - raw_t), raw_t/hab_t = gelu_erf(h) . w2 + b2[0];
 * out[0] = raw_0 when first != 0.  out_index (may be NULL): device int32 added to out (a step
 * descriptor's VGX_STEP_SLOT, for the captured decode step).
 * Replaces src/vault_v3_model.py:881-883, 1238-1246, 2295-2305. */
int vgx_seg_score_tail(const float *h, int64_t ldh, const float *w2, const float *b2, int64_t hidden, int64_t T,
                       int first, float *out, const int32_t *out_index, void *stream);

/* The scorer of one decode token in two launches: the fc1 GEMV (w1: packed F32 [hidden, fd], bias b1)
 * on LayerNorm(feat) and LayerNorm(feat - 0.65 e) (ln_w, ln_b, eps; e = ema, or feat when first != 0),
 * both rows built inside the GEMV's workgroups, into h [2, hidden]; then out[0] (shifted by *out_index
 * when out_index is not NULL) as vgx_seg_score_tail at T = 1, and the EMA state updated as
 * vgx_ema_habituate at T = 1.  The same results as vgx_ema_habituate + vgx_layernorm + the fc1
 * vgx_qlinear + vgx_seg_score_tail, bit for bit.  fd <= 5120 (VGX_E_LIMIT beyond).
 * Replaces the step's scorer, src/vault_v3_model.py:2294-2305 (runtime/vault3.c:2201-2216). */
int vgx_seg_score_step(const float *feat, int64_t fd, float *ema, int first, const void *w1, int64_t hidden,
                       const float *b1, const float *ln_w, const float *ln_b, float eps, const float *w2,
                       const float *b2, float *h, float *out, const int32_t *out_index, void *stream);

/* One half of vgx_seg_score_step as a job that a GEMV launch can carry (vgx_qlinear_side).
 * phase 1: the fc1 GEMV on the two LayerNormed rows, into h; phase 2 (after phase 1): the score into
 * out[0] (shifted by *out_index) and the EMA update.  Phase 1 reads ema, phase 2 writes it. */
typedef struct vgx_score_side {
    int phase;
    const float *feat;          /* the token's features [fd], fd <= 5120 */
    int64_t fd;
    float *ema;                 /* the EMA state [fd] */
    int first;                  /* the stream's first token: e = feat, no EMA update */
    const void *w1;             /* packed F32 fc1 weight [hidden x fd] */
    int64_t hidden;
    const float *b1, *ln_w, *ln_b;
    float eps;
    const float *w2, *b2;       /* fc2 [hidden], bias [1] */
    float *h;                   /* [2][hidden]: written by phase 1, read by phase 2 */
    float *out;
    const int32_t *out_index;   /* may be NULL */
} vgx_score_side;

/* vgx_qlinear_ex, and the scorer job *side (may be NULL): when the GEMV runs the 16-wave pieces kernel
 * (batch 1, 192-320 blocks per row: the down projection of a decode step, which leaves a quarter of the
 * CUs idle) the job takes extra workgroups of the same launch; otherwise it is launched after the GEMV.
 * Results equal those of the separate calls bit for bit.  No counterpart in the reference: it removes
 * the scorer's launches from the decode step (src/vault_v3_model.py:2294-2305 is the computation). */
int vgx_qlinear_side(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                     int64_t batch, const float *norm_w, float eps, const float *bias, float *y, int64_t ldy,
                     int epilogue, const vgx_score_side *side, void *stream);

/* ---------------------------------------------------------------- top candidates of a row ------ */

/* The T (<= 256) largest logits of each row, sorted by value descending, ties by index ascending
 * (-0 ranks as +0; NaN logits are never candidates): idx[b * T + i], val[b * T + i]; rows with fewer
 * than T candidates are padded with index -1 and value -inf.  V up to 2^20.
 * workspace: vgx_topk_workspace_bytes.  For the output
 * governor's candidate screen (the top-k scans of v3_govern_logits, runtime/vault3.c:3133-3181). */
int64_t vgx_topk_workspace_bytes(int64_t B, int64_t V, int64_t T);
int vgx_topk(const float *logits, int64_t ld, int64_t B, int64_t V, int64_t T, int64_t *idx, float *val,
             void *workspace, int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- host control logic ----------- */
/* Host-side rules of the decode loop that read token byte strings; no device memory is involved.
 * Token ids are uint32 in [0, vocab); byte strings come from the VLT3 VTOK table. */

/* Token byte strings: token i is pool[offsets[i] .. offsets[i + 1]) (offsets has n_tokens + 1
 * entries, non-decreasing); ids >= n_tokens have no bytes.  The handle copies the data.
 * Replaces v3_token_bytes over the VTOK table (runtime/vault3.c:2303-2308). */
typedef struct vgx_tokens vgx_tokens;
vgx_tokens *vgx_tokens_create(const uint8_t *pool, const uint64_t *offsets, uint32_t n_tokens);
void vgx_tokens_destroy(vgx_tokens *t);

/* Segment-memory resonance for a state with seg_cap bank slots, window W and config n_sink.
 * vgx_res_rebuild: the tagged-shingle index over the bank's tokens (mem_tok, mem_seg: mem_cnt slots in
 * bank order); returns the number of distinct segments.  Replaces rebuild_shingle_index
 * (runtime/vault3.c:1178-1260; src/vault_v3_model.py:1249-1307).
 * vgx_res_update: one step's query resonance at ring slot c, absolute position pos, n_pin pinned
 * tokens; tok_prev / tok_cur are the W-slot token rings (tok_cur[c] = this step's token).  Returns the
 * mode (0: no bias, 1: arch / sup, 2: also hop1) and writes per bank slot (mem_cnt entries) the arch
 * and sup biases (mode >= 1) and the hop-1 bias (mode 2).  The biased heads are those with
 * h % grp >= grp / 3 of layers [L / 4, L - L / 14): hop1 in layers below L / 2 in mode 2, else arch
 * for h % grp < grp - (grp - grp / 3) / 2 and sup above.  Replaces update_query_resonance
 * (runtime/vault3.c:1426-1786) and _update_step_resonance (src/vault_v3_model.py:1685-1716). */
typedef struct vgx_resonance vgx_resonance;
vgx_resonance *vgx_res_create(const vgx_tokens *t, uint32_t window, uint32_t seg_cap, uint32_t n_sink,
                              uint32_t im_start_id, uint32_t im_end_id);
void vgx_res_destroy(vgx_resonance *r);
int vgx_res_rebuild(vgx_resonance *r, const uint32_t *mem_tok, const uint32_t *mem_seg, uint32_t mem_cnt);
int vgx_res_update(vgx_resonance *r, const uint32_t *tok_prev, const uint32_t *tok_cur, uint32_t c, uint64_t pos,
                   uint32_t n_pin, float *arch, float *sup, float *hop1);

/* Authority-spoof quarantine: 1 when the lower-cased bytes of the last min(24, pos - n_pin + 1)
 * tokens of the rings hold "opi_signed_directive" or "urgent opi delegation" (only with n_pin > n_sink
 * and pos >= n_pin); the step's segment score is then -1e30.  Replaces check_spoof_quarantine
 * (runtime/vault3.c:1798-1831) and _check_spoof_step (src/vault_v3_model.py:1795-1830). */
int vgx_spoof_check(const vgx_tokens *t, const uint32_t *tok_prev, const uint32_t *tok_cur, uint32_t window,
                    uint32_t c, uint64_t pos, uint32_t n_pin, uint32_t n_sink);

/* Output governor: up to 8 rules of 4..32 canonical bytes (Unicode look-alikes folded, separators
 * dropped); a candidate token is blocked when appending its bytes to the canonical history (or
 * decoding the raw tail plus its bytes as Base64 / hex) spells a rule forward or reversed.
 * vgx_gov_arm_system derives the rules from a system prompt (returns the rule count); vgx_gov_screen
 * takes the top candidates of a logits row (vgx_topk: value desc, index asc, at least 4 x top_k_guard
 * of them or the whole row) and returns the ids to set to -3.4e38, in up to four passes over the best
 * top_k_guard (0 or > 64: 64) still unmasked candidates; vgx_gov_commit feeds the chosen token (eos /
 * im_start / im_end reset the stream).  Replaces v3_gov_init, v3_gov_add_rule, v3_gov_arm_system,
 * v3_gov_reset_stream, v3_govern_logits, v3_gov_commit (runtime/vault3.c:2814-3193; vault3.h:180-216)
 * and CAAIGovernor (src/vault_v3_model.py:397-560). */
typedef struct vgx_governor vgx_governor;
vgx_governor *vgx_gov_create(const vgx_tokens *t, uint32_t eos_id, uint32_t im_start_id, uint32_t im_end_id);
void vgx_gov_destroy(vgx_governor *g);
void vgx_gov_reset_stream(vgx_governor *g);
int vgx_gov_add_rule(vgx_governor *g, const uint8_t *pat, size_t len);
int vgx_gov_arm_system(vgx_governor *g, const uint8_t *text, size_t len);
int vgx_gov_active(const vgx_governor *g);
int vgx_gov_screen(const vgx_governor *g, const int64_t *cand, const float *cand_val, uint32_t n_cand,
                   uint32_t top_k_guard, uint32_t vocab, int64_t *masked, uint32_t max_masked);
int vgx_gov_commit(vgx_governor *g, uint32_t id);

#ifdef __cplusplus
}
#endif

#endif /* VAULT_AMD_H */
