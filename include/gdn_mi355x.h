/*
 * gdn_mi355x.h -- C ABI of the MI355X (gfx950) Gated DeltaNet layer path.
 *
 * One extern "C" entry point per kernel of the GDN path of nano-vllm-extend's
 * Qwen3.5 hybrid model.  Each entry point names the reference function it
 * replaces (paths relative to the reference repository root).
 *
 * Conventions (all entry points):
 *  - Every pointer is a device pointer.  bf16 tensors are passed as raw 16-bit
 *    words (`uint16_t`), fp32 as `float`, slot ids as int64 (torch.long).
 *  - Strides are in elements, not bytes.
 *  - `stream` is a hipStream_t (NULL = default stream).  Launches are
 *    asynchronous; nothing synchronises, allocates or keeps global state, so
 *    every entry point is safe under HIP-graph capture and reentrant.
 *  - Outputs are caller-allocated.  State pools are mutated in place where
 *    stated, exactly as the reference kernels mutate them.
 *  - Return value: 0 on success, GDN_ERR_* (< 0) for rejected arguments,
 *    or a positive hipError_t from the launch.
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 4

#define GDN_OK 0
#define GDN_ERR_INVALID_ARG (-1) /* shape / stride / pointer rejected */
#define GDN_ERR_UNSUPPORTED (-2) /* valid but not built (e.g. head dim) */
#define GDN_ERR_SCRATCH (-3)     /* needs more than the fixed scratch of an allocation-free entry point */

/* Bytes of the fixed device scratch array of gdn_conv_chunk_prefill_noalloc
 * (one per GPU, held until the process ends). */
#define GDN_NOALLOC_SCRATCH_BYTES (128LL << 20)

/* ABI version of the loaded library (GDN_ABI_VERSION). */
int gdn_abi_version(void);

/*
 * Fused gate/beta.  Replaces fused_g_beta / _gdn_g_beta_kernel
 * (nanovllm/models/qwen3_5.py:320-360) and its eager chain (:936-937, :982-992).
 *   g[i]    = -exp(A_log[h]) * softplus(a[i] + dt_bias[h])   (fp32, softplus
 *             threshold 20: z > 20 ? z : log(1 + exp(z)))
 *   beta[i] = sigmoid(b[i])                                 (bf16)
 * with h = i % Hv, i in [0, total).  If mask != NULL, g = 0 on rows
 * (i / Hv) whose mask byte is 0 (padding rows).
 * a, b: bf16 [total]; A_log, dt_bias: [Hv] in bf16 (param_is_fp32 = 0) or fp32 (1).
 */
int gdn_g_beta(const uint16_t* b, const uint16_t* a, const void* A_log, const void* dt_bias,
               int param_is_fp32, const uint8_t* mask, float* g, uint16_t* beta, int64_t total,
               int Hv, void* stream);

/*
 * Varlen causal depthwise conv1d + SiLU with in-place conv-state roll.
 * Replaces causal_conv_silu_varlen / _causal_conv_silu_varlen_kernel
 * (nanovllm/models/qwen3_5.py:402-473).
 *   x      [N, C] bf16, row stride sx_row, channel stride 1 (packed varlen rows)
 *   state  conv state of sequence r at state + row(r)*ss_seq + c*ss_ch + j,
 *          j in [0, K-1), row(r) = ids ? ids[r] : r.  Read as the K-1 left
 *          padding, then overwritten with the row's last K-1 raw inputs
 *          (old state entries when the row has fewer than K-1 tokens).
 *   w      [C, K] bf16 contiguous
 *   y      q / k / v parts: y[0 : N*key_dim) = [N, key_dim], then
 *          [N, key_dim], then [N, C - 2*key_dim].  With C == 3*key_dim this is
 *          the reference's [3, N, C/3] layout.
 *   lens, cu_start: int32 [n_seqs] (tokens and first packed row per sequence).
 */
int gdn_conv_varlen(const uint16_t* x, int64_t sx_row, uint16_t* state, int64_t ss_seq,
                    int64_t ss_ch, const int64_t* ids, const uint16_t* w, uint16_t* y,
                    int key_dim, const int32_t* lens, const int32_t* cu_start, int n_seqs,
                    int64_t N, int C, int K, void* stream);

/*
 * Single-token conv + SiLU with in-place state roll in the slot pool.
 * Replaces conv_decode_step / _conv_decode_step_kernel
 * (nanovllm/models/qwen3_5.py:515-558).
 *   y[b, c] = silu(x[b,c]*w[c,K-1] + sum_{i<K-1} s[i]*w[c,i]),  s = pool row ids[b]
 *   then s[i] <- s[i+1], s[K-2] <- x[b,c]   (pure bit copies)
 * x: [B, C] bf16 row stride sx_row; pool slot stride sp_slot, channel stride sp_ch,
 * state entries contiguous; y: [B, C] row stride sy_row.  Duplicate ids (the
 * CUDA-graph dummy slot) are tolerated: they race only on that slot.
 */
int gdn_conv_decode(const uint16_t* x, int64_t sx_row, uint16_t* pool, int64_t sp_slot,
                    int64_t sp_ch, const int64_t* ids, const uint16_t* w, uint16_t* y,
                    int64_t sy_row, int B, int C, int K, void* stream);

/*
 * Padded-batch conv + SiLU with per-row state writeback.
 * Replaces causal_conv_silu / _causal_conv_silu_kernel
 * (nanovllm/models/qwen3_5.py:249-317).
 *   x [n, C, T] with arbitrary strides; state [n, C, K-1] (strides ss_n, ss_c,
 *   entries contiguous); y [n, C, T] contiguous.  endp[r] in [-1, T]: the
 *   row's new state is its K-1 inputs before position endp[r]; -1 skips it.
 */
int gdn_conv_padded(const uint16_t* x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
                    uint16_t* state, int64_t ss_n, int64_t ss_c, const uint16_t* w,
                    uint16_t* y, const int32_t* endp, int n, int C, int T, int K,
                    void* stream);

/*
 * Chunked gated delta rule over packed varlen sequences (chunk size 64).
 * Replaces the fla chunk_gated_delta_rule call (nanovllm/models/qwen3_5.py:956-960,
 * semantics of the torch port _torch_chunk_gated_delta_rule :152-227).
 *   q, k  [N, Hk, D] bf16, token strides sq_tok / sk_tok, head stride D
 *   v     [N, Hv, D] bf16, token stride sv_tok, head stride D
 *   g     [N, Hv] fp32 contiguous; beta [N, Hv] bf16 contiguous
 *   value head h reads key head h / (Hv / Hk)   (grouped-value layout)
 *   cu_seqlens int64 [n_seqs + 1] (device)
 *   cu_seqlens_host  the same offsets in host memory, or NULL.  With them,
 *         when few workgroups would otherwise run (n_seqs * Hv * D/64 < 128),
 *         long sequences are cut into segments that run in parallel: the
 *         first segment from h0; each middle one as its zero-start result R
 *         and its transition P (the recurrence on the identity's columns);
 *         a scan S_{s+1} = P_s S_s + R_s (fp32); then the later segments
 *         again with outputs.  Same results up to rounding.
 *   max_segments  0 = automatic (segments of >= 16 chunks), 1 = never split,
 *         k >= 2 = up to k (at most 12) segments per sequence
 *   h0    initial state of sequence r at h0 + row(r)*state_stride, [Hv, D, D]
 *         fp32 dense; NULL = zero state.  hT likewise receives the final
 *         state (NULL = not written); row(r) = state_ids ? state_ids[r] : r.
 *         h0 == hT (in-place update of a slot pool) is allowed.
 *   o     [N, Hv, D] bf16 contiguous, 8-byte aligned; q, k, v 16-byte aligned
 *         with token strides a multiple of 8 and below 2^24 elements
 *   l2norm != 0: q, k rows are L2-normalised in fp32 (eps 1e-6) first.
 *   workspace: device buffer of at least gdn_chunk_prefill_workspace_size()
 *         bytes, 256-byte aligned, owned by the caller.  It receives one
 *         record of 19 KiB + 256 D bytes per (chunk, value head) from the
 *         first launch, then (segmented calls) the segment states; contents
 *         need no initialisation and are dead after the call.
 * D must be 64 or 128.  Two launches on `stream` (four when segmented): a prep kernel over all
 * chunks in parallel (row norms, K^T, K K^T, Q K^T, the triangular inverse),
 * then a state kernel per (sequence, value head, 64 value columns) that walks
 * the chunks in order with its state slice in registers (fp16 matrix-core
 * operands, fp32 accumulation and state).
 */
int gdn_chunk_prefill(const uint16_t* q, int64_t sq_tok, const uint16_t* k, int64_t sk_tok,
                      const uint16_t* v, int64_t sv_tok, const float* g, const uint16_t* beta,
                      const float* h0, float* hT, const int64_t* state_ids, int64_t state_stride,
                      const int64_t* cu_seqlens, const int64_t* cu_seqlens_host, int max_segments,
                      int n_seqs, int64_t N, int Hk, int Hv, int D,
                      float scale, int l2norm, uint16_t* o, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* Workspace bytes gdn_chunk_prefill needs for N packed tokens in n_seqs
 * sequences (an upper bound over the sequence lengths); -1 on bad args. */
int64_t gdn_chunk_prefill_workspace_size(int64_t N, int n_seqs, int Hv, int D);

/* Column split of the chunk prefills' state pass when no sequence is cut into
 * segments (no counterpart in the reference: a tuning and test control).  The
 * state's value columns are independent, so a sequence's heads can run in
 * workgroups of 64 columns (the default) or of 32, which finish each chunk
 * sooner but take twice the CUs; results are the same either way, bit for
 * bit.  mode 0 = the k longest sequences (k <= 4, from a list-schedule
 * estimate over the CUs) in 32-column workgroups, 1 = all in 64-column ones,
 * 2 = all in 32-column ones.  Process-wide; set it between calls.  Returns
 * GDN_ERR_INVALID_ARG for another mode. */
int gdn_set_column_split(int mode);

/*
 * Fused varlen prefill of the layer core's first three steps: gates, causal
 * conv1d + SiLU with the conv-state roll, and the chunked gated delta rule.
 * Replaces the sequence fused_g_beta (nanovllm/models/qwen3_5.py:934) ->
 * causal_conv_silu_varlen (:942-947) -> chunk_gated_delta_rule (:956-961) of
 * _gdn_prefill_varlen (:922-965), with the same results as the three entry
 * points above called in that order (gdn_g_beta, gdn_conv_varlen with
 * key_dim = Hk*D, gdn_chunk_prefill with l2norm), bit for bit.
 *   x      [N, C] bf16 raw q | k | v rows, C = 2*Hk*D + Hv*D, row stride
 *          sx_row (a multiple of 8, below 2^24), channel stride 1, 16-byte
 *          aligned
 *   conv_state, ss_seq, ss_ch, conv_w: as gdn_conv_varlen with K = 4; the
 *          pool row of sequence r is state_ids[r] (r if NULL), the same row
 *          as the recurrent state's
 *   b, a   [N, Hv] bf16 contiguous; A_log, dt_bias [Hv] (param_is_fp32 as
 *          gdn_g_beta; no padding mask)
 *   h0, hT, state_ids, state_stride, cu_seqlens, cu_seqlens_host, max_segments,
 *          scale, l2norm, o: as gdn_chunk_prefill
 *   fresh  uint8 [n_seqs] or NULL: fresh[r] != 0 runs sequence r from zero
 *          recurrent and conv states without reading its pool rows (the
 *          reference zeroes a fresh prefill's slot first, model_runner.py:305-322;
 *          this folds that into the call).  Its final states are written.
 *   workspace: at least gdn_conv_chunk_prefill_workspace_size() bytes,
 *          256-byte aligned (the chunk records, as gdn_chunk_prefill's)
 *   phase  3 = the whole call; 1 = the prep kernel only; 2 = the state pass
 *          only (after a phase-1 call with the same arguments and workspace,
 *          ordered after it on the caller's side: the two state calls of a
 *          split may run on different streams)
 *   select_host  uint8 [n_seqs] in host memory or NULL: the state pass runs
 *          only the selected sequences (needs cu_seqlens_host, n_seqs <= 64);
 *          each sequence's state pass, conv roll included, must run exactly once
 * Two launches, as gdn_chunk_prefill: the prep kernel also runs the gates and
 * the q and k channels' conv of its chunk; the state kernel runs the v
 * channels' conv and rolls the conv states.
 */
int gdn_conv_chunk_prefill(const uint16_t* x, int64_t sx_row, uint16_t* conv_state, int64_t ss_seq,
                           int64_t ss_ch, const uint16_t* conv_w, const uint16_t* b, const uint16_t* a,
                           const void* A_log, const void* dt_bias, int param_is_fp32, const float* h0,
                           float* hT, const int64_t* state_ids, const uint8_t* fresh, int64_t state_stride,
                           const int64_t* cu_seqlens, const int64_t* cu_seqlens_host, int max_segments,
                           int phase, const uint8_t* select_host, int n_seqs, int64_t N, int Hk, int Hv, int D,
                           float scale, int l2norm, uint16_t* o, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* Workspace bytes of gdn_conv_chunk_prefill; -1 on bad args. */
int64_t gdn_conv_chunk_prefill_workspace_size(int64_t N, int n_seqs, int Hv, int D);

/*
 * gdn_conv_chunk_prefill with no workspace argument and no allocation: its
 * records and segment scratch live in a fixed file-scope device array of
 * GDN_NOALLOC_SCRATCH_BYTES per GPU.  No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Arguments
 * as gdn_conv_chunk_prefill with phase = 3 (prep and state pass together) and
 * no select_host; it calls no hipMalloc / hipFree.  A call whose workspace
 * (gdn_conv_chunk_prefill_workspace_size) fits the array (128 MiB less 256
 * bytes: ~2,200 chunk-heads of records at D = 128, e.g. ~8,000 tokens at 16
 * value heads) runs as that entry point would, the same bits.  A larger one
 * runs as pieces in order on the stream, without segments: groups of whole
 * sequences whose records fit, and a sequence longer than the array holds as
 * token ranges of whole chunks, each starting from the state and conv taps
 * the range before it left in the pools (hT and conv_state) -- the same bits
 * as gdn_conv_chunk_prefill with max_segments = 1.  Pieces need
 * cu_seqlens_host, and token ranges need hT; without them a larger call
 * returns GDN_ERR_SCRATCH before any launch.  All calls on one GPU share the
 * array: calls that overlap on one GPU race; calls in order on a stream are
 * safe.
 */
int gdn_conv_chunk_prefill_noalloc(const uint16_t* x, int64_t sx_row, uint16_t* conv_state, int64_t ss_seq,
                                   int64_t ss_ch, const uint16_t* conv_w, const uint16_t* b, const uint16_t* a,
                                   const void* A_log, const void* dt_bias, int param_is_fp32, const float* h0,
                                   float* hT, const int64_t* state_ids, const uint8_t* fresh, int64_t state_stride,
                                   const int64_t* cu_seqlens, const int64_t* cu_seqlens_host, int max_segments,
                                   int n_seqs, int64_t N, int Hk, int Hv, int D, float scale, int l2norm,
                                   uint16_t* o, void* stream);

/*
 * Recurrent gated delta rule for decode: T >= 1 tokens per sequence, state
 * read once and written once.  Replaces recurrent_gdn_inplace /
 * _recurrent_inplace_kernel (nanovllm/models/qwen3_5.py:561-613, T = 1, in
 * place) and recurrent_gated_delta_rule -> fla fused_recurrent /
 * _torch_recurrent_gated_delta_rule (:230-238, :616-651, gathered state).
 * Per token: q,k L2-normalised (eps 1e-6), q *= scale, S *= exp(g),
 * delta = beta*(v - S^T k), S += k delta^T, o = S^T q.
 *   q, k  [B, T, Hk, D] bf16 with batch strides sq_b/sk_b and token strides
 *         sq_t/sk_t (head stride D); v [B, T, Hv, D] likewise
 *   g [B, T, Hv] fp32, beta [B, T, Hv] bf16, contiguous
 *   s_in  state of sequence b at s_in + row(b)*s_in_stride ([Hv, D, D] dense)
 *   s_out final state written at s_out + row(b)*s_out_stride (may equal s_in:
 *         in-place pool update); NULL = not written
 *   row(b) = ids ? ids[b] : b; with ids (or B > 1) both slot strides must
 *         be at least Hv*D*D (rows may not overlap), else GDN_ERR_INVALID_ARG
 *   inter [B, T, Hv, D, D] fp32 per-token states (NULL = not written)
 *   o     [B, T, Hv, D] bf16 contiguous
 *   src_states, src_accepted, src_T (src_states and src_accepted both NULL,
 *         or both set): deferred commit of a speculative-verify step.  Row b
 *         starts from src_states[b, src_accepted[b] - 1] (src_states the
 *         previous verify's per-token states [B, src_T, Hv, D, D], rows in
 *         the same order; src_accepted int64 [B]) when src_accepted[b] >= 1,
 *         else from its s_in row.  src_states may be this call's inter: each
 *         state is read before it is written.
 * Duplicate ids (dummy slot) are tolerated.  D must be 64 or 128.
 */
int gdn_recurrent(const uint16_t* q, int64_t sq_b, int64_t sq_t, const uint16_t* k,
                  int64_t sk_b, int64_t sk_t, const uint16_t* v, int64_t sv_b, int64_t sv_t,
                  const float* g, const uint16_t* beta, const float* s_in, int64_t s_in_stride,
                  float* s_out, int64_t s_out_stride, const int64_t* ids, float* inter,
                  uint16_t* o, int B, int T, int Hk, int Hv, int D, float scale, int l2norm,
                  const float* src_states, const int64_t* src_accepted, int src_T, void* stream);

/*
 * The decode step after the q/k conv, in one launch: the gates (as
 * gdn_g_beta), the conv1d + SiLU of the v channels with their conv-state roll
 * (as gdn_conv_decode), and the in-place recurrent update (as gdn_recurrent
 * with T = 1, s_in = s_out = s_pool).  Replaces fused_g_beta
 * (nanovllm/models/qwen3_5.py:345-360) and the v part of conv_decode_step
 * (:546-558) ahead of recurrent_gdn_inplace (:597-613) in the T == 1 branch
 * (:1008-1030), with the same results bit for bit.
 *   q, k   the decode conv's q and k outputs (gdn_conv_decode over the first
 *          2*Hk*D channels), row strides sq_b, sk_b, head dim contiguous; or
 *          both NULL with Hk == Hv: the q and k channels' decode conv and
 *          their conv-state roll run in the kernel too (whole heads per
 *          workgroup), the same bits as gdn_conv_decode on them first
 *   x      [B, C] raw rows (C = 2*Hk*D + Hv*D), row stride sx_row (multiple of 4)
 *   conv_pool, cp_slot, cp_ch, conv_w: as gdn_conv_decode with K = 4, over all
 *          C channels (only the v channels are read and rolled here)
 *   a, b   [B, Hv] bf16 contiguous; A_log, dt_bias [Hv] (param_is_fp32 as gdn_g_beta)
 *   s_pool, s_stride, ids, o, scale, l2norm: as gdn_recurrent (o [B, Hv, D])
 *   z, sz_b, norm_w, eps: with z != NULL the gated RMSNorm of the layer
 *          (Qwen3_5RMSNormGated, qwen3_5.py:1083-1085, :121-131) is applied in
 *          the same kernel and o receives its output instead of the core
 *          output, the same bits as gdn_rmsnorm_gated on that core output:
 *          z [B, Hv*D] bf16 gate rows (row stride sz_b), norm_w [D] bf16.
 *          The kernel then runs whole heads per workgroup, as it does without
 *          z from B*Hv >= 2048; below that it otherwise splits a head's
 *          columns over workgroups, which sums S^T k in another order
 * One launch; each v channel (and with q == k == NULL each q and k channel)
 * belongs to one workgroup, which rolls its taps.
 */
int gdn_recurrent_decode_fused(const uint16_t* q, int64_t sq_b, const uint16_t* k, int64_t sk_b,
                               const uint16_t* x, int64_t sx_row, uint16_t* conv_pool, int64_t cp_slot,
                               int64_t cp_ch, const uint16_t* conv_w, const uint16_t* a, const uint16_t* b,
                               const void* A_log, const void* dt_bias, int param_is_fp32, float* s_pool,
                               int64_t s_stride, const int64_t* ids, uint16_t* o, int B, int Hk, int Hv, int D,
                               float scale, int l2norm, const uint16_t* z, int64_t sz_b, const uint16_t* norm_w,
                               float eps, void* stream);

/*
 * Speculative-verify commit: pool[ids[b]] <- inter[b, accepted[b] - 1]
 * (accepted[b] in [1, T]; 0 leaves the slot untouched); slot_stride >=
 * Hv*D*D.  No counterpart in
 * the reference (spec decode is disabled for qwen3_5, nanovllm/config.py:84);
 * it consumes the per-token state format of gdn_recurrent.
 */
int gdn_state_commit(float* pool, int64_t slot_stride, const int64_t* ids, const float* inter,
                     const int32_t* accepted, int B, int T, int Hv, int D, void* stream);

/*
 * Measurement pass, no counterpart in the reference: every state tile
 * pool[ids[b], h] (D x D fp32) is read into registers and written back
 * unchanged, with the one-token decode kernel's tile layout, launch shape and
 * cache policy -- the decode step's state traffic without its arithmetic.
 * The pool's contents are left as they were (duplicate ids write identical
 * values).  slot_stride >= Hv*D*D.
 */
int gdn_state_tile_pass(float* pool, int64_t slot_stride, const int64_t* ids, int B, int Hv, int D,
                        void* stream);

/*
 * Measurement pass, no counterpart in the reference: gdn_state_tile_pass with
 * the tiles written to a second pool at the same offsets (dst[ids[b], h] =
 * src[ids[b], h]), the same launch shape and cache policy -- the out-of-place
 * form of the same traffic.  src and dst must not overlap; slot_stride >=
 * Hv*D*D for both.
 */
int gdn_state_tile_copy(const float* src, float* dst, int64_t slot_stride, const int64_t* ids, int B, int Hv,
                        int D, void* stream);

/*
 * The layer's projections: C = A B^T, bf16 operands, fp32 accumulation, bf16
 * result.  Replaces F.linear in ColumnParallelLinear / RowParallelLinear
 * (nanovllm/layers/linear.py:56-75, :133-158) at the GDN layer's in_proj_qkv,
 * in_proj_z, in_proj_b, in_proj_a (nanovllm/models/qwen3_5.py:929-939,
 * :1008-1010; one call over the four weights concatenated) and out_proj
 * (:964, :1086).
 *   A [M, K] row stride lda; B [N, K] (the nn.Linear weight) row stride ldb;
 *   C [M, N] row stride ldc.  K a multiple of 64; lda, ldb multiples of 8 and
 *   A, B 16-byte aligned (C rows go out in 16-byte pieces when ldc is a
 *   multiple of 8 and C 16-byte aligned, else element by element).
 *   g, beta, A_log, dt_bias, param_is_fp32, gate_col, Hv (g == NULL: none):
 *   the columns [gate_col, gate_col + Hv) of C are the b projection and
 *   [gate_col + Hv, gate_col + 2 Hv) the a projection; from their bf16 values
 *   beta [M, Hv] bf16 and g [M, Hv] fp32 are also written, as gdn_g_beta
 *   computes them (fused_g_beta, qwen3_5.py:345-360).
 */
int gdn_gemm_bf16(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, uint16_t* C, int64_t ldc, int M,
                  int N, int K, float* g, uint16_t* beta, const void* A_log, const void* dt_bias, int param_is_fp32,
                  int gate_col, int Hv, void* stream);

/*
 * gdn_gemm_bf16 with C's columns written to up to four separate tensors: part
 * s (of n_parts, 1..4) holds columns [col_end[s - 1], col_end[s]) (from 0) at
 * C[s], row stride ldc[s]; col_end increasing, multiples of 16 except the last,
 * which is N.  The same values as one C of N columns.  For the GDN layer's
 * in_proj over the four concatenated weights (the call sites of
 * nanovllm/models/qwen3_5.py:929-939, whose four projections each produce a
 * tensor of their own): qkv, z, b and a come out as separate contiguous
 * tensors, whose rows the prefill and the gated norm read faster than strided
 * columns of one [M, N] buffer, and which the gate readers take without a
 * copy.  Gate outputs as in gdn_gemm_bf16 (gate_col counts C's columns).
 */
int gdn_gemm_bf16_cols(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, int M, int N, int K,
                       int n_parts, uint16_t* const* C, const int64_t* ldc, const int* col_end, float* g,
                       uint16_t* beta, const void* A_log, const void* dt_bias, int param_is_fp32, int gate_col,
                       int Hv, void* stream);

/*
 * Gated RMSNorm on the value head dim.  Replaces Qwen3_5RMSNormGated /
 * _rms_gated_forward (nanovllm/models/qwen3_5.py:121-131, :697-709):
 *   y = bf16( float(bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))) * silu(float(z)) )
 * x, z: [n_tok, H, D] bf16 with token strides sx_tok / sz_tok (head stride D);
 * w [D] bf16; y [n_tok, H, D] contiguous.
 */
int gdn_rmsnorm_gated(const uint16_t* x, int64_t sx_tok, const uint16_t* z, int64_t sz_tok,
                      const uint16_t* w, uint16_t* y, int64_t n_tok, int H, int D, float eps,
                      void* stream);

/*
 * The gated norm over some token ranges only (the same arithmetic):
 * ranges int64 [3 * n_ranges] on the device, (first token, token count,
 * selected tokens before this range) each; n_sel_tok = all selected tokens.
 * x, z, y as gdn_rmsnorm_gated (y rows at the tokens' own positions), n_tok
 * rows each: a range token outside [0, n_tok) is skipped.  No reference
 * counterpart: it lets the norm of the sequences whose state pass ends early
 * run while the longest ones are still in the state kernel.
 */
int gdn_rmsnorm_gated_ranges(const uint16_t* x, int64_t sx_tok, const uint16_t* z, int64_t sz_tok,
                             const uint16_t* w, uint16_t* y, int64_t n_tok, const int64_t* ranges, int n_ranges,
                             int64_t n_sel_tok, int H, int D, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_MI355X_H */
