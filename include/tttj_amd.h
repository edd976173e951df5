/*
 * tttj_amd.h -- C ABI of the MI355X (gfx950) pre-LN transformer forward library.
 *
 * Every entry point takes raw device pointers, plain integer shapes and an explicit HIP stream
 * (passed as void*, i.e. the value of torch.cuda.current_stream().cuda_stream), returns an int
 * status (TT_OK = 0) and never throws.  On failure tt_last_error_string() describes the problem.
 * Activations and weights are IEEE fp16 (passed as void*), masks are one byte per token (a torch
 * bool tensor's storage: 0 = padded, non-zero = valid).  The library allocates no device memory:
 * callers pass every buffer, including the workspace.
 *
 * The reference exposes this path as Python/Triton functions and one pybind11 extension; each
 * declaration below names the reference interface it replaces (paths relative to the reference
 * repository root).
 */
#ifndef TTTJ_AMD_H
#define TTTJ_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define TT_OK 0
#define TT_ERR_INVALID 1 /* unsupported shape / bad argument, detected before any launch */
#define TT_ERR_HIP 2     /* a HIP runtime call or kernel launch failed */

/* Epilogues of tt_linear_fwd: Y = X W^T + b, then
 *   TT_EPI_BIAS           y = acc + b
 *   TT_EPI_BIAS_GELU      y = gelu_erf(acc + b)
 *   TT_EPI_RESID_MASKED   y = residual + (valid[row] ? acc + b : 0)      (attention out_proj)
 *   TT_EPI_MASKED_RESID   y = valid[row] ? residual + acc + b : 0         (ffn_out + block mask)
 *   TT_EPI_QKV            columns [0,D) -> Q [B,H,S,hd], [D,2D) -> K [B,H,S,hd],
 *                         [2D,3D) -> V^T [B,H,hd,Sp] with Sp = S rounded up to a multiple of
 *                         64 (y points at Q; K and V^T follow at offsets B*S*D and 2*B*S*D
 *                         elements; the V^T region holds B*D*Sp elements).  Needs batch/seq/heads.
 * `valid` may be NULL (all rows valid).  With `valid`, rows whose byte is 0 are written as +0.0
 * by TT_EPI_BIAS, TT_EPI_BIAS_GELU and TT_EPI_QKV (Q, K and V^T entries of that token), and a
 * tile whose rows are all masked does no MMA work (it only writes those fill values).  For the
 * non-QKV epilogues `seq` may be 0, or the rows per sequence: with `valid`, row tiles are then
 * visited in an order that spreads each sequence's padded tail over the XCDs (results unchanged).
 * `residual` may alias `y` (in-place update). */
#define TT_EPI_BIAS 0
#define TT_EPI_BIAS_GELU 1
#define TT_EPI_RESID_MASKED 2
#define TT_EPI_MASKED_RESID 3
#define TT_EPI_QKV 4

/* Library version string and the offload architecture it was built for. */
const char* tt_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char* tt_last_error_string(void);

/* Number of visible HIP devices (no kernel launch); <0 on error. */
int tt_device_count(void);

/* Packed fp16 weight layout.  Replaces the packing of kernels/sequence_resident.py:74-109 and the
 * offset table of kernels/fused_megakernel.py:28-44 (which assume F == D); generalised to any F.
 * Per layer, in this order, each segment starting on a 64-element boundary:
 *   0 norm1.weight[D]  1 norm1.bias[D]  2 Wqkv[3D,D] (q rows, k rows, v rows)  3 bqkv[3D]
 *   4 out_proj.weight[D,D]  5 out_proj.bias[D]  6 norm2.weight[D]  7 norm2.bias[D]
 *   8 ffn_in.weight[F,D]  9 ffn_in.bias[F]  10 ffn_out.weight[D,F]  11 ffn_out.bias[D]
 * and six segments derived from those by tt_pack_derived (the LayerNorms folded into the
 * projections that follow them):
 *   12 Wqkv'[3D,D] = Wqkv diag(norm1.weight)  13 cqkv[3D] fp32 = row sums of Wqkv'
 *   14 bqkv'[3D] fp32 = bqkv + Wqkv norm1.bias  15 W1'[F,D] = ffn_in.weight diag(norm2.weight)
 *   16 c1[F] fp32 = row sums of W1'  17 b1'[F] fp32 = ffn_in.bias + ffn_in.weight norm2.bias
 * (fp32 segments hold two fp16 slots per value), then final_norm.weight[D], final_norm.bias[D]
 * after the last layer.  Writes the TT_LAYER_SEGMENTS per-layer segment offsets (elements,
 * relative to the layer start), the layer stride, the final-norm offset and the total element
 * count. */
#define TT_LAYER_SEGMENTS 18
int tt_weight_layout(int d_model, int ffn_dim, int num_layers,
                     int64_t layer_offsets[TT_LAYER_SEGMENTS], int64_t* layer_stride,
                     int64_t* final_norm_offset, int64_t* total_elems);

/* Fill segments 12-17 of every layer of a packed weight buffer from its segments 0-11 (one kernel
 * launch on `stream`; call after the base segments are written and whenever they change).  With
 * LayerNorm y = (x - mean) rstd gamma + beta, LN(x) W^T + b = rstd (x W'^T - mean c) + b': the
 * layer-wise plan then multiplies the raw residual stream by W' and applies the per-row
 * statistics in the GEMM epilogue instead of launching a LayerNorm.  No counterpart in the
 * reference, which launches residual_layer_norm (kernels/case8_fusions.py:82-221) or fuses the
 * norm into its Triton tiles (kernels/case13_linear.py:179-259). */
int tt_pack_derived(void* weights, int d_model, int ffn_dim, int num_layers, void* stream);

/* Execution plans of tt_transformer_fwd. */
#define TT_PLAN_AUTO 0       /* the persistent megakernel for at most 64 tokens with d_model
                              * 256..512 (multiples of 64), ffn_dim a multiple of 64 and head_dim
                              * 32 or 64; else the fused-LN layer-wise plan for d_model <= 128
                              * (multiple of 64, ffn_dim too) and at most 2048 tokens; else
                              * layer-wise.  When AUTO resolves to the megakernel
                              * (tt_resolve_plan), its workspace rules apply: zero-filled before
                              * the first call and kept for that one shape. */
#define TT_PLAN_LAYERWISE 1  /* one launch per op: LN, GEMMs with fused epilogues, attention */
#define TT_PLAN_MEGAKERNEL 2 /* one persistent launch (<= one workgroup per CU) for the stack */
#define TT_PLAN_FUSED_LN 3   /* layer-wise with LN1 / LN2 computed inside the QKV / ffn_in GEMM
                              * tiles (five launches per layer; d_model <= 512) */

/* Bytes of workspace tt_transformer_fwd needs for this shape and plan.  The workspace of the
 * megakernel plan -- asked for, or picked by TT_PLAN_AUTO for few tokens (tt_resolve_plan says
 * which) -- holds its dependency counters and launch epoch: it must be zero-filled before its
 * first use and then passed unchanged to every later call with the same shape (one workspace per
 * shape; it is not re-entrant: calls that share it must be ordered on one stream).  Layer-wise
 * workspaces need no initial contents and may be shared by calls of any shape that fits.  Replaces the workspace
 * allocation of fused_megakernel_forward / dag_megakernel_forward
 * (kernels/fused_megakernel.py:1928-1937, kernels/dag_megakernel.py:2092-2097) and the persistent
 * scheduler buffer of SequenceResidentTransformer (kernels/sequence_resident.py:148-150). */
int tt_workspace_bytes(int batch, int seq, int d_model, int num_heads, int ffn_dim, int num_layers,
                       int plan, int64_t* bytes);

/* The plan TT_PLAN_AUTO resolves to for this shape (plan returned unchanged otherwise; AUTO
 * only picks a fused plan for shapes its kernels take); < 0 on bad arguments.  Replaces the case dispatch of optimized_transformer.py:45-93. */
int tt_resolve_plan(int batch, int seq, int d_model, int num_heads, int ffn_dim, int plan);

/* Health word of a megakernel workspace (synchronises `stream`): *status = 0 when every
 * dependency wait of every launch so far completed, 1 if some wait exceeded its bound (the
 * outputs of that launch and later ones are then invalid and the workspace must be zero-filled
 * again).  No counterpart in the reference, whose spin-waits are unbounded
 * (kernels/dag_megakernel.py:1355-1367). */
int tt_megakernel_status(const void* workspace, int batch, int seq, int d_model, int ffn_dim,
                         int num_layers, int* status, void* stream);

/* Byte offset, inside a megakernel workspace for this shape, of its 32-bit error word: 0 while
 * every dependency wait completed, non-zero once one gave up (then that launch wrote NaN over all
 * of y, and so does every later launch until the workspace is zero-filled again).  Lets a caller
 * copy the word asynchronously and check it later, without the stream synchronisation of
 * tt_megakernel_status.  No counterpart in the reference (its waits are unbounded,
 * kernels/dag_megakernel.py:1355-1367). */
int tt_megakernel_error_offset(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                               int num_layers, int64_t* offset);

/* Attach a host word to a megakernel workspace (after it is zero-filled; zero-filling detaches
 * it): at the end of every later launch on that workspace the last workgroup writes the error
 * flag (0 or 1) to *host_status, so a caller can check a launch's health by reading host memory,
 * without a stream synchronisation or an extra copy.  host_status must be device-accessible
 * pinned host memory (hipHostMalloc) that outlives the workspace's use, or NULL to detach.  The
 * attachment itself is a stream-ordered kernel on `stream`.  No counterpart in the reference. */
int tt_megakernel_attach_status(void* workspace, int64_t workspace_bytes, int batch, int seq,
                                int d_model, int num_heads, int ffn_dim, int num_layers,
                                int32_t* host_status, void* stream);

/* Test hook: polls per megakernel dependency wait (each poll followed by a one-step s_sleep)
 * before the wait gives up, for every later launch; limit < 0 restores the default (2^22).  A
 * small limit makes waits give up early while every wave still exits, which lets tests exercise
 * the error path.  Process wide, not thread-safe.  No counterpart in the reference. */
int tt_megakernel_set_spin_limit(int64_t limit);

/* Number of DAG tasks of the megakernel plan for this shape (<0 on bad arguments). */
int tt_megakernel_tasks(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                        int num_layers);

/* tt_transformer_fwd with the megakernel plan, also writing a per-task trace: 4 uint64 words per
 * task (task index | workgroup << 32, start, dependencies-satisfied, end; the times are the
 * 100 MHz s_memrealtime clock) into the device buffer `trace` of `trace_words` words
 * (>= 4 * tt_megakernel_tasks).  Replaces the CAPTURE trace slots of the reference's persistent
 * kernels (kernels/fused_megakernel.py:20-26, 224-238). */
int tt_megakernel_trace_fwd(const void* weights, const void* x, const uint8_t* mask, void* y,
                            void* workspace, int64_t workspace_bytes, int batch, int seq,
                            int d_model, int num_heads, int ffn_dim, int num_layers, int causal,
                            uint64_t* trace, int64_t trace_words, void* stream);

/* y[r] = LayerNorm(x[r]) * gamma + beta (eps, biased variance, fp32 statistics), fp16 out;
 * rows with valid[r] == 0 are written as +0.0 (valid may be NULL).  d % 8 == 0, d <= 8192.
 * Replaces residual_layer_norm / _residual_layer_norm_kernel (kernels/case8_fusions.py:82-256)
 * and the standalone LayerNorm of nn.LayerNorm in torch_transformer_benchmark.py:128,130,160. */
int tt_layernorm_fwd(const void* x, const void* gamma, const void* beta, const uint8_t* valid,
                     void* y, int rows, int d, float eps, void* stream);

/* Y[M,N] = X[M,K] W[N,K]^T + b with one of the TT_EPI_* epilogues; fp16 in/out, fp32 accumulate
 * on MFMA when K % 64 == 0 and N % 64 == 0, else (N, K multiples of 8, e.g. d_model 32) on a
 * small vector-ALU kernel with the same epilogues.  M * K may exceed 2^31; N * K may not.  For
 * TT_EPI_QKV, N == 3*D with D = heads*head_dim and M == batch*seq.  Replaces _linear_tile with EPILOGUE 0-3 (kernels/fused_megakernel.py:447-541),
 * linear_gelu (kernels/case13_linear.py:149-176), the packed-QKV F.linear
 * (kernels/layerwise_hybrid.py:188-192) and _head_major_qkv_kernel (case13_linear.py:114-146). */
int tt_linear_fwd(const void* x, const void* w, const void* bias, const void* residual,
                  const uint8_t* valid, void* y, int m, int n, int k, int epilogue, int batch,
                  int seq, int heads, void* stream);

/* Test hook: force tile configuration `index` (0: 256x256 on 8 waves, 1: 256x128, 2: 128x128,
 * 3: 128x64, 4: 64x64, 5: 32x32 narrow tiles with K split over the block's waves; 6-9: 128x256,
 * 128x128, 128x64, 256x128 staged through registers; 10: 256x128 on 8 waves with a three-stage
 * K ring) for every later GEMM whose N it divides; -1 restores the automatic choice.  Process
 * wide, not thread-safe.  No counterpart in the reference (its tile choices are compile-time
 * constants per case, kernels/fused_megakernel.py:121-171). */
int tt_gemm_tile_override(int index);

/* Per-sequence mask summary used by the attention and GEMM kernels: info[b] = 1 + index of the
 * last valid token of sequence b (0 if none), info[batch + b] = 1 if the valid tokens of b form a
 * prefix.  mask may be NULL (then every sequence is a full prefix).  Replaces the host-side
 * all-valid check of kernels/sequence_resident.py:172-192 without a host synchronisation. */
int tt_mask_info(const uint8_t* mask, int32_t* info, int batch, int seq, void* stream);

/* Flash attention over the TT_EPI_QKV layout: q, k [B,H,S,hd], vt [B,H,hd,Sp] -> ctx [B,S,H*hd]
 * token-major.  softmax(q k^T * hd^-0.5) with keys masked when (causal && key > query) or
 * mask[b,key] == 0; padded query rows are written as +0.0.  hd in {8, 16, 32, 64, 128, 256}
 * (8 / 16 on the vector ALUs with fp32 probabilities, the others on MFMA).  `info` is the
 * tt_mask_info output for the same mask (may be NULL only if mask is NULL).  Replaces
 * _attention_mxhd (kernels/fused_megakernel.py:544-790) and packed_causal_attention
 * (kernels/case8_attention.py:48-206), and BaselineSelfAttention's score/softmax/PV
 * (torch_transformer_benchmark.py:97-117). */
int tt_attention_fwd(const void* q, const void* k, const void* vt, const uint8_t* mask,
                     const int32_t* info, void* ctx, int batch, int seq, int heads, int head_dim,
                     int causal, void* stream);

/* 1 if tt_transformer_fwd with a mask runs this shape on packed variable-length rows, 0 if it
 * runs every token (padded rows skipped per tile), < 0 on bad arguments.  Packed rows: the valid
 * tokens of every sequence, in order, become the rows of the residual stream, the LayerNorm
 * output, the attention context and the FFN hidden activations (a right-padded sequence of l
 * valid tokens takes min(l rounded up to 8, S) rows, any other mask its valid count), and the
 * LayerNorms and GEMMs run over those rows only; the row count stays on the device.  Taken by
 * the layer-wise plan when all four projections run on MFMA tiles.  No counterpart in the
 * reference, which masks padded rows but computes them (kernels/fused_megakernel.py:628-638);
 * its prefix-length extraction is kernels/case14_hybrid.py:645-669. */
int tt_forward_packs_rows(int batch, int seq, int d_model, int num_heads, int ffn_dim, int plan);

/* Test hook: 0 makes every later masked forward run all tokens (no packed rows), -1 restores the
 * automatic choice.  Process wide, not thread-safe.  No counterpart in the reference. */
int tt_forward_packing_override(int enable);

/* tt_attention_fwd with q already multiplied by hd^-1/2 log2(e) and rounded to fp16 once -- the
 * form the forward's QKV projection writes (tt_stage_offsets) and its attention launches read:
 * ctx = softmax_2(q k^T) v with the same masks.  Replaces the same reference functions as
 * tt_attention_fwd, for callers that fold the softmax scale into their Q projection. */
int tt_attention_fwd_prescaled(const void* q, const void* k, const void* vt, const uint8_t* mask,
                               const int32_t* info, void* ctx, int batch, int seq, int heads,
                               int head_dim, int causal, void* stream);

/* Where a forward's intermediates of its LAST layer are left in the workspace, for per-stage checks
 * of the fused plans (the megakernel's tasks and the fused-LN tiles never materialise LN1 / LN2 or
 * the other stages on their own): byte offsets of the Q / K / V^T planes (the TT_EPI_QKV layout;
 * Q is stored multiplied by hd^-1/2 log2(e), the form the attention kernels read), of the attention
 * context [B,S,D] (-1 when the plan overwrites it with the LN2 output) and of the FFN hidden
 * activations GELU(LN2(x') W1^T + b1) [B,S,F] (in packed-row order, see tt_forward_packs_rows,
 * after a masked forward that packs rows).  Same arguments as tt_workspace_bytes.  Replaces the
 * stage CAPTURE of the reference's fused kernels (kernels/csrc/sequence_resident.cu:30-39,
 * kernels/fused_megakernel.py:224-238), compared against eager in
 * benchmarks/benchmark_steps_1_2.py:73-117. */
int tt_stage_offsets(int batch, int seq, int d_model, int num_heads, int ffn_dim, int num_layers,
                     int plan, int64_t* qkv, int64_t* ctx, int64_t* hidden);

/* Whole forward of the block stack + final norm:
 *   y = mask(final_norm(block_L(...block_1(x)))), block(x) = mask(x' + W2 gelu(W1 LN2(x') + b1)
 *   + b2) with x' = x + mask(Wo attn(LN1 x) + bo)
 * over the packed weights of tt_weight_layout.  x, y [B,S,D] fp16 (y must not alias x), mask
 * [B,S] bytes or NULL.  `plan` is one of TT_PLAN_*: the layer-wise plan launches LN, the four
 * GEMMs and attention per layer; the megakernel plan runs every layer in one launch of at most
 * one workgroup per CU, whose workgroups hand work to each other through dependency counters
 * (it relies on all of them being resident, i.e. on the device not being shared with other
 * kernels while it runs; its waits are bounded, see tt_megakernel_status).  Replaces
 * LayerwiseHybridTransformer.forward (kernels/layerwise_hybrid.py:255-361),
 * SequenceResidentTransformer.run (kernels/sequence_resident.py:158-225), fused_megakernel_forward
 * (kernels/fused_megakernel.py:1860-2001) and dag_megakernel_forward
 * (kernels/dag_megakernel.py:2060-2138). */
int tt_transformer_fwd(const void* weights, const void* x, const uint8_t* mask, void* y,
                       void* workspace, int64_t workspace_bytes, int batch, int seq, int d_model,
                       int num_heads, int ffn_dim, int num_layers, int causal, int plan,
                       void* stream);

/* Size in bytes of the scratch array tt_transformer_fwd_noalloc works in (64 MiB). */
int tt_noalloc_scratch_bytes(int64_t* bytes);

/* tt_transformer_fwd without a workspace argument and without any allocation.  No counterpart in
 * the reference: it exists for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The intermediates live in a
 * fixed scratch array of the library (tt_noalloc_scratch_bytes, 64 MiB), one per GPU, which the
 * runtime allocates when the library's code object is loaded on that GPU and keeps until the
 * process ends; shapes that need more (tt_workspace_bytes) fail with TT_ERR_INVALID before any
 * launch.  Same arguments, plans and results as tt_transformer_fwd.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, threads) race on it, so order
 * them on one stream.  The megakernel plan clears its dependency counters at the start of each
 * call (a fill kernel, no memset), which also clears the previous call's error word: read it with
 * tt_noalloc_status before the next call. */
int tt_transformer_fwd_noalloc(const void* weights, const void* x, const uint8_t* mask, void* y,
                               int batch, int seq, int d_model, int num_heads, int ffn_dim,
                               int num_layers, int causal, int plan, void* stream);

/* Health of the latest tt_transformer_fwd_noalloc call on the current device (synchronises
 * `stream`): *status = 0 when it ran a layer-wise plan or every dependency wait of its megakernel
 * launch completed, 1 if a wait gave up (that call wrote NaN over all of y).  Read it after the
 * call and before the next one, whose counter reset clears the word.  No counterpart in the
 * reference (its waits are unbounded, kernels/dag_megakernel.py:1355-1367); the no-alloc entry
 * point itself exists for callers that cannot allocate (graph capture, serving loops). */
int tt_noalloc_status(int* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TTTJ_AMD_H */
