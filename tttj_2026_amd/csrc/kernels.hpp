// Internal launch functions shared by the C-ABI entry points and the forward executor.
#pragma once

#include "common.hpp"

namespace tt {

struct EpiArgs {
  const half* bias;      // [N]
  const half* resid;     // [M, ldy] (may alias y)
  const uint8_t* valid;  // [M] or nullptr
  half* y;
  int ldy;
  int mode;              // TT_EPI_*
  int batch, seq, heads, head_dim, d_model;  // TT_EPI_QKV only
  // TT_EPI_QKV: factor on the Q columns before their fp16 rounding.  The forward passes
  // hd^-1/2 log2(e), the form its attention launches read Q in (AttnArgs::q_prescaled).
  float q_scale = 1.f;
  // LayerNorm folded into this projection (TT_EPI_QKV / TT_EPI_BIAS_GELU, on the narrow and
  // small kernels): X is the raw residual stream, W = W diag(gamma), and the epilogue computes
  // rstd (acc - mean c) + b' instead of acc + bias.  The row statistics come from ln_slots
  // partial (mean, M2) slots per row (row stride ln_stride float2), each over K / ln_slots
  // columns.
  const float2* ln_part;  // [M][ln_stride] or nullptr
  const float* ln_colsum; // c [N]
  const float* ln_bias;   // b' [N]
  int ln_slots, ln_stride;
  // Producer side (residual modes): partial (mean, M2) slots of the values written, one per
  // stats_width columns (stats_width = linear_stats_width(...)), row stride ln_stride.
  float2* part_out;       // [M][ln_stride] or nullptr
  // Packed variable-length rows (MFMA tiles only): the live row count is *m_dev (<= the M the
  // launch is sized for), read on the device, so only the tiles of valid tokens run; and for
  // TT_EPI_QKV, rowmap[m] = {(b H S + s) hd, b H hd Sp + s} places packed row m, token (b, s), in
  // the Q / K and V^T planes.
  const int* m_dev;
  const int2* rowmap;
};

int launch_layernorm(const half* x, const half* gamma, const half* beta, const uint8_t* valid,
                     half* y, int rows, int d, float eps, hipStream_t stream);
// LayerNorm over packed variable-length rows: output row r reads input row in_row[r] (r itself
// without a map; a negative entry, or valid[r] == 0, writes +0.0), only rows r < *n_dev run (all
// `rows` without a count), and copy_out, if given, receives the gathered input row as well (+0.0
// for a negative entry).
int launch_layernorm_rows(const half* x, const half* gamma, const half* beta, const uint8_t* valid,
                          const int* in_row, const int* n_dev, half* copy_out, half* y, int rows,
                          int d, float eps, hipStream_t stream);

int launch_linear(const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                  hipStream_t stream);
// Columns per partial-statistics slot the GEMM launch_linear would run for this shape writes
// (the column range of one wave, or of one thread group on the narrow and small kernels).
int linear_stats_width(int m, int n, int k, int mode);
// Whether launch_linear runs this shape on the narrow (32 x 32) or small (vector-ALU) kernel.
bool linear_is_narrow(int m, int n, int k, int mode);

// Derived segments 12-17 of the packed weights (lnfold.hip).
int launch_pack_derived(half* w, int64_t stride, const int64_t* off, int D, int F, int L,
                        hipStream_t stream);

// info[b] = 1 + last valid position of sequence b, info[B + b] = whether its valid tokens form a
// prefix; counts (optional) [B] = valid tokens per sequence.
int launch_mask_info(const uint8_t* mask, int32_t* info, int batch, int seq, hipStream_t stream,
                     int32_t* counts = nullptr);

// Packed variable-length token maps of a masked batch (varlen.hip has the layout): writes *n_dev
// = the packed row count, row_tok[r] = b S + s of packed row r (-1 for rows that pad a sequence
// to 8), slot[b S + s] = its packed row or -1, rowmap[r] (EpiArgs::rowmap), pvalid[r] = whether
// packed row r is a valid token, and clears the Q / K / V^T entries of the padded tokens that
// the attention's tiles read (below the sequence's last key tile), which no packed QKV projection
// writes.  info is the mask_info of the same mask; counts holds its per-sequence valid counts.
int launch_varlen_maps(const uint8_t* mask, const int32_t* info, int32_t* counts, int32_t* n_dev,
                       int32_t* row_tok, int32_t* slot, int2* rowmap, uint8_t* pvalid, half* q,
                       half* k, half* vt, int B, int S, int H, int hd, hipStream_t stream);
// launch_mask_info (with counts) and launch_varlen_maps in one launch, one block per sequence
// (each scans the masks of the sequences before it); the two launches for batches whose scan
// would be long.
int launch_varlen_prep(const uint8_t* mask, int32_t* info, int32_t* counts, int32_t* n_dev,
                       int32_t* row_tok, int32_t* slot, int2* rowmap, uint8_t* pvalid, half* q,
                       half* k, half* vt, int B, int S, int H, int hd, hipStream_t stream);

// q_prescaled: q holds Q multiplied by attention_q_scale(head_dim) (the forward's QKV epilogue
// writes it so, EpiArgs::q_scale); otherwise the kernels multiply it when they load it.
int launch_attention(const half* q, const half* k, const half* vt, const uint8_t* mask,
                     const int32_t* info, half* ctx, int batch, int seq, int heads, int head_dim,
                     int causal, hipStream_t stream, bool q_prescaled = false,
                     const int* out_row = nullptr);
// hd^-1/2 log2(e): the factor of the scores in the exp2-domain softmax.
float attention_q_scale(int head_dim);
int attention_head_dim_supported(int head_dim);

struct AttnArgs;
// head_dim 256: the MFMA flash block with accumulators in AGPRs (attention_wide.hip).
int launch_attention_wide(const AttnArgs& args, const int32_t* info, int head_dim, int causal,
                          hipStream_t stream);
// head_dim 8 / 16: one lane per query, scores and P V on the vector ALUs (attention_small.hip).
int launch_attention_small(const AttnArgs& args, const int32_t* info, int head_dim, int causal,
                           hipStream_t stream);

// Byte offsets, in the megakernel's workspace, of the last layer's Q / K / V^T planes (the
// TT_EPI_QKV layout), attention context [T, D] and FFN hidden activations [T, F].
void megakernel_stage_offsets(int B, int S, int D, int F, int L, int64_t* qkv, int64_t* ctx,
                              int64_t* hidden);

// Persistent whole-model megakernel (megakernel.hip).  The workspace must be zero-filled before
// its first use and then reused unchanged between launches of the same shape.
size_t megakernel_workspace_bytes(int B, int S, int D, int F, int L);
int megakernel_supported(int B, int S, int D, int H, int F, int L);
int launch_megakernel(const half* weights, const int64_t off[TT_LAYER_SEGMENTS], int64_t stride,
                      int64_t final_off,
                      const half* x, const uint8_t* mask, half* y, char* workspace,
                      int64_t workspace_bytes, int B, int S, int D, int H, int F, int L, int causal,
                      uint64_t* trace, hipStream_t stream);
int megakernel_tasks(int B, int S, int D, int H, int F, int L);
int megakernel_status(const char* workspace, int B, int S, int D, int F, int L, int* status,
                      hipStream_t stream);
// Byte offset of the 32-bit error word (non-zero once a dependency wait gave up) in the workspace.
size_t megakernel_error_offset(int B, int S, int D, int F, int L);
// Zero the dependency counters and control words of a megakernel workspace with a fill kernel (no
// memset node, so the call may be captured into a graph); the next launch is then epoch 1.
int megakernel_reset(void* workspace, int64_t workspace_bytes, int B, int S, int D, int H, int F,
                     int L, hipStream_t stream);
// Store the address of a pinned host word into the workspace's control area (stream-ordered); at
// the end of every later launch the last workgroup writes the error flag there (0 or 1).
int megakernel_attach_status(void* workspace, int64_t workspace_bytes, int B, int S, int D, int H,
                             int F, int L, uint32_t* host_status, hipStream_t stream);
// Polls per dependency wait before it gives up, for later launches (< 0: the default).
void megakernel_set_spin_limit(int64_t limit);

// The whole forward (tt_transformer_fwd's body, forward.hip) on the given workspace; with
// reset_counters the megakernel plan first clears its dependency counters (a workspace shared
// with calls of other shapes).
int transformer_fwd(const void* weights, const void* x, const uint8_t* mask, void* y,
                    void* workspace, int64_t workspace_bytes, int batch, int seq, int d_model,
                    int num_heads, int ffn_dim, int num_layers, int causal, int plan,
                    bool reset_counters, void* stream);

// LayerNorm-prologue GEMM tiles (megakernel.hip): Y = LN(x) W^T + b for 64 x 64 tiles with the
// TT_EPI_QKV or TT_EPI_BIAS_GELU epilogue, D <= 512.
int ln_tile_supported(int D, int N);
int launch_ln_tile(const half* x, const half* gamma, const half* beta, const half* w,
                   const EpiArgs& ep, int B, int S, int D, int N, hipStream_t stream);

}  // namespace tt
