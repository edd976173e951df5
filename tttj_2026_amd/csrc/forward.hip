// Forward executor and the C-ABI bookkeeping entry points (layout, workspace, errors, version).
//
// tt_transformer_fwd runs the whole block stack in one C call on the caller's stream, so a
// forward costs one host->library crossing whatever the layer count:
//   mask_info (only with a mask)
//   per layer: LN1 -> QKV GEMM (head-major Q/K, transposed V) -> flash attention
//              -> out_proj GEMM (+bias, masked branch, residual)  -> LN2
//              -> ffn_in GEMM (+bias, exact GELU) -> ffn_out GEMM (+bias, residual, row mask)
//   final LN (+row mask) into y.
// The caller's x is read, never written; the residual stream lives in the workspace.
#include "common.hpp"
#include "kernels.hpp"

#include <cstdarg>
#include <cstring>
#include <mutex>

namespace tt {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

static int64_t align64(int64_t v) { return (v + 63) / 64 * 64; }
static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

struct Layout {
  int64_t off[TT_LAYER_SEGMENTS];
  int64_t stride, final_off, total;
};

// Segments 12-17 are derived from 0-11 (tt_pack_derived): the QKV and ffn_in weights with the
// LayerNorm gain folded in, W' = W diag(gamma) (fp16), their row sums c = sum_k W'[n, k] and the
// folded biases b' = b + W beta (both fp32, two halfs per value).
static Layout weight_layout(int64_t D, int64_t F, int64_t L) {
  const int64_t sizes[TT_LAYER_SEGMENTS] = {D, D, 3 * D * D, 3 * D, D * D, D, D, D, F * D, F, D * F,
                                            D, 3 * D * D, 6 * D, 6 * D, F * D, 2 * F, 2 * F};
  Layout lay{};
  int64_t o = 0;
  for (int i = 0; i < TT_LAYER_SEGMENTS; ++i) {
    lay.off[i] = o;
    o += align64(sizes[i]);
  }
  lay.stride = o;
  lay.final_off = L * o;
  lay.total = lay.final_off + 2 * align64(D);
  return lay;
}

struct Workspace {
  half *xa, *xn, *qkv, *hbuf;
  float2* part;   // partial row statistics of the residual stream, D / 4 slots per row at most
  int32_t* info;
  // packed variable-length rows (varlen.hip): valid counts per sequence, the packed row count,
  // packed row -> token, token -> packed row, and packed row -> Q / K and V^T offsets
  int32_t *vl_counts, *vl_n, *row_tok, *slot;
  int2* rowmap;
  uint8_t* pvalid;   // packed row -> valid token (0 for the rows that pad a sequence to 8)
  size_t off_xn, off_qkv, off_hbuf;  // byte offsets of xn, qkv and hbuf from the base
  size_t bytes;
};

static Workspace carve(char* base, int64_t B, int64_t S, int64_t D, int64_t F) {
  const int64_t T = B * S, Sp = (S + 63) / 64 * 64;
  Workspace w{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + o : nullptr;
    o += align256(bytes);
    return p;
  };
  w.xa = (half*)take(T * D * 2);
  w.off_xn = o;
  w.xn = (half*)take(T * D * 2);  // LN1 output of layer 0, then the attention context
  w.off_qkv = o;
  w.qkv = (half*)take((2 * T * D + B * D * Sp) * 2);
  w.off_hbuf = o;
  w.hbuf = (half*)take(T * F * 2);
  w.part = (float2*)take(T * (D / 4) * sizeof(float2));
  w.info = (int32_t*)take(2 * B * 4);
  w.vl_counts = (int32_t*)take(B * 4);
  w.vl_n = (int32_t*)take(4);
  w.row_tok = (int32_t*)take(T * 4);
  w.slot = (int32_t*)take(T * 4);
  w.rowmap = (int2*)take(T * sizeof(int2));
  w.pvalid = (uint8_t*)take(T);
  w.bytes = o;
  return w;
}

// Whether the layer-wise plan folds LN2 (and LN1 of layers >= 1) into the next projection: only
// where both QKV and ffn_in run on the narrow / small kernels (few tokens).
static bool folds_layernorm(bool fused_ln, int64_t T, int64_t D, int64_t F) {
  return !fused_ln && linear_is_narrow((int)T, (int)(3 * D), (int)D, TT_EPI_QKV) &&
         linear_is_narrow((int)T, (int)F, (int)D, TT_EPI_BIAS_GELU);
}

// Whether a masked layer-wise forward packs the valid tokens (varlen.hip): when the LayerNorms
// are not fused or folded and all four projections run on the MFMA tiles (the packed row count
// is read on the device by those kernels), and the Q / V^T planes stay below 2^31 elements.
static bool g_packing_off = false;  // test hook (tt_forward_packing_override)

static bool packs_rows(bool fused_ln, bool fold, int64_t B, int64_t S, int64_t D, int64_t H,
                       int64_t F) {
  const int64_t T = B * S, Sp = (S + 63) / 64 * 64;
  if (g_packing_off || fused_ln || fold || T * D >= (1LL << 31) || B * D * Sp >= (1LL << 31))
    return false;
  return !linear_is_narrow((int)T, (int)(3 * D), (int)D, TT_EPI_QKV) &&
         !linear_is_narrow((int)T, (int)D, (int)D, TT_EPI_RESID_MASKED) &&
         !linear_is_narrow((int)T, (int)F, (int)D, TT_EPI_BIAS_GELU) &&
         !linear_is_narrow((int)T, (int)D, (int)F, TT_EPI_MASKED_RESID) && H > 0;
}

static int check_model_shape(int B, int S, int D, int H, int F, int L) {
  TT_REQUIRE(B > 0 && S > 0 && D > 0 && H > 0 && F > 0 && L > 0,
             "transformer: non-positive shape B=%d S=%d D=%d H=%d F=%d L=%d", B, S, D, H, F, L);
  TT_REQUIRE(D % H == 0, "transformer: d_model %d not divisible by heads %d", D, H);
  const int rc = attention_head_dim_supported(D / H);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(D % 8 == 0 && F % 8 == 0, "transformer: d_model %d and ffn_dim %d must be multiples of 8", D, F);
  TT_REQUIRE(D <= 8192, "transformer: d_model %d > 8192", D);
  TT_REQUIRE((int64_t)B * S < (1LL << 31) / 8, "transformer: too many tokens");
  return TT_OK;
}

}  // namespace tt

using namespace tt;

// 0.2: 18 segments per layer in the packed weights (tt_pack_derived fills 12-17; the folded
// LayerNorm and megakernel paths read them), packed variable-length rows for masked batches.
extern "C" const char* tt_version(void) { return "tttj_amd 0.2 gfx950"; }

extern "C" const char* tt_last_error_string(void) { return g_last_error.c_str(); }

extern "C" int tt_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return -1;
  return n;
}

extern "C" int tt_weight_layout(int d_model, int ffn_dim, int num_layers,
                                int64_t layer_offsets[TT_LAYER_SEGMENTS], int64_t* layer_stride,
                                int64_t* final_norm_offset, int64_t* total_elems) {
  TT_REQUIRE(d_model > 0 && ffn_dim > 0 && num_layers > 0, "weight_layout: bad shape");
  const Layout lay = weight_layout(d_model, ffn_dim, num_layers);
  if (layer_offsets) memcpy(layer_offsets, lay.off, sizeof(lay.off));
  if (layer_stride) *layer_stride = lay.stride;
  if (final_norm_offset) *final_norm_offset = lay.final_off;
  if (total_elems) *total_elems = lay.total;
  return TT_OK;
}

extern "C" int tt_pack_derived(void* weights, int d_model, int ffn_dim, int num_layers,
                               void* stream) {
  TT_REQUIRE(weights != nullptr && d_model > 0 && ffn_dim > 0 && num_layers > 0,
             "pack_derived: bad arguments");
  const Layout lay = weight_layout(d_model, ffn_dim, num_layers);
  return launch_pack_derived((half*)weights, lay.stride, lay.off, d_model, ffn_dim, num_layers,
                             (hipStream_t)stream);
}

// Token count up to which the automatic plan runs the persistent megakernel (d_model >= 256).
// Measured on MI355X (same-process medians): C2 (B1 S64 D256 H8 F1024 L4) 88.7 us against 91.8
// for the layer-wise plan, whose back-to-back launches pipeline with almost no gap; C1 (B4 S128,
// 512 tokens) 60.5 against 60.0, so from there on the layer-wise plan stays the choice.
static constexpr int64_t kMegaMaxTokens = 64;
static constexpr int kMegaMinDModel = 256;
static constexpr int kMegaMaxDModel = 512;  // the megakernel keeps a LayerNorm'd 64 x D tile in LDS
// The automatic plan computes LN1 / LN2 inside the QKV / ffn_in 64 x 64 tiles (fewer launches on
// the latency-bound path) only for narrow models with few tokens: measured on MI355X, d_model 128
// gains up to 2048 tokens (the reference's cases 2-4: 94 / 92 / 102 us fused against 101 / 97 /
// 115 layer-wise) and loses from 8192 (case 1: 161 against 147 us); at d_model 256 the layer-wise
// plan with narrow GEMM tiles is as fast or faster (C1 68 / 68 us, C2 106 against 118 us).
static constexpr int64_t kFusedLnMaxTokens = 2048;
static constexpr int kFusedLnMaxDModel = 128;

// The automatic plan only picks a fused plan for shapes its kernels take (64-multiple d_model
// and ffn_dim; head_dim 32 / 64 for the megakernel); an explicit plan is returned as asked and
// the forward reports an unsupported shape as an error.
static int resolve_plan(int plan, int B, int S, int D, int H, int F) {
  if (plan != TT_PLAN_AUTO) return plan;
  const int64_t T = (int64_t)B * S;
  const bool tiles64 = D % 64 == 0 && F % 64 == 0 && D <= kMegaMaxDModel;
  const int hd = H > 0 ? D / H : 0;
  if (T <= kMegaMaxTokens && D >= kMegaMinDModel && tiles64 && (hd == 32 || hd == 64))
    return TT_PLAN_MEGAKERNEL;
  if (tiles64 && D <= kFusedLnMaxDModel && T <= kFusedLnMaxTokens) return TT_PLAN_FUSED_LN;
  return TT_PLAN_LAYERWISE;
}

extern "C" int tt_workspace_bytes(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                                  int num_layers, int plan, int64_t* bytes) {
  int rc = check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(bytes != nullptr, "workspace_bytes: null output");
  TT_REQUIRE(plan >= TT_PLAN_AUTO && plan <= TT_PLAN_FUSED_LN, "workspace_bytes: bad plan %d", plan);
  plan = resolve_plan(plan, batch, seq, d_model, num_heads, ffn_dim);
  if (plan == TT_PLAN_MEGAKERNEL) {
    if ((rc = megakernel_supported(batch, seq, d_model, num_heads, ffn_dim, num_layers)) != TT_OK)
      return rc;
    *bytes = (int64_t)megakernel_workspace_bytes(batch, seq, d_model, ffn_dim, num_layers);
  } else {
    *bytes = (int64_t)carve(nullptr, batch, seq, d_model, ffn_dim).bytes;
  }
  return TT_OK;
}

extern "C" int tt_stage_offsets(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                                int num_layers, int plan, int64_t* qkv, int64_t* ctx,
                                int64_t* hidden) {
  int rc = check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(qkv && ctx && hidden, "stage_offsets: null output");
  TT_REQUIRE(plan >= TT_PLAN_AUTO && plan <= TT_PLAN_FUSED_LN, "stage_offsets: bad plan %d", plan);
  plan = resolve_plan(plan, batch, seq, d_model, num_heads, ffn_dim);
  if (plan == TT_PLAN_MEGAKERNEL) {
    if ((rc = megakernel_supported(batch, seq, d_model, num_heads, ffn_dim, num_layers)) != TT_OK)
      return rc;
    megakernel_stage_offsets(batch, seq, d_model, ffn_dim, num_layers, qkv, ctx, hidden);
    return TT_OK;
  }
  const Workspace w = carve(nullptr, batch, seq, d_model, ffn_dim);
  *qkv = (int64_t)w.off_qkv;
  *hidden = (int64_t)w.off_hbuf;
  // the context buffer is overwritten by the LN2 output unless LN2 is fused or folded
  const bool fused_ln = plan == TT_PLAN_FUSED_LN;
  *ctx = (fused_ln || folds_layernorm(fused_ln, (int64_t)batch * seq, d_model, ffn_dim))
             ? (int64_t)w.off_xn
             : -1;
  return TT_OK;
}

extern "C" int tt_resolve_plan(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                               int plan) {
  if (plan < TT_PLAN_AUTO || plan > TT_PLAN_FUSED_LN || batch <= 0 || seq <= 0 || d_model <= 0 ||
      num_heads <= 0 || ffn_dim <= 0) {
    fail(TT_ERR_INVALID,
         "resolve_plan: bad arguments (batch=%d seq=%d d_model=%d heads=%d ffn=%d plan=%d)", batch,
         seq, d_model, num_heads, ffn_dim, plan);
    return -1;
  }
  return resolve_plan(plan, batch, seq, d_model, num_heads, ffn_dim);
}

extern "C" int tt_forward_packing_override(int enable) {
  TT_REQUIRE(enable == 0 || enable == -1, "forward_packing_override: %d is not 0 or -1", enable);
  g_packing_off = enable == 0;
  return TT_OK;
}

extern "C" int tt_forward_packs_rows(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                                     int plan) {
  if (check_model_shape(batch, seq, d_model, num_heads, ffn_dim, 1) != TT_OK) return -1;
  if (plan < TT_PLAN_AUTO || plan > TT_PLAN_FUSED_LN) {
    fail(TT_ERR_INVALID, "forward_packs_rows: bad plan %d", plan);
    return -1;
  }
  plan = resolve_plan(plan, batch, seq, d_model, num_heads, ffn_dim);
  if (plan == TT_PLAN_MEGAKERNEL) return 0;
  const bool fused_ln = plan == TT_PLAN_FUSED_LN;
  const int64_t T = (int64_t)batch * seq;
  return packs_rows(fused_ln, folds_layernorm(fused_ln, T, d_model, ffn_dim), batch, seq, d_model,
                    num_heads, ffn_dim)
             ? 1
             : 0;
}

extern "C" int tt_megakernel_trace_fwd(const void* weights, const void* x, const uint8_t* mask,
                                       void* y, void* workspace, int64_t workspace_bytes,
                                       int batch, int seq, int d_model, int num_heads, int ffn_dim,
                                       int num_layers, int causal, uint64_t* trace,
                                       int64_t trace_words, void* stream) {
  int rc = check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(weights && x && y && workspace && trace, "megakernel_trace_fwd: null pointer");
  TT_REQUIRE(x != y, "megakernel_trace_fwd: y must not alias x");
  const int64_t need = 4LL * megakernel_tasks(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  TT_REQUIRE(trace_words >= need, "megakernel_trace_fwd: trace holds %lld words, need %lld",
             (long long)trace_words, (long long)need);
  const Layout lay = weight_layout(d_model, ffn_dim, num_layers);
  return launch_megakernel((const half*)weights, lay.off, lay.stride, lay.final_off,
                           (const half*)x, mask, (half*)y, (char*)workspace, workspace_bytes,
                           batch, seq, d_model, num_heads, ffn_dim, num_layers, causal,
                           trace, (hipStream_t)stream);
}

extern "C" int tt_megakernel_tasks(int batch, int seq, int d_model, int num_heads, int ffn_dim,
                                   int num_layers) {
  if (check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers) != TT_OK) return -1;
  return megakernel_tasks(batch, seq, d_model, num_heads, ffn_dim, num_layers);
}

extern "C" int tt_megakernel_status(const void* workspace, int batch, int seq, int d_model,
                                    int ffn_dim, int num_layers, int* status, void* stream) {
  TT_REQUIRE(workspace != nullptr && status != nullptr, "megakernel_status: null pointer");
  return megakernel_status((const char*)workspace, batch, seq, d_model, ffn_dim, num_layers, status,
                           (hipStream_t)stream);
}

namespace tt {

// Layer-wise forward over packed variable-length rows (varlen.hip has the layout): LayerNorms
// and GEMMs run over the n packed rows only (n read on the device), the QKV epilogue scatters
// packed rows into the token layout of Q / K / V^T, the attention stores each valid token's
// context at its packed row, and the final LayerNorm scatters back to [B, S, D] with +0.0 for
// padded tokens.  Seven launches per layer, as the padded plan.
static int forward_packed(const half* wts, const Layout& lay, const half* x, const uint8_t* mask,
                          half* y, const Workspace& ws, const int32_t* info, int B, int S, int D,
                          int H, int F, int L, int causal, hipStream_t stream) {
  const int T = B * S, hd = D / H;
  const size_t plane = (size_t)T * D;
  half* q = ws.qkv;
  half* k = ws.qkv + plane;
  half* vt = ws.qkv + 2 * plane;
  int rc;
  for (int l = 0; l < L; ++l) {
    const half* w = wts + (size_t)l * lay.stride;
    // LN1; in the first layer it also gathers the valid tokens of x into the packed residual
    // stream (rows that pad a sequence to 8 get +0.0)
    if (l == 0)
      rc = launch_layernorm_rows(x, w + lay.off[0], w + lay.off[1], nullptr, ws.row_tok, ws.vl_n,
                                 ws.xa, ws.xn, T, D, 1e-5f, stream);
    else
      rc = launch_layernorm_rows(ws.xa, w + lay.off[0], w + lay.off[1], nullptr, nullptr, ws.vl_n,
                                 nullptr, ws.xn, T, D, 1e-5f, stream);
    if (rc != TT_OK) return rc;
    EpiArgs ep{};
    ep.bias = w + lay.off[3];
    ep.y = q;
    ep.ldy = 3 * D;
    ep.mode = TT_EPI_QKV;
    ep.batch = B;
    ep.seq = S;
    ep.heads = H;
    ep.head_dim = hd;
    ep.d_model = D;
    ep.q_scale = attention_q_scale(hd);
    ep.m_dev = ws.vl_n;
    ep.rowmap = ws.rowmap;
    ep.valid = ws.pvalid;  // rows that pad a sequence to 8 write +0.0, as padded tokens do
    if ((rc = launch_linear(ws.xn, w + lay.off[2], T, 3 * D, D, ep, stream)) != TT_OK) return rc;
    if ((rc = launch_attention(q, k, vt, mask, info, ws.xn, B, S, H, hd, causal, stream, true,
                               ws.slot)) != TT_OK)
      return rc;
    ep = EpiArgs{};
    ep.bias = w + lay.off[5];
    ep.resid = ws.xa;
    ep.y = ws.xa;
    ep.ldy = D;
    ep.mode = TT_EPI_RESID_MASKED;
    ep.m_dev = ws.vl_n;
    if ((rc = launch_linear(ws.xn, w + lay.off[4], T, D, D, ep, stream)) != TT_OK) return rc;
    if ((rc = launch_layernorm_rows(ws.xa, w + lay.off[6], w + lay.off[7], nullptr, nullptr,
                                    ws.vl_n, nullptr, ws.xn, T, D, 1e-5f, stream)) != TT_OK)
      return rc;
    ep = EpiArgs{};
    ep.bias = w + lay.off[9];
    ep.y = ws.hbuf;
    ep.ldy = F;
    ep.mode = TT_EPI_BIAS_GELU;
    ep.m_dev = ws.vl_n;
    if ((rc = launch_linear(ws.xn, w + lay.off[8], T, F, D, ep, stream)) != TT_OK) return rc;
    ep = EpiArgs{};
    ep.bias = w + lay.off[11];
    ep.resid = ws.xa;
    ep.y = ws.xa;
    ep.ldy = D;
    ep.mode = TT_EPI_MASKED_RESID;
    ep.m_dev = ws.vl_n;
    if ((rc = launch_linear(ws.hbuf, w + lay.off[10], T, D, F, ep, stream)) != TT_OK) return rc;
  }
  return launch_layernorm_rows(ws.xa, wts + lay.final_off, wts + lay.final_off + align64(D), mask,
                               ws.slot, nullptr, nullptr, y, T, D, 1e-5f, stream);
}

// The forward on a workspace the caller provides (tt_transformer_fwd) or on the library's own
// scratch array (tt_transformer_fwd_noalloc, which clears the megakernel's counters first).
int transformer_fwd(const void* weights, const void* x, const uint8_t* mask, void* y,
                           void* workspace, int64_t workspace_bytes, int batch, int seq,
                           int d_model, int num_heads, int ffn_dim, int num_layers, int causal,
                           int plan, bool reset_counters, void* stream_) {
  int rc = check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(weights && x && y && workspace, "transformer: null pointer");
  TT_REQUIRE(x != y, "transformer: y must not alias x");
  TT_REQUIRE(plan >= TT_PLAN_AUTO && plan <= TT_PLAN_FUSED_LN, "transformer: bad plan %d", plan);
  const int B = batch, S = seq, D = d_model, H = num_heads, F = ffn_dim, L = num_layers;
  const int T = B * S, hd = D / H;
  if (resolve_plan(plan, B, S, D, H, F) == TT_PLAN_MEGAKERNEL) {
    const Layout lay = weight_layout(D, F, L);
    if (reset_counters &&
        (rc = megakernel_reset(workspace, workspace_bytes, B, S, D, H, F, L,
                               (hipStream_t)stream_)) != TT_OK)
      return rc;
    return launch_megakernel((const half*)weights, lay.off, lay.stride, lay.final_off,
                             (const half*)x, mask, (half*)y, (char*)workspace, workspace_bytes, B,
                             S, D, H, F, L, causal, nullptr, (hipStream_t)stream_);
  }
  Workspace ws = carve((char*)workspace, B, S, D, F);
  TT_REQUIRE((int64_t)ws.bytes <= workspace_bytes, "transformer: workspace %lld < %zu bytes",
             (long long)workspace_bytes, ws.bytes);
  const hipStream_t stream = (hipStream_t)stream_;
  const Layout lay = weight_layout(D, F, L);
  const half* wts = (const half*)weights;
  const size_t plane = (size_t)T * D;
  half* q = ws.qkv;
  half* k = ws.qkv + plane;
  half* vt = ws.qkv + 2 * plane;
  // TT_PLAN_FUSED_LN: LN1 / LN2 are computed inside the QKV / ffn_in tiles (launch_ln_tile), five
  // launches per layer instead of seven.
  const bool fused_ln = resolve_plan(plan, B, S, D, H, F) == TT_PLAN_FUSED_LN;
  if (fused_ln && ((rc = ln_tile_supported(D, 3 * D)) != TT_OK || (rc = ln_tile_supported(D, F)) != TT_OK))
    return rc;
  const bool packed = mask != nullptr && packs_rows(fused_ln, folds_layernorm(fused_ln, T, D, F),
                                                    B, S, D, H, F);
  const int32_t* info = nullptr;
  if (packed) {
    if ((rc = launch_varlen_prep(mask, ws.info, ws.vl_counts, ws.vl_n, ws.row_tok, ws.slot,
                                 ws.rowmap, ws.pvalid, q, k, vt, B, S, H, hd, stream)) != TT_OK)
      return rc;
    return forward_packed(wts, lay, (const half*)x, mask, (half*)y, ws, ws.info, B, S, D, H, F, L,
                          causal, stream);
  }
  if (mask != nullptr) {
    if ((rc = launch_mask_info(mask, ws.info, B, S, stream)) != TT_OK) return rc;
    info = ws.info;
  }
  // Layer-wise plan: LN2 of every layer and LN1 of layers >= 1 are folded into the projection
  // that follows them (lnfold.hip): the producer of the residual stream (out_proj, ffn_out)
  // writes partial row statistics in its epilogue, and the QKV / ffn_in GEMMs multiply the raw
  // residual stream by W' = W diag(gamma) and apply rstd (acc - mean c) + b'.  Layer 0's LN1 (the
  // input has no producer here) and the final norm stay standalone launches.
  const int ldp = D / 4;     // float2 slots per row of ws.part (the narrowest producer: 4 columns)
  int part_slots = 0;        // slots per row the last producer wrote
  // The fold pays only where launches dominate: for few tokens, whose QKV / ffn_in GEMMs run on
  // the narrow / small kernels (the statistics loads overlap their K loop).  On the MFMA tiles of
  // larger shapes the epilogue work it adds is exposed and costs more than the LayerNorm launch
  // it removes (measured on MI355X: C5 +3.9%, C4 +5.5%), so LN1 / LN2 stay standalone there.
  const bool fold = folds_layernorm(fused_ln, T, D, F);
  const half* cur = (const half*)x;
  for (int l = 0; l < L; ++l) {
    const half* w = wts + (size_t)l * lay.stride;
    // With a mask, padded rows are skipped from here on: LN writes them as +0.0, the QKV and
    // ffn_in projections write +0.0 (tiles of padded rows do no MMA work), out_proj keeps the
    // residual and ffn_out zeroes them (the block mask).  No valid token reads a padded row's
    // values: keys with mask 0 get probability 0, and every later op is row-wise.
    EpiArgs ep{};
    ep.bias = w + lay.off[3];
    ep.y = q;
    ep.ldy = 3 * D;
    ep.mode = TT_EPI_QKV;
    ep.batch = B;
    ep.seq = S;
    ep.heads = H;
    ep.head_dim = hd;
    ep.d_model = D;
    ep.q_scale = attention_q_scale(hd);  // Q leaves the projection in the attention's form
    if (fused_ln) {
      if ((rc = launch_ln_tile(cur, w + lay.off[0], w + lay.off[1], w + lay.off[2], ep, B, S, D,
                               3 * D, stream)) != TT_OK)
        return rc;
    } else if (l == 0 || !fold) {
      if ((rc = launch_layernorm(cur, w + lay.off[0], w + lay.off[1], mask, ws.xn, T, D, 1e-5f,
                                 stream)) != TT_OK)
        return rc;
      ep.valid = mask;
      if ((rc = launch_linear(ws.xn, w + lay.off[2], T, 3 * D, D, ep, stream)) != TT_OK) return rc;
    } else {
      ep.valid = mask;
      ep.ln_part = ws.part;
      ep.ln_slots = part_slots;
      ep.ln_stride = ldp;
      ep.ln_colsum = (const float*)(w + lay.off[13]);
      ep.ln_bias = (const float*)(w + lay.off[14]);
      if ((rc = launch_linear(cur, w + lay.off[12], T, 3 * D, D, ep, stream)) != TT_OK) return rc;
    }
    if ((rc = launch_attention(q, k, vt, mask, info, ws.xn, B, S, H, hd, causal, stream, true)) !=
        TT_OK)
      return rc;
    ep = EpiArgs{};
    ep.bias = w + lay.off[5];
    ep.resid = cur;
    ep.valid = mask;
    ep.seq = S;  // row-tile balancing of padded batches
    ep.y = ws.xa;
    ep.ldy = D;
    ep.mode = TT_EPI_RESID_MASKED;
    if (fold) {
      ep.part_out = ws.part;
      ep.ln_stride = ldp;
      part_slots = D / linear_stats_width(T, D, D, TT_EPI_RESID_MASKED);
    }
    if ((rc = launch_linear(ws.xn, w + lay.off[4], T, D, D, ep, stream)) != TT_OK) return rc;
    ep = EpiArgs{};
    ep.bias = w + lay.off[9];
    ep.y = ws.hbuf;
    ep.ldy = F;
    ep.mode = TT_EPI_BIAS_GELU;
    if (fused_ln) {
      if ((rc = launch_ln_tile(ws.xa, w + lay.off[6], w + lay.off[7], w + lay.off[8], ep, B, S, D,
                               F, stream)) != TT_OK)
        return rc;
    } else if (!fold) {
      if ((rc = launch_layernorm(ws.xa, w + lay.off[6], w + lay.off[7], mask, ws.xn, T, D, 1e-5f,
                                 stream)) != TT_OK)
        return rc;
      ep.valid = mask;
      ep.seq = S;  // row-tile balancing of padded batches
      if ((rc = launch_linear(ws.xn, w + lay.off[8], T, F, D, ep, stream)) != TT_OK) return rc;
    } else {
      ep.valid = mask;
      ep.seq = S;  // row-tile balancing of padded batches
      ep.ln_part = ws.part;
      ep.ln_slots = part_slots;
      ep.ln_stride = ldp;
      ep.ln_colsum = (const float*)(w + lay.off[16]);
      ep.ln_bias = (const float*)(w + lay.off[17]);
      if ((rc = launch_linear(ws.xa, w + lay.off[15], T, F, D, ep, stream)) != TT_OK) return rc;
    }
    ep = EpiArgs{};
    ep.bias = w + lay.off[11];
    ep.resid = ws.xa;
    ep.valid = mask;
    ep.seq = S;  // row-tile balancing of padded batches
    ep.y = ws.xa;
    ep.ldy = D;
    ep.mode = TT_EPI_MASKED_RESID;
    if (fold && l + 1 < L) {  // statistics for the next layer's LN1
      ep.part_out = ws.part;
      ep.ln_stride = ldp;
      part_slots = D / linear_stats_width(T, D, F, TT_EPI_MASKED_RESID);
    }
    if ((rc = launch_linear(ws.hbuf, w + lay.off[10], T, D, F, ep, stream)) != TT_OK) return rc;
    cur = ws.xa;
  }
  return launch_layernorm(cur, wts + lay.final_off, wts + lay.final_off + align64(D), mask,
                          (half*)y, T, D, 1e-5f, stream);
}

}  // namespace tt

extern "C" int tt_transformer_fwd(const void* weights, const void* x, const uint8_t* mask, void* y,
                                  void* workspace, int64_t workspace_bytes, int batch, int seq,
                                  int d_model, int num_heads, int ffn_dim, int num_layers,
                                  int causal, int plan, void* stream) {
  return transformer_fwd(weights, x, mask, y, workspace, workspace_bytes, batch, seq, d_model,
                         num_heads, ffn_dim, num_layers, causal, plan, false, stream);
}

extern "C" int tt_megakernel_error_offset(int batch, int seq, int d_model, int num_heads,
                                          int ffn_dim, int num_layers, int64_t* offset) {
  int rc = check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(offset != nullptr, "megakernel_error_offset: null output");
  *offset = (int64_t)megakernel_error_offset(batch, seq, d_model, ffn_dim, num_layers);
  return TT_OK;
}

extern "C" int tt_megakernel_attach_status(void* workspace, int64_t workspace_bytes, int batch,
                                           int seq, int d_model, int num_heads, int ffn_dim,
                                           int num_layers, int32_t* host_status, void* stream) {
  int rc = check_model_shape(batch, seq, d_model, num_heads, ffn_dim, num_layers);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(workspace != nullptr, "megakernel_attach_status: null workspace");
  return megakernel_attach_status(workspace, workspace_bytes, batch, seq, d_model, num_heads,
                                  ffn_dim, num_layers, (uint32_t*)host_status,
                                  (hipStream_t)stream);
}

extern "C" int tt_megakernel_set_spin_limit(int64_t limit) {
  megakernel_set_spin_limit(limit);
  return TT_OK;
}
