// tt_transformer_fwd_noalloc: the whole forward without a caller workspace and without any
// allocation, for callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc).  Its intermediates live in a fixed scratch
// array of this library.
#include "common.hpp"
#include "kernels.hpp"

#include <mutex>

using namespace tt;

// Scratch memory of tt_transformer_fwd_noalloc: one array per GPU, allocated by the runtime when
// the code object is loaded on that device and held until the process ends.  Its address is
// taken once per device with hipGetSymbolAddress (the name itself is a host-side stand-in, not a
// device address) and only that address is handed to kernels.
static constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];
// Shape of the latest megakernel-plan call on each device: its error word sits at a
// shape-dependent offset of the array and stays there until the next call clears it.
struct MegaShape {
  bool valid;
  int B, S, D, F, L;
};
static MegaShape g_last_mega[kMaxDevices];

static int scratch_address(void** out) {
  int dev = 0;
  TT_HIP(hipGetDevice(&dev));
  TT_REQUIRE(dev >= 0 && dev < kMaxDevices, "transformer_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> guard(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    TT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    TT_REQUIRE(p != nullptr, "transformer_noalloc: no address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TT_OK;
}

extern "C" int tt_noalloc_scratch_bytes(int64_t* bytes) {
  TT_REQUIRE(bytes != nullptr, "noalloc_scratch_bytes: null output");
  *bytes = (int64_t)kScratchBytes;
  return TT_OK;
}

// Every call on one GPU shares that GPU's array and finds the previous call's contents in it: the
// layer-wise plans overwrite what they read before reading it, and the megakernel plan clears its
// counters first.  Calls that overlap on one GPU (concurrent streams, threads) race on the array.
extern "C" int tt_transformer_fwd_noalloc(const void* weights, const void* x, const uint8_t* mask,
                                          void* y, int batch, int seq, int d_model,
                                          int num_heads, int ffn_dim, int num_layers, int causal,
                                          int plan, void* stream) {
  int64_t need = 0;
  int rc = tt_workspace_bytes(batch, seq, d_model, num_heads, ffn_dim, num_layers, plan, &need);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(need <= (int64_t)kScratchBytes,
             "transformer_noalloc: this shape needs %lld bytes of scratch, more than the %zu "
             "bytes of the library's array (use tt_transformer_fwd with a caller workspace)",
             (long long)need, kScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_address(&ws)) != TT_OK) return rc;
  int dev = 0;
  TT_HIP(hipGetDevice(&dev));
  const bool mega =
      tt_resolve_plan(batch, seq, d_model, num_heads, ffn_dim, plan) == TT_PLAN_MEGAKERNEL;
  rc = transformer_fwd(weights, x, mask, y, ws, (int64_t)kScratchBytes, batch, seq, d_model,
                       num_heads, ffn_dim, num_layers, causal, plan, true, stream);
  std::lock_guard<std::mutex> guard(g_scratch_mu);
  g_last_mega[dev] = MegaShape{mega && rc == TT_OK, batch, seq, d_model, ffn_dim, num_layers};
  return rc;
}

// Health of the latest tt_transformer_fwd_noalloc call on the current device: its megakernel
// error word (the next call's counter reset clears it, so it is read before that call).
extern "C" int tt_noalloc_status(int* status, void* stream) {
  TT_REQUIRE(status != nullptr, "noalloc_status: null output");
  int dev = 0;
  TT_HIP(hipGetDevice(&dev));
  TT_REQUIRE(dev >= 0 && dev < kMaxDevices, "noalloc_status: device %d out of range", dev);
  MegaShape m;
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> guard(g_scratch_mu);
    m = g_last_mega[dev];
    ws = g_scratch_ptr[dev];
  }
  *status = 0;
  if (!m.valid || ws == nullptr) return TT_OK;
  return megakernel_status((const char*)ws, m.B, m.S, m.D, m.F, m.L, status, (hipStream_t)stream);
}

