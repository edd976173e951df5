// Persistent whole-model megakernel: one launch runs every layer and the final norm,
// with a workgroup-level dependency DAG in place of the per-op launches of the layer-wise plan.
//
// Tasks (row block rb = 64 consecutive tokens of one sequence; query block qb = 128 tokens):
//   QKV(l, rb, nt)   64 columns of [Q | K | V^T] = LN1_l(X[rb]) Wqkv^T + b for X = x (l = 0) or
//                    the residual stream xa, with the LayerNorm folded into the weights
//                    (W' = W diag(gamma), epilogue rstd (acc - mean c) + b'); the rows' statistics
//                    are computed from the A operand as it streams through LDS
//   ATT(l, b, h, qb) attention of query block qb of sequence b, head h -> ctx
//   OUT(l, rb, nt)   xa[rb, nt] = resid + mask(ctx Wo^T + bo)
//   FF1(l, rb, nt)   h[rb, nt] = GELU(LN2(xa[rb]) W1^T + b1), LayerNorm folded as in QKV
//   FF2(l, rb, nt, s) split s of K = ffn_dim of xa[rb, nt] = mask(xa + h W2^T + b2): each split
//                    stores an fp32 partial and the last one to arrive sums them in split order
//                    and runs the epilogue
//   FIN(rb)          y[rb] = mask(final_norm(xa[rb]))
// No task waits for a LayerNorm: the norms of QKV / FF1 ride on the GEMM's own A stream.  An FF2
// split waits only for the FF1 tiles of its K range.
// XCD-local hand-off.  The eight XCDs of an MI355X have separate L2 caches; a workgroup's stores
// reach its own XCD's L2 (the vector L1 writes through), while making them visible to another
// XCD takes an L2 write-back and an invalidate, which cost several microseconds per hand-off when
// many workgroups do them at once (measured).  So sequence b belongs to XCD b mod nx and every
// task of the sequence runs on that XCD's workgroups: data only moves through the shared L2.  A
// producer waits for its stores (s_waitcnt vmcnt(0)) and bumps a dependency counter; a consumer
// polls the counter and reads produced data with device-scope loads (sc1), which skip its own
// L1 (it may hold stale copies of those lines) and are served by the L2.  A workgroup reads the
// XCD it runs on from the hardware register XCC_ID and draws a rank on it from that XCD's ticket
// counter (the grid is nx W workgroups, which dispatch deals round-robin over the XCDs, so every
// XCD gets W of them); the workgroups of an XCD take turns over the tasks of its sequences in list
// order (task v of the XCD's list to rank v mod W).  Without a known XCD count the same tasks run
// over all workgroups with agent-scope release / acquire hand-offs (L2 write-back before the
// counter changes, invalidate before the data is read).
// Tasks are listed in a topological order and every task waits only on tasks listed before it;
// all workgroups are resident at once, so the earliest unfinished task can always run: the DAG
// cannot deadlock.  Residency comes from the launch size: at most one workgroup per CU, whose
// 144 KiB of LDS fits one per CU, so on a device not shared with other kernels every workgroup
// is dispatched at once.  (A cooperative launch would guarantee it formally but costs ~17 us more
// per launch on MI355X -- measured -- which is more than the forward of the small shapes this
// plan is for.)
// Dependencies are per (layer, kind, row block, sub-index) counters in the workspace that only
// ever grow; a launch waits for `epoch * count`, where the epoch (launch number) is kept in the
// workspace and advanced by the last workgroup to finish, so no counter is ever reset (the
// workspace must be zero-filled once, before its first use).  Every spin-wait is bounded: on
// expiry the kernel records an error in the workspace and all later waits fall through, so every
// wave exits.
//
// Write-after-read: Q/K/V^T are single buffers, so QKV(l, rb) also waits for every attention
// task of layer l-1 whose keys include rb.  Every other buffer's next writer already depends
// (transitively) on its readers.
//
// The tasks are latency-bound (a 64 x 64 tile has 4 MFMAs per wave per K step), so the GEMM
// tiles keep up to 8 K steps of copies in flight (global -> LDS, waited per step with vmcnt),
// weights are prefetched before a task waits for its inputs, each task issues all of its memory
// traffic as early as its dependencies allow, and row statistics use DPP quad reductions (no LDS
// round trips).
#include "attention_block.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cstring>
#include <mutex>

namespace tt {

namespace {

constexpr int kMB = 64;            // rows per row block
constexpr int kQB = 128;           // queries per attention block (= attention_block's tile)
constexpr int kNB = 64;            // columns per GEMM tile
constexpr int kMaxD = 512;         // fused-LN tiles: LN'd A operand resident in LDS, 64 x D halfs
constexpr int kMKThreads = 256;
constexpr uint32_t kSpinLimit = 1u << 22;  // polls (each followed by s_sleep 1) per wait

// LDS map (halfs), 144 KiB + a small int area at the end.  Tasks whose A operand is a
// LayerNorm computed in LDS (QKV, FF1) use [0, kResA) for it and a ring of kRingW weight-only K
// steps after it; tasks that stream A (OUT, FF2) use the whole map as a ring of kRingAW steps of
// A and W.  The attention tiles reuse the start of the map.
constexpr int kResA = kMB * kMaxD;
constexpr int kStepW = kNB * 64;            // one K step of W: 64 rows x 64 halfs
constexpr int kStepAW = (kMB + kNB) * 64;   // one K step of A then W
constexpr int kLdsHalfs = kResA + 10 * kStepW;
constexpr int kRingW = 8;                   // K steps in flight (weights only)
constexpr int kRingAW = kLdsHalfs / kStepAW;  // = 9
static_assert(kResA + kRingW * kStepW <= kLdsHalfs && kRingAW * kStepAW <= kLdsHalfs, "LDS map");

// Dependency counters, kSub per (layer, kind, row block): QKV, ATT, OUT and FF2 (tiles of a row
// block whose output is complete) use sub-counter 0; FF1 counts finished tiles per FF2 split
// (sub = split); FF2T counts the arrivals of the splits of FF2 tile nt (sub = nt).
enum Counter : int { cQKV = 0, cATT, cOUT, cFF1, cFF2, cFF2T, kNumCounters };
constexpr int kSub = 8;            // >= FF2 splits and >= d_model / 64 (d_model <= kMaxD)
static_assert(kSub * kNB >= kMaxD, "one FF2T sub-counter per output tile of a row block");
constexpr int kMinSplitSteps = 8;  // K steps (of 64) per FF2 split at least

struct MegaParams {
  const half* w;
  int64_t off[TT_LAYER_SEGMENTS];
  int64_t stride, final_off;
  const half* x;
  half* y;
  const uint8_t* mask;
  half *xa, *ctx, *q, *k, *vt, *hbuf;
  float* part;      // FF2 split partials: [nrb][td][ks][256 lanes x 16] fp32
  uint32_t* cnt;    // [L][kNumCounters][nrb][kSub]
  uint32_t* ctrl;   // [0] epoch, [1] finished workgroups, [2] error flag, [4..5] host mirror
                    // address of the error flag (0: none), set by megakernel_attach_status,
                    // [8 + x] ticket counter of XCD x (XCD-local plan)
  uint64_t* trace;  // optional: 4 words per task (task | wg << 32, start, ready, end) or nullptr
  uint32_t spin_limit;  // polls per dependency wait before it gives up (kSpinLimit by default)
  int B, S, D, H, F, L, causal;
  int nsb, nqb, nrb, tq, td, tf;  // row / query blocks per sequence, row blocks, N tiles
  int ks, ksteps;                 // FF2 splits of K = ffn_dim, K steps (of 64) per split
  int per_layer, ntask;
  int nx;                         // XCDs (XCD-local plan; <= 8, one ticket word each)
  float scale_log2;
};

// The launch parameters are read in place from the kernel-argument segment through a pointer in
// the constant address space (scalar loads).  The persistent loop re-derives that pointer per task
// (an opaque copy), so a task reloads the fields it uses instead of the compiler keeping every
// field of every task kind live in registers across the loop.
typedef const __attribute__((address_space(4))) MegaParams MPc;

__device__ __forceinline__ uint32_t ld_relaxed(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Trace stamps (100 MHz constant clock) of the task being run, written by thread 0 when a trace
// buffer is given: start, dependencies satisfied ("ready"), end.
__device__ __forceinline__ void trace_stamp(MPc& p, int task, int slot) {
  if (p.trace != nullptr && threadIdx.x == 0) {
    uint64_t* rec = p.trace + 4 * (size_t)task;
    if (slot == 1) rec[0] = (uint64_t)task | ((uint64_t)blockIdx.x << 32);
    rec[slot] = __builtin_amdgcn_s_memrealtime();
  }
}

__device__ __forceinline__ uint32_t* counter(MPc& p, int layer, int kind, int rb,
                                             int sub = 0) {
  return p.cnt + (((size_t)layer * kNumCounters + kind) * p.nrb + rb) * kSub + sub;
}

// Agent-scope release / acquire for one thread, with the cache maintenance made synchronous.
// The fence emits the L2 write-back (release) or the L1 / L2 invalidate (acquire); both are
// vector-memory operations that complete asynchronously, and the compiler does not always keep
// a wait for them (the write-back was seen issued right before the counter's atomic add with
// nothing in between, and consumers then read stale rows).  Waiting for vmcnt(0) after the fence
// makes the write-back complete before the counter update that follows, and the invalidate
// complete before the workgroup barrier after which the other waves load.
__device__ __forceinline__ void release_agent() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__device__ __forceinline__ void acquire_agent() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Block-wide: wait until *c has reached `target` (mod 2^32), bounded.  Thread 0 polls (the
// counter's device-scope load skips the L1); with agent-scope hand-offs (LOCAL false) it then
// performs the acquire (it invalidates this CU's L1 and the XCD's L2 copies of other XCDs' data
// for the whole workgroup), while XCD-local consumers read produced data with device-scope loads
// instead.  The barrier orders every wave's later loads after the wait.
template <bool LOCAL>
__device__ void mk_wait(MPc& p, const uint32_t* c, uint32_t target) {
  if (threadIdx.x == 0) {
    uint32_t spins = 0;
    while ((int32_t)(ld_relaxed(c) - target) < 0) {
      if (ld_relaxed(p.ctrl + 2) != 0) break;  // an earlier wait expired: fall through
      if (++spins > p.spin_limit) {
        __hip_atomic_store(p.ctrl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if constexpr (!LOCAL) acquire_agent();
  }
  __syncthreads();
}

// Block-wide: publish this block's writes and count one arrival on *c.  Every wave first waits
// for its own stores to complete (they are then in the XCD's L2); with agent-scope hand-offs one
// release after the barrier (L2 write-back of the XCD) covers them all; then the counter is
// bumped.
template <bool LOCAL>
__device__ void mk_signal(uint32_t* c) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    if constexpr (!LOCAL) release_agent();
    __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Wait until at most `newer` (even, <= 28) of this wave's loads are still in flight.
__device__ __forceinline__ void wait_newer(int newer) {
  switch (newer >> 1) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<2>(); break;
    case 2: wait_vmcnt<4>(); break;
    case 3: wait_vmcnt<6>(); break;
    case 4: wait_vmcnt<8>(); break;
    case 5: wait_vmcnt<10>(); break;
    case 6: wait_vmcnt<12>(); break;
    case 7: wait_vmcnt<14>(); break;
    case 8: wait_vmcnt<16>(); break;
    case 9: wait_vmcnt<18>(); break;
    case 10: wait_vmcnt<20>(); break;
    case 11: wait_vmcnt<22>(); break;
    case 12: wait_vmcnt<24>(); break;
    case 13: wait_vmcnt<26>(); break;
    default: wait_vmcnt<28>(); break;
  }
}
static_assert(2 * (kRingW - 1) <= 28 && 4 * (kRingAW - 2) <= 28, "wait_newer range");

// LayerNorm of the rows of one row block, G lanes per row (G >= D / 8 chunks of 8 halfs, so
// 64 / G rows per wave instruction), every row's loads of a wave issued before any reduction.
// OUT_LDS: write the normalised rows [0, 64) into the resident A area of LDS as
// [D/64][64 rows][64 halfs] with 16-byte chunks swizzled by row (rows past nrows are zero);
// otherwise write rows [0, nrows) to dst (global, row stride D), as +0.0 where the mask is 0.
struct NoHook {
  __device__ void operator()() const {}
};

template <int G, bool OUT_LDS, int POLICY = kLoadDefault, typename Hook = NoHook,
          typename Pre = NoHook>
__device__ void mk_layernorm_block(const half* src, const half* gamma, const half* beta,
                                   const uint8_t* valid, int row0, int nrows, int D, half* dst,
                                   Hook hook = Hook{}, Pre pre = Pre{}) {
  constexpr int RPP = 64 / G;                 // rows per wave pass
  constexpr int PASSES = kMB / (4 * RPP);     // passes per wave (4 waves cover the 64 rows)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane % G;                     // this lane's 16-byte chunk of its row
  const int nch = D >> 3;
  const bool act = c < nch;
  half8 g = {}, bb = {};
  if (act) {
    g = *(const half8*)(gamma + 8 * c);
    bb = *(const half8*)(beta + 8 * c);
  }
  pre();  // e.g. the wait for the rows: the affine vectors are in flight meanwhile
  half8 v[PASSES];
  const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(src + (size_t)row0 * D, (uint32_t)nrows * D * 2);
#pragma unroll
  for (int i = 0; i < PASSES; ++i) {
    const int r = (i * 4 + wave) * RPP + lane / G;
    v[i] = half8{};
    if (act && r < nrows) {
      if constexpr (POLICY == kLoadDefault) v[i] = *(const half8*)(src + (size_t)(row0 + r) * D + 8 * c);
      else v[i] = __builtin_bit_cast(half8, load16<POLICY>(sr, (uint32_t)(r * D + 8 * c) * 2));
    }
  }
  hook();  // issued after the row loads, so the reductions below do not wait for its loads
#pragma unroll
  for (int i = 0; i < PASSES; ++i) {
    const int r = (i * 4 + wave) * RPP + lane / G;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)v[i][e];
    const float mean = seg_sum<G>(s) / (float)D;
    float qs = 0.f;
    if (act) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = (float)v[i][e] - mean;
        qs += t * t;
      }
    }
    const float rstd = rsqrtf(seg_sum<G>(qs) / (float)D + 1e-5f);
    if (!act) continue;
    bool keep = r < nrows;
    if constexpr (!OUT_LDS) keep = keep && (valid == nullptr || valid[row0 + r] != 0);
    half8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = keep ? (half)(((float)v[i][e] - mean) * rstd * (float)g[e] + (float)bb[e]) : (half)0.f;
    if constexpr (OUT_LDS) {
      *(half8*)(dst + ((c >> 3) * kMB + r) * 64 + (((c & 7) ^ (r & 7)) << 3)) = o;
    } else if (r < nrows) {
      *(half8*)(dst + (size_t)(row0 + r) * D + 8 * c) = o;
    }
  }
}

template <bool OUT_LDS, int POLICY = kLoadDefault, typename Hook = NoHook, typename Pre = NoHook>
__device__ void mk_layernorm(const half* src, const half* gamma, const half* beta,
                             const uint8_t* valid, int row0, int nrows, int D, half* dst,
                             Hook hook = Hook{}, Pre pre = Pre{}) {
  const int nch = D >> 3;
  if (nch <= 8)
    mk_layernorm_block<8, OUT_LDS, POLICY>(src, gamma, beta, valid, row0, nrows, D, dst, hook, pre);
  else if (nch <= 16)
    mk_layernorm_block<16, OUT_LDS, POLICY>(src, gamma, beta, valid, row0, nrows, D, dst, hook, pre);
  else if (nch <= 32)
    mk_layernorm_block<32, OUT_LDS, POLICY>(src, gamma, beta, valid, row0, nrows, D, dst, hook, pre);
  else
    mk_layernorm_block<64, OUT_LDS, POLICY>(src, gamma, beta, valid, row0, nrows, D, dst, hook, pre);
}

// ---- 64 x 64 GEMM tile, K streamed through an LDS ring of K steps ----
// A K step holds [64 rows][64 halfs] per operand with 16-byte chunks swizzled by row.  Copy i of
// a wave moves 8 rows (1 KiB): rows 8 (wave + 4 i) + lane / 8, logical chunk (lane % 8) ^ (row % 8).
// `ld` is the operand's row stride and k0 the first column of the step.
__device__ __forceinline__ void mk_copy_w(const half* W, int ld, int n0, int k0, half* dst) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave + 4 * i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (lane >> 3);
    lds_copy16(W + (size_t)(n0 + r) * ld + k0 + 8 * c, dst + (wave + 4 * i) * 8 * 64);
  }
}

template <int POLICY>
__device__ __forceinline__ void mk_copy_a(const half* A, int ld, int row0, int nrows, int k0,
                                          half* dst) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = min((wave + 4 * i) * 8 + (lane >> 3), nrows - 1);  // clamped rows: never stored
    const int c = (lane & 7) ^ (lane >> 3);
    lds_copy16<POLICY>(A + (size_t)(row0 + r) * ld + k0 + 8 * c, dst + (wave + 4 * i) * 8 * 64);
  }
}

// Where K step s of a tile lives: RESA tiles keep W only, after the resident A area; streaming
// tiles keep A then W, from the start of the map.
template <bool RESA>
struct Ring {
  static constexpr int NS = RESA ? kRingW : kRingAW;
  __device__ static half* w(half* lds, int s) {
    return RESA ? lds + kResA + (s % NS) * kStepW : lds + (s % NS) * kStepAW + kMB * 64;
  }
  __device__ static half* a(half* lds, int s) { return lds + (s % NS) * kStepAW; }
};

// Issue the weight copies of the first min(NS - 1, nk) K steps, columns k0 + 64 s (before the
// task waits for its inputs: weights never change).
template <bool RESA>
__device__ __forceinline__ void mk_prefetch_w(const half* W, int ld, int n0, int k0, int nk,
                                              half* lds) {
  for (int s = 0; s < Ring<RESA>::NS - 1 && s < nk; ++s)
    mk_copy_w(W, ld, n0, k0 + s * 64, Ring<RESA>::w(lds, s));
}

// Accumulator of the 64 x 64 tile: sum over K steps s < nk of A[row0 + m][k0 + 64 s ..] .
// W[n0 + n][k0 + 64 s ..] (row strides lda, ldw).  A comes from `A` (streamed, RESA == false)
// or from the resident LayerNorm'd area (RESA == true, the fused-LN plan's tiles).  The W copies of the first NS - 1 steps must have been issued
// by mk_prefetch_w<RESA> with the same arguments; loads the caller issues between the two are
// complete when the first step is.  Four waves in 2 x 2, each a 32 x 32 MFMA block (W as the
// MFMA's A operand, so the accumulator is C^T): acc[4 g + e] = C[32 wm + lane % 32]
// [32 wn + 8 g + 4 (lane / 32) + e].
// STATS (streaming only, the K range being whole rows): also the LayerNorm statistics of the 64 A
// rows, computed from the K steps as they pass through LDS -- 4 lanes per row take a step's 64
// values, whose (mean, M2) are merged into the running ones (Chan et al.) -- and left in
// srow[row] = (mean, rstd), biased variance, eps 1e-5.  The ring is free when this returns.
template <bool RESA, bool STATS, int POLICY = kLoadDefault>
__device__ floatx16 mk_tile_core(const half* A, int lda, const half* W, int ldw, int n0, int k0,
                                 int nk, int row0, int nrows, half* lds, float2* srow) {
  static_assert(!(RESA && STATS), "statistics come from the streamed A operand");
  using R = Ring<RESA>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31, fhi = lane >> 5, fx = lane & 7;
  const int sr = threadIdx.x >> 2, sq = threadIdx.x & 3;  // statistics: row, quarter of a step
  const int pro = min(nk, R::NS - 1);  // K steps whose W copies mk_prefetch_w issued
  if constexpr (!RESA) {
    for (int s = 0; s < pro; ++s) mk_copy_a<POLICY>(A, lda, row0, nrows, k0 + s * 64, R::a(lds, s));
  }
  floatx16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  float mean = 0.f, m2 = 0.f;
  auto step = [&](int kt) {
    const half* wb = R::w(lds, kt);
    const half* ab = RESA ? lds + kt * kMB * 64 : R::a(lds, kt);
    half8 a[4], b[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int pc = (2 * kk + fhi) ^ fx;
      b[kk] = *(const half8*)(ab + (wm * 32 + frow) * 64 + pc * 8);
      a[kk] = *(const half8*)(wb + (wn * 32 + frow) * 64 + pc * 8);
    }
    half8 u0, u1;
    if constexpr (STATS) {
      u0 = *(const half8*)(ab + sr * 64 + (((2 * sq) ^ (sr & 7)) << 3));
      u1 = *(const half8*)(ab + sr * 64 + (((2 * sq + 1) ^ (sr & 7)) << 3));
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma32x32x16(a[kk], b[kk], acc);
    if constexpr (STATS) {
      float v[16];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = (float)u0[e];
        v[8 + e] = (float)u1[e];
      }
      const float2 st = slot_stats<4, 16>(v);  // this step's 64 values of row sr
      if (kt == 0) {
        mean = st.x;
        m2 = st.y;
      } else {
        const float n = 64.f * (float)kt, tot = n + 64.f, d = st.x - mean;
        mean = fmaf(d, 64.f / tot, mean);
        m2 += fmaf(d * d, n * 64.f / tot, st.y);
      }
    }
  };
  if (nk <= R::NS - 1) {
    // Every K step is already in flight: one wait and one barrier.
    wait_vmcnt<0>();
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) step(kt);
  }
  // Issue order of this wave's loads: W copies of the prologue steps (mk_prefetch_w), then the
  // caller's epilogue loads, then the A copies of the prologue steps, then W and A of each later
  // step together.  Step kt is complete once at most the loads issued after its last copy are in
  // flight: `newer` counts those.
  for (int kt = 0; kt < nk && nk > R::NS - 1; ++kt) {
    const int issued = min(nk, kt + R::NS - 1);  // steps whose copies are out
    int newer;
    if (RESA) newer = 2 * (issued - 1 - kt);
    else if (kt < pro) newer = 2 * (pro - 1 - kt) + 4 * (issued - pro);
    else newer = 4 * (issued - 1 - kt);
    wait_newer(newer);
    // Step kt visible to all waves; step kt - 1's buffer is free.  A barrier without the memory
    // fence of __syncthreads(), whose vmcnt(0) would also wait for the later steps' copies.
    raw_barrier();
    const int nxt = kt + R::NS - 1;
    if (nxt < nk) {
      mk_copy_w(W, ldw, n0, k0 + nxt * 64, R::w(lds, nxt));
      if constexpr (!RESA) mk_copy_a<POLICY>(A, lda, row0, nrows, k0 + nxt * 64, R::a(lds, nxt));
    }
    step(kt);
  }
  if constexpr (STATS) {
    if (sq == 0) srow[sr] = make_float2(mean, rsqrtf(m2 / (float)(64 * nk) + 1e-5f));
  }
  __syncthreads();  // the ring and the resident area are free for the next task
  return acc;
}

// Store 4 consecutive features (row m, columns n .. n + 3) of an epilogue's result: row-major
// into ep.y, or for TT_EPI_QKV scattered into the Q / K planes ([B, H, S, hd]) and V^T
// ([B, H, hd, S padded to 64]).
template <int MODE>
__device__ __forceinline__ void mk_store4(const EpiArgs& ep, int m, int n, half4 h) {
  if constexpr (MODE == TT_EPI_QKV) {
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
    const int which = n / D, nn = n - which * D;
    const int hh = nn / hd, d = nn - hh * hd;
    const int bb = m / S, sq = m - bb * S;
    const size_t bh = (size_t)bb * ep.heads + hh;
    const size_t plane = (size_t)ep.batch * S * D;
    if (which < 2) {
      *(half4*)(ep.y + which * plane + (bh * S + sq) * hd + d) = h;
    } else {
      const size_t ldv = (size_t)(S + 63) / 64 * 64;
      half* vt = ep.y + 2 * plane + (bh * hd + d) * ldv + sq;
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[(size_t)e * ldv] = h[e];
    }
  } else {
    *(half4*)(ep.y + (size_t)m * ep.ldy + n) = h;
  }
}

// Epilogue operands of this lane's 16 columns and row, loaded before the K loop so that their
// latency overlaps it: bias; for the residual modes the residual row and its mask bit.
struct TileCols {
  half4 bias[4], res[4];
  bool ok;
};

// Bias of this lane's 16 columns (a weight: may be loaded before the task's inputs are ready).
__device__ __forceinline__ void mk_load_bias(TileCols& c, const half* bias, int n0) {
  const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) & 1;
#pragma unroll
  for (int g = 0; g < 4; ++g) c.bias[g] = *(const half4*)(bias + n0 + wn * 32 + 8 * g + 4 * (lane >> 5));
  c.ok = true;
}

// Residual of this lane's row and 16 columns and the row's mask bit.
template <int POLICY = kLoadDefault>
__device__ __forceinline__ void mk_load_resid(TileCols& c, const EpiArgs& ep, int row0, int nrows,
                                              int n0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ml = min(wm * 32 + (lane & 31), nrows - 1);
  c.ok = ep.valid == nullptr || ep.valid[row0 + ml] != 0;
  const __amdgpu_buffer_rsrc_t rr =
      buffer_rsrc(ep.resid + (size_t)row0 * ep.ldy, (uint32_t)nrows * ep.ldy * 2);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int col = n0 + wn * 32 + 8 * g + 4 * (lane >> 5);
    if constexpr (POLICY == kLoadDefault)
      c.res[g] = *(const half4*)(ep.resid + (size_t)(row0 + ml) * ep.ldy + col);
    else
      c.res[g] = __builtin_bit_cast(
          half4, __builtin_amdgcn_raw_buffer_load_b64(rr, (uint32_t)(ml * ep.ldy + col) * 2, 0, POLICY));
  }
}

template <int MODE>
__device__ __forceinline__ TileCols mk_load_cols(const EpiArgs& ep, int row0, int nrows, int n0) {
  TileCols c;
  mk_load_bias(c, ep.bias, n0);
  if constexpr (MODE == TT_EPI_RESID_MASKED || MODE == TT_EPI_MASKED_RESID)
    mk_load_resid(c, ep, row0, nrows, n0);
  return c;
}

// Epilogue straight from registers: bias, then GELU / residual add with the row mask / none,
// rounded to fp16 and stored (rows past nrows are not stored).
template <int MODE>
__device__ void mk_epilogue(const floatx16& acc, const TileCols& c, const EpiArgs& ep, int row0,
                            int nrows, int n0) {
  constexpr bool RESID = MODE == TT_EPI_RESID_MASKED || MODE == TT_EPI_MASKED_RESID;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ml = wm * 32 + (lane & 31);
  if (ml >= nrows) return;
  const int m = row0 + ml;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int n = n0 + wn * 32 + 8 * g + 4 * (lane >> 5);
    half4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = acc[4 * g + e] + (float)c.bias[g][e];
      if constexpr (MODE == TT_EPI_QKV) v *= n < ep.d_model ? ep.q_scale : 1.f;
      if constexpr (MODE == TT_EPI_BIAS_GELU) {
        h[e] = (half)gelu_erf(v);
      } else if constexpr (RESID) {
        const half br = (half)v;  // branch rounded to fp16 first (eager boundary)
        const half sum = (half)((float)c.res[g][e] + (float)br);
        if constexpr (MODE == TT_EPI_RESID_MASKED) h[e] = c.ok ? sum : c.res[g][e];
        else h[e] = c.ok ? sum : (half)0.f;
      } else {
        h[e] = (half)v;
      }
    }
    mk_store4<MODE>(ep, m, n, h);
  }
}

// Folded-LayerNorm operands of this lane's 16 columns: c = sum_k W'[n][k] with W' = W diag(gamma),
// and b' = b + W beta (fp32 segments written when the weights are packed).
struct FoldCols {
  floatx4 c[4], b[4];
};

__device__ __forceinline__ FoldCols mk_load_fold(const float* csum, const float* bfold, int n0) {
  const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) & 1;
  FoldCols f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int n = n0 + wn * 32 + 8 * g + 4 * (lane >> 5);
    f.c[g] = *(const floatx4*)(csum + n);
    f.b[g] = *(const floatx4*)(bfold + n);
  }
  return f;
}

// Epilogue of a projection of LayerNorm(A) computed as A W'^T: per element
// rstd (acc - mean c) + b', with the row's (mean, rstd) from srow; then GELU (TT_EPI_BIAS_GELU)
// or the Q / K / V^T scatter (TT_EPI_QKV).
template <int MODE>
__device__ void mk_epilogue_fold(const floatx16& acc, const FoldCols& f, const float2* srow,
                                 const EpiArgs& ep, int row0, int nrows, int n0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ml = wm * 32 + (lane & 31);
  if (ml >= nrows) return;
  const float2 rs = srow[ml];
  const int m = row0 + ml;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int n = n0 + wn * 32 + 8 * g + 4 * (lane >> 5);
    half4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = fmaf(rs.y, fmaf(-rs.x, f.c[g][e], acc[4 * g + e]), f.b[g][e]);
      if constexpr (MODE == TT_EPI_BIAS_GELU) v = gelu_erf(v);
      if constexpr (MODE == TT_EPI_QKV) v *= n < ep.d_model ? ep.q_scale : 1.f;
      h[e] = (half)v;
    }
    mk_store4<MODE>(ep, m, n, h);
  }
}

// Y[row0 + m, n0 + n] for the 64 x 64 tile of Y = A W^T + b (K = whole rows), epilogue MODE.
// The W copies of the first NS - 1 K steps must have been issued by mk_prefetch_w<RESA>.
template <int MODE, bool RESA>
__device__ void mk_gemm_tile(const half* A, const half* W, int K, int row0, int nrows, int n0,
                             const EpiArgs& ep, half* lds) {
  const TileCols c = mk_load_cols<MODE>(ep, row0, nrows, n0);
  const floatx16 acc =
      mk_tile_core<RESA, false>(A, K, W, K, n0, 0, K / 64, row0, nrows, lds, nullptr);
  mk_epilogue<MODE>(acc, c, ep, row0, nrows, n0);
}

// kv_end (1 + last valid key) and prefix flag of sequence b, computed by the block.
__device__ void mk_mask_summary(MPc& p, int b, int* sred, int& kv_end, bool& prefix) {
  if (p.mask == nullptr) {
    kv_end = p.S;
    prefix = true;
    return;
  }
  int last = -1, count = 0;
  for (int s = threadIdx.x; s < p.S; s += kMKThreads)
    if (p.mask[(size_t)b * p.S + s]) {
      last = s;
      ++count;
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    last = max(last, __shfl_xor(last, off, 64));
    count += __shfl_xor(count, off, 64);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sred[wave] = last;
    sred[4 + wave] = count;
  }
  __syncthreads();
  last = max(max(sred[0], sred[1]), max(sred[2], sred[3]));
  count = sred[4] + sred[5] + sred[6] + sred[7];
  __syncthreads();
  kv_end = last + 1;
  prefix = count == last + 1;
}

// ---- Standalone LayerNorm-prologue GEMM tiles (layer-wise plan for few tokens) ----
// Block (rb, nt): LayerNorm of the 64-row block rb (gamma, beta) straight into LDS, then the
// 64-column tile nt of Y = LN(X) W^T + b with epilogue MODE (TT_EPI_QKV or TT_EPI_BIAS_GELU).
// Replaces a LayerNorm launch + a GEMM launch: the norm is recomputed by each column tile of
// the row block (D <= kMaxD), which costs a few microseconds of VALU less than a separate
// launch and its global round trip when the launches themselves are the critical path.
struct LnTileArgs {
  const half* x;      // [B * S, D] rows to normalise
  const half* gamma;
  const half* beta;
  const half* w;      // [N, D]
  EpiArgs ep;         // bias, output and the QKV layout fields
  int S, D, N;
};

template <int MODE>
__global__ __launch_bounds__(kMKThreads) void ln_tile_kernel(LnTileArgs a) {
  extern __shared__ __align__(16) half lds[];
  const int nsb = (a.S + kMB - 1) / kMB;
  const int tiles = a.N / kNB;
  const int rb = blockIdx.x / tiles, nt = blockIdx.x - rb * tiles;
  const int b = rb / nsb, sb = rb - b * nsb;
  const int row0 = b * a.S + sb * kMB, nrows = min(kMB, a.S - sb * kMB);
  const int n0 = nt * kNB;
  // Row loads first, then the weight prefetch, then the reductions: the norm waits only for the
  // rows, and the weights stream in meanwhile.
  mk_layernorm<true>(a.x, a.gamma, a.beta, nullptr, row0, nrows, a.D, lds,
                     [&] { mk_prefetch_w<true>(a.w, a.D, n0, 0, a.D / 64, lds); });
  mk_gemm_tile<MODE, true>(nullptr, a.w, a.D, row0, nrows, n0, a.ep, lds);
}

template <int HD, bool CAUSAL, bool LOCAL>
__global__ __launch_bounds__(kMKThreads) void megakernel(MegaParams) {
  MPc* const pk = (MPc*)__builtin_amdgcn_kernarg_segment_ptr();
  MPc& p = *pk;
  // Loads of data written in this launch by other workgroups: with the XCD-local hand-off they
  // bypass the CU's L1 (served by the XCD's L2); with the agent-scope hand-off the acquire has
  // already invalidated the L1.
  constexpr int PS = LOCAL ? kLoadDevice : kLoadDefault;
  extern __shared__ __align__(16) half lds[];
  half* sk = lds;                     // attention tiles reuse the start of the map
  half* sv = lds + 2 * kBKV * HD;
  int* sred = (int*)(lds + kLdsHalfs);                    // 16 ints
  float2* srow = (float2*)(lds + kLdsHalfs + 32);         // 64 (mean, rstd) pairs

  const uint32_t epoch = ld_relaxed(p.ctrl) + 1u;  // this launch's number (workspace starts at 0)
  // Q is written multiplied by scale_log2 (QKV task epilogue), the form attention_block reads
  const AttnArgs aa{p.q, p.k, p.vt, p.mask, p.ctx, p.B, p.S, p.H, p.scale_log2, 1};
  const int ksw = 64 * p.ksteps;                   // columns of h per FF2 split

  // This workgroup's task list.  Agent-scope plan: the whole list, task t to workgroup t mod G.
  // XCD-local plan: sequence b belongs to XCD b mod nx.  A workgroup reads the XCD it runs on
  // from the hardware and draws a rank there from that XCD's ticket counter (the grid is nx W
  // workgroups and dispatch deals them round-robin over the XCDs, from whichever XCD it starts
  // at, so every XCD receives W of them); the W workgroups of an XCD take turns over the tasks
  // of its sequences in list order.  A rank outside [0, W) (a dispatch that is not even) is
  // recorded as an error: that workgroup runs no task, and the waits of the others give up.
  int x0 = 0, dstep = 1, rank = blockIdx.x, nw = gridDim.x;
  if constexpr (LOCAL) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    x0 = (int)(xcc & 0xF) % p.nx;
    dstep = p.nx;
    nw = gridDim.x / p.nx;
    if (threadIdx.x == 0) {
      const uint32_t ticket = __hip_atomic_fetch_add(p.ctrl + 8 + x0, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t r = ticket - (epoch - 1u) * (uint32_t)nw;
      sred[8] = r < (uint32_t)nw ? (int)r : -1;
      if (r >= (uint32_t)nw)
        __hip_atomic_store(p.ctrl + 2, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    rank = sred[8];
    __syncthreads();
  }
  const int nd = (x0 < p.B && rank >= 0) ? (p.B - 1 - x0) / dstep + 1 : 0;  // sequences in the list
  // Tasks per sequence and layer of each kind (QKV, ATT, OUT, FF1, FF2), and the first index of
  // each kind in a layer of the full list.
  const int cnt[5] = {p.nsb * p.tq, p.H * p.nqb, p.nsb * p.td, p.nsb * p.tf, p.nsb * p.td * p.ks};
  const int pdl = cnt[0] + cnt[1] + cnt[2] + cnt[3] + cnt[4];
  const int nlayer = p.L * nd * pdl;

  for (int v = rank; v < nlayer + nd * p.nsb; v += nw) {
    MPc* pt = pk;
    asm volatile("" : "+s"(pt));
    MPc& p = *pt;
    if (v >= nlayer) {  // FIN(rb)
      const int i = v - nlayer, j = i / p.nsb, sb = i - j * p.nsb;
      const int b = x0 + dstep * j, rb = b * p.nsb + sb;
      const int t = p.L * p.per_layer + rb;
      trace_stamp(p, t, 1);
      const int row0 = b * p.S + sb * kMB, nrows = min(kMB, p.S - sb * kMB);
      const int64_t dpad = (p.D + 63) / 64 * 64;
      mk_layernorm<false, PS>(p.xa, p.w + p.final_off, p.w + p.final_off + dpad, p.mask, row0,
                              nrows, p.D, p.y, NoHook{}, [&] {
                                mk_wait<LOCAL>(p, counter(p, p.L - 1, cFF2, rb), epoch * (uint32_t)p.td);
                                trace_stamp(p, t, 2);
                              });
      trace_stamp(p, t, 3);
      continue;
    }
    // ---- decode: layer l, kind, sequence b, index i1 within the sequence's tasks of that kind
    const int l = v / (nd * pdl);
    int i0 = v - l * nd * pdl;
    int kind = 0, first = 0;
    while (kind < 4 && i0 >= nd * cnt[kind]) {
      i0 -= nd * cnt[kind];
      first += p.B * cnt[kind];
      ++kind;
    }
    const int j = i0 / cnt[kind], i1 = i0 - j * cnt[kind];
    const int b = x0 + dstep * j;
    const int t = l * p.per_layer + first + b * cnt[kind] + i1;  // number in the full list
    trace_stamp(p, t, 1);
    const half* wl = p.w + (size_t)l * p.stride;

    if (kind == 1) {  // ATT(l, b, h, qb): heaviest query blocks first when causal
      const int h = i1 / p.nqb;
      int qb = i1 - h * p.nqb;
      if (CAUSAL) qb = p.nqb - 1 - qb;
      const int bh = b * p.H + h;
      int kv_end;
      bool prefix;
      mk_mask_summary(p, b, sred, kv_end, prefix);
      const int q_hi = min(p.S, (qb + 1) * kQB);
      const int key_hi = CAUSAL ? min(kv_end, q_hi) : kv_end;
      const int need = (max(key_hi, q_hi) + kMB - 1) / kMB;  // row blocks of keys and queries
      for (int jj = 0; jj < need; ++jj)
        mk_wait<LOCAL>(p, counter(p, l, cQKV, b * p.nsb + jj), epoch * (uint32_t)p.tq);
      trace_stamp(p, t, 2);
      attention_block<HD, CAUSAL, PS>(aa, bh, qb, kv_end, prefix, sk, sv);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (threadIdx.x == 0) {
        if constexpr (!LOCAL) release_agent();
        for (int jj = 2 * qb; jj < min(2 * qb + 2, p.nsb); ++jj)
          __hip_atomic_fetch_add(counter(p, l, cATT, b * p.nsb + jj), 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
      trace_stamp(p, t, 3);
      continue;
    }

    // GEMM tasks: i1 = (sb * tiles + nt) (* ks + split for FF2)
    int split = 0, ii = i1;
    if (kind == 4) {
      split = ii % p.ks;
      ii /= p.ks;
    }
    const int tiles = (kind == 0) ? p.tq : (kind == 3) ? p.tf : p.td;
    const int sb = ii / tiles, nt = ii - sb * tiles;
    const int rb = b * p.nsb + sb;
    const int row0 = b * p.S + sb * kMB, nrows = min(kMB, p.S - sb * kMB);
    const int n0 = nt * kNB;
    const int nkd = p.D / 64;
    EpiArgs ep{};
    if (kind == 0) {  // QKV: LayerNorm 1 folded into W'
      const half* W = wl + p.off[12];
      mk_prefetch_w<false>(W, p.D, n0, 0, nkd, lds);
      const FoldCols f = mk_load_fold((const float*)(wl + p.off[13]), (const float*)(wl + p.off[14]), n0);
      if (l > 0) {
        mk_wait<LOCAL>(p, counter(p, l - 1, cFF2, rb), epoch * (uint32_t)p.td);
        // write-after-read on Q/K/V^T: attention of layer l-1 reading rows rb is done
        for (int jj = CAUSAL ? (sb & ~1) : 0; jj < p.nsb; jj += 2)
          mk_wait<LOCAL>(p, counter(p, l - 1, cATT, b * p.nsb + jj), epoch * (uint32_t)p.H);
      }
      trace_stamp(p, t, 2);
      const floatx16 acc = mk_tile_core<false, true, PS>(l == 0 ? p.x : p.xa, p.D, W, p.D, n0, 0,
                                                         nkd, row0, nrows, lds, srow);
      ep.y = p.q;
      ep.ldy = 3 * p.D;
      ep.batch = p.B;
      ep.seq = p.S;
      ep.heads = p.H;
      ep.head_dim = HD;
      ep.d_model = p.D;
      ep.q_scale = p.scale_log2;
      mk_epilogue_fold<TT_EPI_QKV>(acc, f, srow, ep, row0, nrows, n0);
      mk_signal<LOCAL>(counter(p, l, cQKV, rb));
    } else if (kind == 2) {  // OUT
      const half* W = wl + p.off[4];
      mk_prefetch_w<false>(W, p.D, n0, 0, nkd, lds);
      TileCols c;
      mk_load_bias(c, wl + p.off[5], n0);
      mk_wait<LOCAL>(p, counter(p, l, cATT, rb), epoch * (uint32_t)p.H);
      trace_stamp(p, t, 2);
      ep.resid = (l == 0) ? p.x : p.xa;
      ep.valid = p.mask;
      ep.y = p.xa;
      ep.ldy = p.D;
      mk_load_resid<PS>(c, ep, row0, nrows, n0);
      const floatx16 acc =
          mk_tile_core<false, false, PS>(p.ctx, p.D, W, p.D, n0, 0, nkd, row0, nrows, lds, nullptr);
      mk_epilogue<TT_EPI_RESID_MASKED>(acc, c, ep, row0, nrows, n0);
      mk_signal<LOCAL>(counter(p, l, cOUT, rb));
    } else if (kind == 3) {  // FF1: LayerNorm 2 folded into W'
      const half* W = wl + p.off[15];
      mk_prefetch_w<false>(W, p.D, n0, 0, nkd, lds);
      const FoldCols f = mk_load_fold((const float*)(wl + p.off[16]), (const float*)(wl + p.off[17]), n0);
      mk_wait<LOCAL>(p, counter(p, l, cOUT, rb), epoch * (uint32_t)p.td);
      trace_stamp(p, t, 2);
      const floatx16 acc =
          mk_tile_core<false, true, PS>(p.xa, p.D, W, p.D, n0, 0, nkd, row0, nrows, lds, srow);
      ep.y = p.hbuf;
      ep.ldy = p.F;
      mk_epilogue_fold<TT_EPI_BIAS_GELU>(acc, f, srow, ep, row0, nrows, n0);
      mk_signal<LOCAL>(counter(p, l, cFF1, rb, nt / p.ksteps));
    } else {  // FF2 split `split`: columns [split ksw, (split + 1) ksw) of h and W2
      const half* W = wl + p.off[10];
      const int k0 = split * ksw;
      const bool reducer = split == p.ks - 1;
      mk_prefetch_w<false>(W, p.F, n0, k0, p.ksteps, lds);
      TileCols c;
      if (reducer) mk_load_bias(c, wl + p.off[11], n0);
      mk_wait<LOCAL>(p, counter(p, l, cFF1, rb, split), epoch * (uint32_t)p.ksteps);
      trace_stamp(p, t, 2);
      ep.resid = p.xa;
      ep.valid = p.mask;
      ep.y = p.xa;
      ep.ldy = p.D;
      if (reducer) mk_load_resid<PS>(c, ep, row0, nrows, n0);
      floatx16 acc = mk_tile_core<false, false, PS>(p.hbuf, p.F, W, p.F, n0, k0, p.ksteps, row0,
                                                    nrows, lds, nullptr);
      // Split-K: splits 0 .. ks-2 store fp32 partial tiles (per lane, in accumulator order) and
      // count their arrival; the last split (numbered after them, so it may wait for them) adds
      // the partials and its own accumulator in split order and runs the epilogue.
      float* part = p.part + (size_t)(rb * p.td + nt) * p.ks * (kMKThreads * 16);
      if (!reducer) {
        floatx4* mine = (floatx4*)(part + (size_t)split * (kMKThreads * 16)) + 4 * threadIdx.x;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          mine[g] = floatx4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
        mk_signal<LOCAL>(counter(p, l, cFF2T, rb, nt));
        trace_stamp(p, t, 3);
        continue;
      }
      if (p.ks > 1) {
        mk_wait<LOCAL>(p, counter(p, l, cFF2T, rb, nt), epoch * (uint32_t)(p.ks - 1));
        const __amdgpu_buffer_rsrc_t pr = buffer_rsrc(part, (uint32_t)(p.ks - 1) * kMKThreads * 64);
        floatx4 sum[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) sum[g] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int s2 = 0; s2 < p.ks - 1; ++s2) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const uint32_t off = ((uint32_t)s2 * kMKThreads * 16 + (4 * threadIdx.x + g) * 4) * 4;
            sum[g] += __builtin_bit_cast(floatx4, load16<PS>(pr, off));
          }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[4 * g + e] = sum[g][e] + acc[4 * g + e];
      }
      mk_epilogue<TT_EPI_MASKED_RESID>(acc, c, ep, row0, nrows, n0);
      mk_signal<LOCAL>(counter(p, l, cFF2, rb));
    }
    trace_stamp(p, t, 3);
  }

  // The last workgroup to finish advances the epoch for the next launch and clears the
  // finish count (every workgroup read the epoch before it arrives here; the next launch is
  // stream-ordered after this one).  If a dependency wait of this or an earlier launch gave up
  // (error word set), the results are invalid: that workgroup then overwrites all of y with NaN
  // (fp16 0x7E00) -- every arrival is preceded by a release and the last one acquires, so every
  // other workgroup's writes of y precede it -- and the host sees the error word on its next
  // health check.
  __shared__ uint32_t last;
  __syncthreads();
  if (threadIdx.x == 0) {
    last = 0;
    release_agent();
    const uint32_t old = __hip_atomic_fetch_add(p.ctrl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1u == gridDim.x) {
      acquire_agent();
      __hip_atomic_store(p.ctrl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      release_agent();
      __hip_atomic_store(p.ctrl, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t err = ld_relaxed(p.ctrl + 2);
      last = err != 0 ? 1u : 0u;
      // mirror the error flag into the caller's pinned host word, if one is attached
      const uint64_t host = __hip_atomic_load((const uint64_t*)(p.ctrl + 4), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      if (host != 0)
        __hip_atomic_store((uint32_t*)host, err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  __syncthreads();
  if (last) {
    const size_t n8 = (size_t)p.B * p.S * p.D / 8;  // D % 64 == 0
    const u32x4 nan8 = {0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u};
    for (size_t i = threadIdx.x; i < n8; i += blockDim.x) *(u32x4*)(p.y + 8 * i) = nan8;
  }
}

}  // namespace

// ---- host side ----

struct MegaLayout {
  size_t xa, ctx, qkv, hbuf, part, cnt, ctrl, bytes;
};

// FF2 splits of K = F: the most (up to kSub) that divide F / 64 into at least kMinSplitSteps
// K steps each.
static int ff2_splits(int64_t F) {
  const int64_t nk = F / 64;
  int best = 1;
  for (int s = 2; s <= kSub; ++s)
    if (nk % s == 0 && nk / s >= kMinSplitSteps) best = s;
  return best;
}

static size_t al256(size_t v) { return (v + 255) / 256 * 256; }

static MegaLayout mega_layout(int64_t B, int64_t S, int64_t D, int64_t F, int64_t L) {
  const int64_t T = B * S, Sp = (S + 63) / 64 * 64, nrb = B * ((S + kMB - 1) / kMB);
  MegaLayout m{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += al256(bytes);
    return at;
  };
  m.xa = take(T * D * 2);
  m.ctx = take(T * D * 2);
  m.qkv = take((2 * T * D + B * D * Sp) * 2);
  m.hbuf = take(T * F * 2);
  const int ks = ff2_splits(F);
  m.part = take(ks > 1 ? (size_t)nrb * (D / kNB) * ks * kMKThreads * 16 * 4 : 0);
  m.cnt = take((size_t)L * kNumCounters * nrb * kSub * 4);
  m.ctrl = take(64);
  m.bytes = o;
  return m;
}

size_t megakernel_workspace_bytes(int B, int S, int D, int F, int L) {
  return mega_layout(B, S, D, F, L).bytes;
}

void megakernel_stage_offsets(int B, int S, int D, int F, int L, int64_t* qkv, int64_t* ctx,
                              int64_t* hidden) {
  const MegaLayout m = mega_layout(B, S, D, F, L);
  *qkv = (int64_t)m.qkv;
  *ctx = (int64_t)m.ctx;
  *hidden = (int64_t)m.hbuf;
}

int megakernel_supported(int B, int S, int D, int H, int F, int L) {
  TT_REQUIRE(D / H == 32 || D / H == 64, "megakernel: head_dim %d not in {32, 64}", D / H);
  TT_REQUIRE(D % 64 == 0 && F % 64 == 0, "megakernel: d_model and ffn_dim must be multiples of 64");
  TT_REQUIRE(D <= kMaxD, "megakernel: d_model %d > %d (one dependency counter per 64 columns)", D,
             kMaxD);
  TT_REQUIRE((int64_t)B * S <= (1 << 20), "megakernel: too many tokens for the persistent plan");
  (void)L;
  return TT_OK;
}

template <int HD, bool CAUSAL, bool LOCAL>
static int launch_mega(MegaParams& p, int cus, hipStream_t stream) {
  const size_t lds = kLdsHalfs * sizeof(half) + 64 + 64 * sizeof(float2);
  static_assert(2 * kBKV * HD * 2 <= kLdsHalfs, "attention tiles must fit the LDS map");
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  static int per_cu = 0;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute((const void*)megakernel<HD, CAUSAL, LOCAL>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr == hipSuccess)
      attr = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, megakernel<HD, CAUSAL, LOCAL>,
                                                          kMKThreads, lds);
  });
  if (attr != hipSuccess) return fail(TT_ERR_HIP, "megakernel setup: %s", hipGetErrorString(attr));
  if (per_cu < 1) return fail(TT_ERR_HIP, "megakernel: a workgroup does not fit a CU");
  // One workgroup per task up to one per CU (all resident): with few tasks every workgroup
  // prefetches its weights at once, with many each runs a task of every stage in turn.  The
  // XCD-local plan sizes this per XCD (its first XCD holds the most sequences) and launches the
  // same number on every XCD, so that round-robin dispatch puts workgroup g on XCD g mod nx.
  int grid;
  if (LOCAL) {
    const int nd = (p.B + p.nx - 1) / p.nx;
    const int per_xcd = p.L * nd * (p.per_layer / p.B) + nd * p.nsb;
    grid = p.nx * std::max(1, std::min(per_xcd, cus / p.nx));
  } else {
    grid = std::max(1, std::min(p.ntask, cus));
  }
  hipLaunchKernelGGL((megakernel<HD, CAUSAL, LOCAL>), dim3(grid), dim3(kMKThreads), lds, stream, p);
  return launch_status("megakernel");
}

template <int MODE>
static int launch_ln_tile_mode(const LnTileArgs& a, int blocks, hipStream_t stream) {
  const size_t lds = kLdsHalfs * sizeof(half) + 64;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute((const void*)ln_tile_kernel<MODE>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  });
  if (attr != hipSuccess) return fail(TT_ERR_HIP, "ln_tile setup: %s", hipGetErrorString(attr));
  hipLaunchKernelGGL((ln_tile_kernel<MODE>), dim3(blocks), dim3(kMKThreads), lds, stream, a);
  return launch_status("ln_tile_kernel");
}

int ln_tile_supported(int D, int N) {
  TT_REQUIRE(D % 64 == 0 && D <= kMaxD, "ln_tile: d_model %d must be a multiple of 64 and <= %d",
             D, kMaxD);
  TT_REQUIRE(N % kNB == 0, "ln_tile: N %d must be a multiple of %d", N, kNB);
  return TT_OK;
}

int launch_ln_tile(const half* x, const half* gamma, const half* beta, const half* w,
                   const EpiArgs& ep, int B, int S, int D, int N, hipStream_t stream) {
  int rc = ln_tile_supported(D, N);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(ep.mode == TT_EPI_QKV || ep.mode == TT_EPI_BIAS_GELU,
             "ln_tile: epilogue %d not supported", ep.mode);
  LnTileArgs a{x, gamma, beta, w, ep, S, D, N};
  const int blocks = B * ((S + kMB - 1) / kMB) * (N / kNB);
  if (ep.mode == TT_EPI_QKV) return launch_ln_tile_mode<TT_EPI_QKV>(a, blocks, stream);
  return launch_ln_tile_mode<TT_EPI_BIAS_GELU>(a, blocks, stream);
}

int megakernel_tasks(int B, int S, int D, int H, int F, int L) {
  const int nsb = (S + kMB - 1) / kMB, nrb = B * nsb, nqb = (S + kQB - 1) / kQB;
  const int per_layer = nrb * (3 * D / kNB) + B * H * nqb + nrb * (D / kNB) + nrb * (F / kNB) +
                        nrb * (D / kNB) * ff2_splits(F);
  return L * per_layer + nrb;
}

size_t megakernel_error_offset(int B, int S, int D, int F, int L) {
  return mega_layout(B, S, D, F, L).ctrl + 2 * sizeof(uint32_t);
}

static uint32_t g_spin_limit = kSpinLimit;


void megakernel_set_spin_limit(int64_t limit) {
  g_spin_limit = limit < 0 ? kSpinLimit : (uint32_t)std::min<int64_t>(limit, 0xFFFFFFFFll);
}

constexpr int kMaxDevices = 64;
struct DevInfo {
  int cus = 0, nx = 1;
  bool xcds_known = false, valid = false;
};

int launch_megakernel(const half* weights, const int64_t off[TT_LAYER_SEGMENTS], int64_t stride,
                      int64_t final_off,
                      const half* x, const uint8_t* mask, half* y, char* workspace,
                      int64_t workspace_bytes, int B, int S, int D, int H, int F, int L, int causal,
                      uint64_t* trace, hipStream_t stream) {
  int rc = megakernel_supported(B, S, D, H, F, L);
  if (rc != TT_OK) return rc;
  const MegaLayout m = mega_layout(B, S, D, F, L);
  TT_REQUIRE((int64_t)m.bytes <= workspace_bytes, "megakernel: workspace %lld < %zu bytes",
             (long long)workspace_bytes, m.bytes);
  MegaParams p{};
  p.w = weights;
  memcpy(p.off, off, sizeof(p.off));
  p.stride = stride;
  p.final_off = final_off;
  p.x = x;
  p.y = y;
  p.mask = mask;
  p.xa = (half*)(workspace + m.xa);
  p.ctx = (half*)(workspace + m.ctx);
  p.q = (half*)(workspace + m.qkv);
  p.k = p.q + (size_t)B * S * D;
  p.vt = p.q + 2 * (size_t)B * S * D;
  p.hbuf = (half*)(workspace + m.hbuf);
  p.part = (float*)(workspace + m.part);
  p.cnt = (uint32_t*)(workspace + m.cnt);
  p.ctrl = (uint32_t*)(workspace + m.ctrl);
  p.trace = trace;
  p.spin_limit = g_spin_limit;
  p.B = B;
  p.S = S;
  p.D = D;
  p.H = H;
  p.F = F;
  p.L = L;
  p.causal = causal;
  p.nsb = (S + kMB - 1) / kMB;
  p.nqb = (S + kQB - 1) / kQB;
  p.nrb = B * p.nsb;
  p.tq = 3 * D / kNB;
  p.td = D / kNB;
  p.tf = F / kNB;
  p.ks = ff2_splits(F);
  p.ksteps = F / 64 / p.ks;
  p.per_layer = p.nrb * p.tq + B * H * p.nqb + p.nrb * p.td + p.nrb * p.tf + p.nrb * p.td * p.ks;
  p.ntask = L * p.per_layer + p.nrb;
  p.scale_log2 = attention_q_scale(D / H);
  int dev = 0;
  TT_HIP(hipGetDevice(&dev));
  TT_REQUIRE(dev >= 0 && dev < kMaxDevices, "megakernel: device %d", dev);
  // Device attributes, queried once per device (a forward of the small shapes this plan serves
  // lasts about as long as a few attribute queries).  The XCD-local hand-off needs the XCD count
  // (every XCD gets the same number of workgroups); without it the agent-scope plan runs.
  static std::mutex mu;
  static DevInfo info[kMaxDevices];
  DevInfo di;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!info[dev].valid) {
      int cus = 0, nx = 0;
      TT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
      info[dev].cus = cus;
      info[dev].xcds_known = hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess &&
                             nx >= 1 && nx <= 8 && cus % nx == 0;
      info[dev].nx = info[dev].xcds_known ? nx : 1;
      info[dev].valid = true;
    }
    di = info[dev];
  }
  const int cus = di.cus;
  const bool xcds_known = di.xcds_known;
  p.nx = di.nx;
  const int hd = D / H;
  if (xcds_known) {
    if (hd == 64)
      return causal ? launch_mega<64, true, true>(p, cus, stream) : launch_mega<64, false, true>(p, cus, stream);
    return causal ? launch_mega<32, true, true>(p, cus, stream) : launch_mega<32, false, true>(p, cus, stream);
  }
  if (hd == 64)
    return causal ? launch_mega<64, true, false>(p, cus, stream) : launch_mega<64, false, false>(p, cus, stream);
  return causal ? launch_mega<32, true, false>(p, cus, stream) : launch_mega<32, false, false>(p, cus, stream);
}

__global__ void mk_zero_words(uint32_t* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

int megakernel_reset(void* workspace, int64_t workspace_bytes, int B, int S, int D, int H, int F,
                     int L, hipStream_t stream) {
  int rc = megakernel_supported(B, S, D, H, F, L);
  if (rc != TT_OK) return rc;
  const MegaLayout m = mega_layout(B, S, D, F, L);
  TT_REQUIRE((int64_t)m.bytes <= workspace_bytes, "megakernel: workspace %lld < %zu bytes",
             (long long)workspace_bytes, m.bytes);
  // counters and control words are contiguous: [cnt, ctrl + 64)
  const size_t words = (m.ctrl + 64 - m.cnt) / 4;
  const int blocks = (int)std::min<size_t>((words + 255) / 256, 1024);
  hipLaunchKernelGGL(mk_zero_words, dim3(blocks), dim3(256), 0, stream,
                     (uint32_t*)((char*)workspace + m.cnt), words);
  return launch_status("mk_zero_words");
}

__global__ void mk_set_word64(uint64_t* __restrict__ dst, uint64_t value) {
  if (threadIdx.x == 0) *dst = value;
}

int megakernel_attach_status(void* workspace, int64_t workspace_bytes, int B, int S, int D, int H,
                             int F, int L, uint32_t* host_status, hipStream_t stream) {
  int rc = megakernel_supported(B, S, D, H, F, L);
  if (rc != TT_OK) return rc;
  const MegaLayout m = mega_layout(B, S, D, F, L);
  TT_REQUIRE((int64_t)m.bytes <= workspace_bytes, "megakernel: workspace %lld < %zu bytes",
             (long long)workspace_bytes, m.bytes);
  hipLaunchKernelGGL(mk_set_word64, dim3(1), dim3(64), 0, stream,
                     (uint64_t*)((char*)workspace + m.ctrl + 4 * sizeof(uint32_t)),
                     (uint64_t)(uintptr_t)host_status);
  return launch_status("mk_set_word64");
}

int megakernel_status(const char* workspace, int B, int S, int D, int F, int L, int* status,
                      hipStream_t stream) {
  const MegaLayout m = mega_layout(B, S, D, F, L);
  uint32_t ctrl[3] = {0, 0, 0};
  TT_HIP(hipMemcpyAsync(ctrl, workspace + m.ctrl, sizeof(ctrl), hipMemcpyDeviceToHost, stream));
  TT_HIP(hipStreamSynchronize(stream));
  *status = (int)ctrl[2];
  return TT_OK;
}

}  // namespace tt
