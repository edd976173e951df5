// FP16 MFMA GEMM with fused epilogues: Y[M,N] = X[M,K] W[N,K]^T + b (+ GELU / residual / mask /
// head-major QKV scatter), fp32 accumulation, for the four projections of the pre-LN block.
//
// Design (gfx950):
//  * Both operands are K-contiguous (nn.Linear weights are [N,K]), so a block stages a BM x 64
//    X tile and a BN x 64 W tile in LDS per K step (128-byte rows, 16-byte chunks XOR-swizzled
//    by row so ds_read_b128 fragment reads are bank-conflict free), double-buffered, with the
//    next K step's global loads issued into registers before the current step's MFMAs.
//  * The MFMA is v_mfma_f32_32x32x16_f16 with W as the "A" operand and X as "B", i.e. each wave
//    accumulates C^T: lane l then holds 4 consecutive output features of one token per group,
//    so the epilogue writes 8-byte runs of a row of Y and reads bias / residual the same way.
//  * Block-id -> tile mapping is XCD-aware: workgroup i runs on XCD i % 8, so each XCD is given
//    a contiguous range of tile ids, and tiles are ordered in groups of 8 row-tiles so the tiles
//    one XCD runs at once share X row panels and W column panels in that XCD's L2.
#include "common.hpp"
#include "kernels.hpp"

#include <mutex>

namespace tt {

constexpr int kBK = 64;

__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;
  return (bid % 8) * (nblocks / 8) + bid / 8;
}

__device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int G = 8;
  const int group = G * tiles_n;
  const int first = (t / group) * G;
  const int gm = min(tiles_m - first, G);
  const int r = t % group;
  tm = first + r % gm;
  tn = r / gm;
}

// Apply the epilogue to 4 consecutive output features n..n+3 of row m.
__device__ __forceinline__ void epilogue4(const EpiArgs& ep, int m, int n, float v0, float v1,
                                          float v2, float v3) {
  const half4 b = *(const half4*)(ep.bias + n);
  float v[4] = {v0 + (float)b[0], v1 + (float)b[1], v2 + (float)b[2], v3 + (float)b[3]};
  const int mode = ep.mode;
  if (mode == TT_EPI_BIAS_GELU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
  } else if (mode == TT_EPI_RESID_MASKED || mode == TT_EPI_MASKED_RESID) {
    const bool ok = ep.valid == nullptr || ep.valid[m] != 0;
    const half4 r = *(const half4*)(ep.resid + (size_t)m * ep.ldy + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (mode == TT_EPI_RESID_MASKED)
        v[e] = (float)r[e] + (ok ? v[e] : 0.f);
      else
        v[e] = ok ? (float)r[e] + v[e] : 0.f;
    }
  } else if (mode == TT_EPI_QKV) {
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
    const int which = n / D, nn = n - which * D;
    const int h = nn / hd, d = nn - h * hd;
    const int bb = m / S, s = m - bb * S;
    const size_t plane = (size_t)ep.batch * S * D;
    const size_t bh = (size_t)bb * ep.heads + h;
    if (which < 2) {
      half4 o = {(half)v[0], (half)v[1], (half)v[2], (half)v[3]};
      *(half4*)(ep.y + which * plane + (bh * S + s) * hd + d) = o;
    } else {
      const size_t ldv = (size_t)(S + 63) / 64 * 64;  // V^T rows padded to a multiple of 64 keys
      half* vt = ep.y + 2 * plane + (bh * hd + d) * ldv + s;
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[(size_t)e * ldv] = (half)v[e];
    }
    return;
  }
  half4 o = {(half)v[0], (half)v[1], (half)v[2], (half)v[3]};
  *(half4*)(ep.y + (size_t)m * ep.ldy + n) = o;
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_kernel(
    const half* __restrict__ X, const half* __restrict__ W, int M, int N, int K, EpiArgs ep) {
  constexpr int WAVES_N = BN / WN;
  constexpr int NT = (BM / WM) * WAVES_N * 64;
  constexpr int FN = WN / 32, FM = WM / 32;
  constexpr int XCH = BM * 8 / NT, WCH = BN * 8 / NT;
  static_assert(XCH * NT == BM * 8 && WCH * NT == BN * 8, "tile/thread mismatch");
  constexpr int STAGE = (BM + BN) * kBK;

  extern __shared__ __align__(16) half lds[];

  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WAVES_N, wm = wave / WAVES_N;

  // Thread t loads 16-byte chunk (t & 7) of rows (t >> 3) + i * (NT / 8) of both tiles.  Rows
  // past M are clamped to M-1: they load valid memory and their results are never stored.
  constexpr int RS = NT / 8;
  const int c0 = tid & 7, r0 = tid >> 3;
  const half* xbase = X + c0 * 8;
  const half* wbase = W + (size_t)(n0 + r0) * K + c0 * 8;
  int xrow[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) xrow[i] = min(m0 + r0 + i * RS, M - 1);
  u32x4 rx[XCH], rw[WCH];

  floatx16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

#define TT_GLOAD(k0)                                                                     \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < XCH; ++i)                                      \
        rx[i] = *(const u32x4*)(xbase + (size_t)xrow[i] * K + (k0));                     \
    _Pragma("unroll") for (int i = 0; i < WCH; ++i)                                      \
        rw[i] = *(const u32x4*)(wbase + (size_t)i * RS * K + (k0));                      \
  } while (0)
#define TT_LSTORE(st)                                                                    \
  do {                                                                                   \
    half* sx_ = lds + (st) * STAGE;                                                      \
    half* sw_ = sx_ + BM * kBK;                                                          \
    _Pragma("unroll") for (int i = 0; i < XCH; ++i) {                                    \
      const int row = r0 + i * RS;                                                       \
      *(u32x4*)(sx_ + row * kBK + swz(row, c0) * 8) = rx[i];                             \
    }                                                                                    \
    _Pragma("unroll") for (int i = 0; i < WCH; ++i) {                                    \
      const int row = r0 + i * RS;                                                       \
      *(u32x4*)(sw_ + row * kBK + swz(row, c0) * 8) = rw[i];                             \
    }                                                                                    \
  } while (0)
  // Fragment reads of K step kk+1 are issued before the MFMAs of step kk (two register sets);
  // scheduling barriers pin that order.
#define TT_FRAGS(buf, kk, sx, sw)                                                        \
  do {                                                                                   \
    const int c_ = 2 * (kk) + (lane >> 5);                                               \
    _Pragma("unroll") for (int i = 0; i < FN; ++i) {                                     \
      const int row = wn * WN + i * 32 + (lane & 31);                                    \
      af[buf][i] = *(const half8*)((sw) + row * kBK + swz(row, c_) * 8);                 \
    }                                                                                    \
    _Pragma("unroll") for (int j = 0; j < FM; ++j) {                                     \
      const int row = wm * WM + j * 32 + (lane & 31);                                    \
      bf[buf][j] = *(const half8*)((sx) + row * kBK + swz(row, c_) * 8);                 \
    }                                                                                    \
  } while (0)
#define TT_COMPUTE(st)                                                                   \
  do {                                                                                   \
    const half* sx_ = lds + (st) * STAGE;                                                \
    const half* sw_ = sx_ + BM * kBK;                                                    \
    half8 af[2][FN], bf[2][FM];                                                          \
    TT_FRAGS(0, 0, sx_, sw_);                                                            \
    _Pragma("unroll") for (int kk = 0; kk < kBK / 16; ++kk) {                            \
      if (kk + 1 < kBK / 16) TT_FRAGS((kk + 1) & 1, kk + 1, sx_, sw_);                   \
      __builtin_amdgcn_sched_barrier(0);                                                 \
      _Pragma("unroll") for (int i = 0; i < FN; ++i)                                     \
          _Pragma("unroll") for (int j = 0; j < FM; ++j) acc[i][j] =                     \
              mfma32x32x16(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);                     \
      __builtin_amdgcn_sched_barrier(0);                                                 \
    }                                                                                    \
  } while (0)

  // Main loop: the last K step is peeled so the body has no conditional (a conditional
  // prefetch makes the compiler spill the prefetch registers and wait on the loads at once).
  const int nk = K / kBK;
  TT_GLOAD(0);
  TT_LSTORE(0);
  __syncthreads();
  for (int kt = 0; kt < nk - 1; ++kt) {
    TT_GLOAD((kt + 1) * kBK);
    __builtin_amdgcn_sched_barrier(0);
    TT_COMPUTE(kt & 1);
    TT_LSTORE((kt + 1) & 1);
    __syncthreads();
  }
  TT_COMPUTE((nk - 1) & 1);
#undef TT_FRAGS
#undef TT_COMPUTE
#undef TT_GLOAD
#undef TT_LSTORE

  // Epilogue: acc[i][j][4g+e] = C[m][n] with m = row j*32 + lane%32 of the wave tile and
  // n = i*32 + 8g + 4*(lane/32) + e.
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + wm * WM + j * 32 + (lane & 31);
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * WN + i * 32 + 8 * g + 4 * (lane >> 5);
        epilogue4(ep, m, n, acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                  acc[i][j][4 * g + 3]);
      }
    }
  }
}

// ---- host-side tile selection ----
struct TileCfg {
  int bm, bn;
  float efficiency;  // relative per-CU MFMA efficiency of the tile shape
};

template <int BM, int BN, int WM, int WN>
static int run_tile(const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                    hipStream_t stream) {
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  const size_t lds = 2 * (size_t)(BM + BN) * kBK * sizeof(half);
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    attr_err = hipFuncSetAttribute((const void*)gemm_kernel<BM, BN, WM, WN>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  });
  if (attr_err != hipSuccess)
    return fail(TT_ERR_HIP, "hipFuncSetAttribute(gemm %dx%d): %s", BM, BN, hipGetErrorString(attr_err));
  const int tiles = ((m + BM - 1) / BM) * (n / BN);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN>), dim3(tiles), dim3(NT), lds, stream, x, w, m, n,
                     k, ep);
  return launch_status("gemm_kernel");
}

static const TileCfg kTiles[] = {
    {256, 256, 1.00f},
    {256, 128, 0.92f},
    {128, 128, 0.80f},
    {128, 64, 0.65f},
    {64, 64, 0.50f},
};

static int g_tile_override = -1;  // test hook: force one tile configuration

// Estimated time ~ (tiles per CU, rounded up) x (tile work / relative efficiency): co-resident
// blocks on one CU share its MFMA throughput, so a CU finishing k blocks costs about k blocks.
static int pick_tile(int m, int n, int cus) {
  const int count = (int)(sizeof(kTiles) / sizeof(kTiles[0]));
  if (g_tile_override >= 0 && g_tile_override < count && n % kTiles[g_tile_override].bn == 0)
    return g_tile_override;
  int best = -1;
  double best_cost = 0;
  for (int i = 0; i < count; ++i) {
    const TileCfg& t = kTiles[i];
    if (n % t.bn != 0) continue;
    const long tiles = (long)((m + t.bm - 1) / t.bm) * (n / t.bn);
    const long per_cu = (tiles + cus - 1) / cus;
    const double cost = (double)per_cu * t.bm * t.bn / t.efficiency;
    if (best < 0 || cost < best_cost * 0.999) {
      best = i;
      best_cost = cost;
    }
  }
  return best;
}

static int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
  }
  return cus;
}

int launch_linear(const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                  hipStream_t stream) {
  TT_REQUIRE(m >= 0 && n > 0 && k > 0, "linear: bad shape m=%d n=%d k=%d", m, n, k);
  TT_REQUIRE(k % kBK == 0, "linear: K=%d must be a multiple of %d", k, kBK);
  TT_REQUIRE(n % 64 == 0, "linear: N=%d must be a multiple of 64", n);
  TT_REQUIRE(ep.mode >= TT_EPI_BIAS && ep.mode <= TT_EPI_QKV, "linear: bad epilogue %d", ep.mode);
  TT_REQUIRE(ep.bias != nullptr && ep.y != nullptr, "linear: null bias/output");
  if (ep.mode == TT_EPI_RESID_MASKED || ep.mode == TT_EPI_MASKED_RESID)
    TT_REQUIRE(ep.resid != nullptr, "linear: residual epilogue needs a residual");
  if (ep.mode == TT_EPI_QKV) {
    TT_REQUIRE(ep.heads > 0 && ep.head_dim > 0 && ep.head_dim % 4 == 0 &&
                   ep.heads * ep.head_dim == ep.d_model && n == 3 * ep.d_model &&
                   (long)ep.batch * ep.seq == m,
               "linear(qkv): inconsistent shape m=%d n=%d batch=%d seq=%d heads=%d hd=%d", m, n,
               ep.batch, ep.seq, ep.heads, ep.head_dim);
  }
  if (m == 0) return TT_OK;
  switch (pick_tile(m, n, device_cus())) {
    case 0: return run_tile<256, 256, 128, 128>(x, w, m, n, k, ep, stream);
    case 1: return run_tile<256, 128, 128, 64>(x, w, m, n, k, ep, stream);
    case 2: return run_tile<128, 128, 64, 64>(x, w, m, n, k, ep, stream);
    case 3: return run_tile<128, 64, 64, 32>(x, w, m, n, k, ep, stream);
    default: return run_tile<64, 64, 32, 32>(x, w, m, n, k, ep, stream);
  }
}

}  // namespace tt

extern "C" int tt_gemm_tile_override(int index) {
  const int count = (int)(sizeof(tt::kTiles) / sizeof(tt::kTiles[0]));
  TT_REQUIRE(index >= -1 && index < count, "gemm_tile_override: index %d out of [-1, %d)", index, count);
  tt::g_tile_override = index;
  return TT_OK;
}

extern "C" int tt_linear_fwd(const void* x, const void* w, const void* bias, const void* residual,
                             const uint8_t* valid, void* y, int m, int n, int k, int epilogue,
                             int batch, int seq, int heads, void* stream) {
  TT_REQUIRE(x && w && bias && y, "linear: null pointer");
  tt::EpiArgs ep{};
  ep.bias = (const tt::half*)bias;
  ep.resid = (const tt::half*)residual;
  ep.valid = valid;
  ep.y = (tt::half*)y;
  ep.ldy = n;
  ep.mode = epilogue;
  ep.batch = batch;
  ep.seq = seq;
  ep.heads = heads;
  ep.d_model = n / 3;
  ep.head_dim = heads > 0 ? (n / 3) / heads : 0;
  return tt::launch_linear((const tt::half*)x, (const tt::half*)w, m, n, k, ep,
                           (hipStream_t)stream);
}
