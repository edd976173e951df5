// FP16 MFMA GEMM with fused epilogues: Y[M,N] = X[M,K] W[N,K]^T + b (+ GELU / residual / mask /
// head-major QKV scatter), fp32 accumulation, for the four projections of the pre-LN block.
//
// Design (gfx950):
//  * Both operands are K-contiguous (nn.Linear weights are [N,K]), so a block stages a BM x 64
//    X tile and a BN x 64 W tile in LDS per K step (128-byte rows, 16-byte chunks XOR-swizzled
//    by row bits 1-3 so ds_read_b128 fragment reads are bank-conflict free), double-buffered.
//    The copies are global_load_lds_dwordx4 (global -> LDS without a register round trip), or
//    buffer loads through VGPRs into padded rows on the register path; issued for the
//    next K step during the first half of the current one, one between consecutive MFMAs, with
//    the next k-step's fragment reads interleaved the same way (sched_group_barrier).
//  * The MFMA is v_mfma_f32_32x32x16_f16 with W as the "A" operand and X as "B", i.e. each wave
//    accumulates C^T: lane l then holds 4 consecutive output features of one token per group.
//    The epilogue (bias, GELU, residual, row mask, QKV head-major scatter) stages each wave's
//    tile through LDS and writes whole rows with 16-byte stores.
//  * Block-id -> tile mapping is XCD-aware: workgroup i runs on XCD i % 8, so each XCD is given
//    a contiguous range of tile ids, and tiles are ordered in groups of 8 row-tiles so the tiles
//    one XCD runs at once share X row panels and W column panels in that XCD's L2.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

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

// Row-tile order for masked launches.  The XCD-aware mapping hands each XCD a contiguous range of
// row tiles, which for right-padded batches is whole sequences: the XCD with the longest sequence
// would then set the time while padded tiles elsewhere finish early.  With S a multiple of BM,
// row tile (q, p) (sequence q, position p) is visited in diagonal order -- list index
// L = d * nseq + q holds (q, (q + d) mod P) -- so every XCD's range mixes positions of different
// sequences and the skipped (padded) tiles spread over all XCDs.  A bijection on [0, tiles_m).
__device__ __forceinline__ int balance_row_tile(int tm, int tiles_m, int seq, int bm) {
  if (seq <= 0 || seq % bm != 0) return tm;
  const int P = seq / bm;             // row tiles per sequence
  if (tiles_m % P != 0) return tm;
  const int nseq = tiles_m / P;
  const int d = tm / nseq, q = tm - d * nseq;
  return q * P + (q + d) % P;
}

// Scalar store of 4 consecutive output features n..n+3 of row m into the QKV layout (used only
// for the V^T part when tokens of one 8-row group may belong to two sequences, S % 8 != 0).
__device__ __forceinline__ void store_vt4(const EpiArgs& ep, int m, int n, half4 h) {
  const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
  const int nn = n - 2 * D;
  const int hh = nn / hd, d = nn - hh * hd;
  const int bb = m / S, s = m - bb * S;
  const size_t plane = (size_t)ep.batch * S * D;
  const size_t ldv = (size_t)(S + 63) / 64 * 64;
  half* vt = ep.y + 2 * plane + (((size_t)bb * ep.heads + hh) * hd + d) * ldv + s;
#pragma unroll
  for (int e = 0; e < 4; ++e) vt[(size_t)e * ldv] = h[e];
}

__device__ __forceinline__ half8 swap_halves(half8 t) {
  return half8{t[4], t[5], t[6], t[7], t[0], t[1], t[2], t[3]};
}

// Output of a tile whose rows are all padded (valid == 0): no MMA work, only the fill values the
// epilogue would produce for masked rows -- the residual for TT_EPI_RESID_MASKED (the masked
// branch adds nothing), +0.0 for every other mode.  16-byte stores over the tile's BM x BN block
// (for the V part of the QKV projection: V^T rows, 8 tokens at a time when they share a sequence).
template <int BM, int BN, int MODE>
__device__ void fill_padded_tile(const EpiArgs& ep, int M, int m0, int n0) {
  constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
  const u32x4 zero = {0u, 0u, 0u, 0u};
  if constexpr (MODE == TT_EPI_QKV) {
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
    const size_t plane = (size_t)ep.batch * S * D;
    if (n0 < 2 * D) {  // Q or K rows: 8 features of one head of token m per chunk
      for (int e = threadIdx.x; e < BM * CPR; e += blockDim.x) {
        const int m = m0 + e / CPR, n = n0 + 8 * (e % CPR);
        if (m >= M) continue;
        const int which = n / D, nn = n - which * D;
        const int hh = nn / hd, d = nn - hh * hd;
        const int bb = m / S, sq = m - bb * S;
        *(u32x4*)(ep.y + which * plane + (((size_t)bb * ep.heads + hh) * S + sq) * hd + d) = zero;
      }
    } else {           // V^T: feature row n, tokens m .. m + 7
      const size_t ldv = (size_t)(S + 63) / 64 * 64;
      for (int e = threadIdx.x; e < BN * (BM / 8); e += blockDim.x) {
        const int n = n0 + e / (BM / 8), m = m0 + 8 * (e % (BM / 8));
        const int nn = n - 2 * D, hh = nn / hd, d = nn - hh * hd;
        half* row = ep.y + 2 * plane + ((size_t)hh * hd + d) * ldv;
        const int bb = m / S, sq = m - bb * S;
        if (S % 8 == 0 && m + 8 <= M) {
          *(u32x4*)(row + (size_t)bb * ep.heads * hd * ldv + sq) = zero;
        } else {
          for (int t = m; t < min(m + 8, M); ++t) {
            const int b2 = t / S, s2 = t - b2 * S;
            row[(size_t)b2 * ep.heads * hd * ldv + s2] = (half)0.f;
          }
        }
      }
    }
  } else {
    for (int e = threadIdx.x; e < BM * CPR; e += blockDim.x) {
      const int m = m0 + e / CPR, c = 8 * (e % CPR);
      if (m >= M) continue;
      half* dst = ep.y + (size_t)m * ep.ldy + n0 + c;
      if constexpr (MODE == TT_EPI_RESID_MASKED) {
        const half* src = ep.resid + (size_t)m * ep.ldy + n0 + c;
        if (src != dst) *(u32x4*)dst = *(const u32x4*)src;
      } else {
        *(u32x4*)dst = zero;
      }
    }
  }
}

// LDS tile of R rows x 64 halfs (128-byte rows) holding a K slice of one operand.  Global ->
// LDS copies use global_load_lds_dwordx4: one instruction moves 1 KiB, lane l writing LDS bytes
// [16 l, 16 l + 16) of an 8-row group, i.e. row l / 8, physical chunk l % 8.  The chunk swizzle is
// applied on the global side: lane l fetches logical chunk (l % 8) ^ ((r >> 1) % 8) of its row r,
// so the physical chunk of logical chunk c in row r is c ^ ((r >> 1) % 8).

// Register-path staging (PATH = 1): each thread moves 16-byte chunks global -> VGPR -> LDS with
// buffer loads and ds_write_b128, two K stages ahead in two register sets, so a CU keeps three K
// stages of operands in flight instead of one.  That is what a grid of about one tile per CU
// streaming a long K needs (its time is the latency of the bytes each CU has in flight); with
// several tiles per CU the direct global -> LDS copies (PATH = 0) are as fast.  (buffer_rsrc:
// common.hpp.)

// Blocks of NW waves (4: a 2 x 2 wave grid; 8: 4 x 2, i.e. four waves along M), each wave owning
// a (BM / (NW / 2)) x (BN / 2) block of C as FM x FN 32x32 MFMA tiles.  Two 4-wave blocks of up to
// 128 x 128 share a CU (one's epilogue runs beside the other's main loop); an 8-wave block puts two
// waves on every SIMD by itself.
// K stages in the LDS ring: three for the 8-wave 256 x 128 direct-copy tile (3 x 48 KiB), so a
// stage's copies are issued two stages before it is read; two for every other tile.
constexpr int gemm_stages(int bm, int bn, int path, int nw) {
  return (path == 0 && nw == 8 && bm * bn <= 256 * 128) ? 3 : 2;
}
// LDS row stride (halfs) of a staged operand row: 128-byte rows (direct copies, XOR-swizzled) or
// 144-byte padded rows (register path).
constexpr int gemm_ldr(int path) { return path == 1 ? kBK + 8 : kBK; }

template <int BM, int BN, int MODE, int PATH, int NW = 4>
__global__ __launch_bounds__(64 * NW, (NW == 4 && BM * BN <= 128 * 128) ? 2 : 1) void gemm_kernel(
    const half* __restrict__ X, const half* __restrict__ W, int M, int N, int K, EpiArgs ep) {
  constexpr int NS = gemm_stages(BM, BN, PATH, NW);
  constexpr int WGM = NW / 2;
  constexpr int WM = BM / WGM, WN = BN / 2;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int ROWS = BM + BN;       // LDS rows per stage: X rows [0, BM), W rows [BM, BM + BN)
  // LDS row stride in halfs: 128-byte rows with XOR-swizzled chunks for the direct copies (one
  // copy instruction fills 1 KiB contiguously, so rows cannot be padded); rows padded to 144 bytes
  // and unswizzled on the register path.  Either way the 16 rows one ds_read_b128 phase reads fall
  // in 16 different bank groups.
  constexpr int LDR = gemm_ldr(PATH);
  constexpr int STAGE = ROWS * LDR;   // halfs per stage
  static_assert(PATH != 1 || NW == 4, "the register path is laid out for 4 waves");
  constexpr int XL = BM / (8 * NW);   // X copies per wave per stage (8 rows each)
  constexpr int WL = BN / (8 * NW);   // W copies per wave per stage
  constexpr int NL = XL + WL;
  constexpr int KSUB = kBK / 16;      // MFMA k-steps per stage
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "copy split");

  extern __shared__ __align__(16) half lds[];

  // Packed variable-length rows: the grid covers the M the launch was sized for, the live rows
  // are *ep.m_dev; blocks past the live tiles leave at once, and the live tiles keep the
  // XCD-aware order among themselves (their count rounded up to the 8 XCDs).
  if (ep.m_dev != nullptr) M = __builtin_amdgcn_readfirstlane(min(M, *ep.m_dev));
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  int tile_id;
  if (ep.m_dev != nullptr) {
    const int live = tiles_m * tiles_n, live8 = (live + 7) & ~7;
    if ((int)blockIdx.x >= live8) return;
    tile_id = xcd_remap(blockIdx.x, live8);
    if (tile_id >= live) return;
  } else {
    tile_id = xcd_remap(blockIdx.x, gridDim.x);
  }
  int tm, tn;
  tile_coords(tile_id, tiles_m, tiles_n, tm, tn);
  if (ep.valid != nullptr && ep.m_dev == nullptr) tm = balance_row_tile(tm, tiles_m, ep.seq, BM);
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wn = wave & 1, wm = wave >> 1;

  // Padded-row skip: with a row mask, a tile whose rows are all padded (e.g. the tail of a
  // right-padded sequence) does no MMA work.  (Packed rows hold at most 7 padded rows in a row,
  // and their fill would need the row map: not taken there.)
  if (ep.valid != nullptr && ep.m_dev == nullptr) {
    int v = 0;
    if ((int)threadIdx.x < BM && m0 + (int)threadIdx.x < M) v = ep.valid[m0 + threadIdx.x];
    if (!__syncthreads_or(v)) {
      fill_padded_tile<BM, BN, MODE>(ep, M, m0, n0);
      return;
    }
  }

  floatx16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // The block's bias slice goes to LDS once, as fp32 (made visible by the prologue's barrier).
  __shared__ __align__(16) float sbias[BN];
  if (threadIdx.x < BN / 4) {
    const half4 b = *(const half4*)(ep.bias + n0 + 4 * threadIdx.x);
    *(floatx4*)(sbias + 4 * threadIdx.x) = floatx4{(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
  }
  constexpr bool ZERO_MASKED = MODE == TT_EPI_BIAS || MODE == TT_EPI_BIAS_GELU || MODE == TT_EPI_QKV;

  // Fragment addressing: A = W rows (output features), B = X rows (tokens); lane l reads row
  // l % 32 of a 32-row block at logical chunk 2 kk + l / 32, physically XOR bits 1-3 of the row
  // (the direct-copy layout below).
  const int frow = lane & 31, fhi = lane >> 5, fx = (lane >> 1) & 7;
  half8 af[2][FN], bf[2][FM];
  auto frags = [&](int buf, int kk, const half* stage) {
    const int pc = PATH ? 2 * kk + fhi : (2 * kk + fhi) ^ fx;
#pragma unroll
    for (int i = 0; i < FN; ++i)
      af[buf][i] = *(const half8*)(stage + (BM + wn * WN + i * 32 + frow) * LDR + pc * 8);
#pragma unroll
    for (int j = 0; j < FM; ++j)
      bf[buf][j] = *(const half8*)(stage + (wm * WM + j * 32 + frow) * LDR + pc * 8);
  };

  if constexpr (PATH == 0) {
    // Copy sources: copy i of this wave fills 8-row group wave + NW i of the stage.  X rows past M
    // are clamped to M - 1 (valid memory whose results are never stored).
    // Offsets are relative to the block's first X row and W row (64-bit bases), so M * K may
    // exceed 2^31 (long sequences); BM * K and BN * K stay far below it.
    // Chunk layout: physical chunk = logical ^ bits 1-3 of the row, so that the 16 consecutive rows
    // one ds_read_b128 phase reads land in 16 different bank groups (with bits 0-2, rows r and
    // r + 8 would share banks).  Row (wave + NW i) * 8 + lrow has bits 1-3 = (wave & 1) << 2 |
    // lrow >> 1 for every i (NW is even).
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ (((wave & 1) << 2) | (lrow >> 1));
    const half* Xb = X + (size_t)m0 * K;
    const half* Wb = W + (size_t)n0 * K;
    const int nk = K / kBK;
    int src_off[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int r = (wave + NW * i) * 8 + lrow;
      if (i < XL) src_off[i] = min(r, M - 1 - m0) * K + lchunk * 8;
      else src_off[i] = (r - BM) * K + lchunk * 8;
    }
    // The wave index is made provably uniform so the LDS destination (M0) is scalar arithmetic;
    // the source is a uniform base advanced by k0 plus the lane's fixed 32-bit offset, which
    // lets the copy use the scalar-base addressing mode (no per-copy 64-bit VALU adds).  Copies
    // of stages past the last one re-read the last stage into the buffer nobody reads any more,
    // so that no copy sits behind a branch: every k-step below is one basic block, which the
    // interleaving hints need.
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    auto copy = [&](int i, int kt, half* stage) {
      const half* base = ((i < XL) ? Xb : Wb) + min(kt, nk - 1) * kBK;
      lds_copy16(base + (uint32_t)src_off[i], stage + (wave_u + NW * i) * 8 * kBK);
    };

    // Copies of the next stage per k-step: C0 in the first (they have the whole stage to land),
    // the rest spread evenly over the others, so that no wave issues a burst of copies (each one
    // holds the wave's issue for ~100 cycles when the CU's copy queue is busy).  The 8-wave
    // 256 x 256 block (two stages) issues all of them in the first k-step, since they have one
    // stage to land; with the three-stage ring a copy has two stages, and one copy in the first
    // k-step, the rest spread (1, 2, 2, 1 for 256 x 128), keeps the two waves of a SIMD from
    // blocking together (measured on MI355X: C5 out_proj 24.2 -> 23.3, ffn_out 68.9 -> 65.8 us;
    // spreading the two-stage block's copies slows ffn_in by 6-10%).
    constexpr int C0 = NW == 8 ? (NS == 3 ? 1 : NL) : (NL + 3) / 4;
    constexpr int CPER = (NL - C0 + KSUB - 2) / (KSUB - 1);
    // One stage: KSUB k-steps of FN x FM MFMAs; the next k-step's fragment reads and this
    // k-step's copies of stage kn are interleaved one per MFMA.
    auto stage = [&](const half* cur, half* nxt, int kn) {
      frags(0, 0, cur);
#pragma unroll
      for (int kk = 0; kk < KSUB; ++kk) {
        __builtin_amdgcn_sched_barrier(0);
        if (kk + 1 < KSUB) frags((kk + 1) & 1, kk + 1, cur);
        const int c_lo = kk == 0 ? 0 : min(NL, C0 + (kk - 1) * CPER);
        const int c_hi = kk == 0 ? C0 : min(NL, C0 + kk * CPER);
#pragma unroll
        for (int c = c_lo; c < c_hi; ++c) copy(c, kn, nxt);
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = mfma32x32x16(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);
        const int nds = kk + 1 < KSUB ? FN + FM : 0;
#pragma unroll
        for (int t = 0; t < FN * FM; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
          if (t < nds) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // DS read
          if (t < c_hi - c_lo) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // copy
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    if constexpr (NS == 2) {
      // Prologue: stage 0.  Then two stages per iteration, so both buffers are constant offsets
      // (fragment reads use immediate offsets).  Before each stage: its copies have landed in LDS
      // (vmcnt 0: every copy of this wave is older than the ones the stage issues) and every wave
      // is done reading the buffer the stage's own copies overwrite.
#pragma unroll
      for (int i = 0; i < NL; ++i) copy(i, 0, lds);
      int kt = 0;
      for (; kt + 2 <= nk; kt += 2) {
        wait_vmcnt<0>();
        raw_barrier();
        stage(lds, lds + STAGE, kt + 1);
        wait_vmcnt<0>();
        raw_barrier();
        stage(lds + STAGE, lds, kt + 2);
      }
      if (kt < nk) {
        wait_vmcnt<0>();
        raw_barrier();
        stage(lds, lds + STAGE, kt + 1);
      }
    } else {
      // Three-buffer ring, three stages per iteration (constant buffers again).  Stage kt reads
      // buffer kt % 3 and issues the copies of stage kt + 2 into buffer (kt + 2) % 3, the one stage
      // kt - 1 read.  Before stage kt each wave waits until at most NL of its copies are in flight
      // (those of stage kt + 1; copies complete in issue order), and the barrier makes every
      // wave's copies of stage kt visible and frees the buffer of stage kt - 1.  Copies past the
      // last stage re-read it into a buffer no remaining stage reads: (kt + 2) % 3 differs from
      // (nk - 1) % 3 for kt = nk - 2 and nk - 1.
      half* const s0 = lds;
      half* const s1 = lds + STAGE;
      half* const s2 = lds + 2 * STAGE;
#pragma unroll
      for (int i = 0; i < NL; ++i) copy(i, 0, s0);
#pragma unroll
      for (int i = 0; i < NL; ++i) copy(i, 1, s1);
      int kt = 0;
      for (; kt + 3 <= nk; kt += 3) {
        wait_vmcnt<NL>();
        raw_barrier();
        stage(s0, s2, kt + 2);
        wait_vmcnt<NL>();
        raw_barrier();
        stage(s1, s0, kt + 3);
        wait_vmcnt<NL>();
        raw_barrier();
        stage(s2, s1, kt + 4);
      }
      if (kt < nk) {
        wait_vmcnt<NL>();
        raw_barrier();
        stage(s0, s2, kt + 2);
      }
      if (kt + 1 < nk) {
        wait_vmcnt<NL>();
        raw_barrier();
        stage(s1, s0, kt + 3);
      }
    }
    wait_vmcnt<0>();  // the re-read copies past the end land before the epilogue reuses LDS

  } else {
    // Register path.  Thread t moves chunk t % 8 of rows t / 8 + 32 i (i < RX: X rows, then W
    // rows) of every stage.  The buffers start at the block's first X / W row, so offsets stay
    // below BM * K and BN * K; X rows past M are clamped to M - 1 (valid memory whose results are
    // never stored), so no load depends on the buffer's range check.
    constexpr int RL = (BM + BN) / 32;   // 16-byte chunks per thread per stage
    constexpr int RX = BM / 32;
    const int tid = threadIdx.x;
    const int lr = tid >> 3, lc = tid & 7;
    // The tile origin is wave-uniform; readfirstlane states it, so the buffer descriptors live in
    // SGPRs (after the padded-tile early return the compiler cannot prove it, and a descriptor in
    // VGPRs turns every load into a waterfall loop).
    const int m0u = __builtin_amdgcn_readfirstlane(m0), n0u = __builtin_amdgcn_readfirstlane(n0);
    const int xrows = min(M - m0u, BM);
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X + (size_t)m0u * K, xrows * K * 2);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W + (size_t)n0u * K, BN * K * 2);
    int roff[RL];  // byte offset of the thread's chunk in K stage 0
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      const int r = i < RX ? min(lr + 32 * i, xrows - 1) : lr + 32 * (i - RX);
      roff[i] = (r * K + lc * 8) * 2;
    }
    const int dst0 = lr * LDR + lc * 8;
    const int nk = K / kBK;
    // chunk i of K stage kt (stages past the end re-read the last one; never used)
    auto ld = [&](int i, int kt) -> u32x4 {
      const int kb = min(kt, nk - 1) * (kBK * 2);
      return __builtin_amdgcn_raw_buffer_load_b128(i < RX ? xr : wr, roff[i] + kb, 0, 0);
    };
    u32x4 sa[RL], sb[RL];
#pragma unroll
    for (int i = 0; i < RL; ++i) sa[i] = ld(i, 0);
#pragma unroll
    for (int i = 0; i < RL; ++i) sb[i] = ld(i, 1);
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      *(u32x4*)(lds + dst0 + i * 32 * LDR) = sa[i];
      sa[i] = ld(i, 2);
    }
    lds_barrier();
    // Stage kt: MFMAs on LDS buffer kt % 2; the chunks of stage kt + 1 (in S) go to the other
    // buffer during the first two k-steps, each followed by the load of stage kt + 3 into its
    // register.  The body has no branches, so the MFMAs, fragment reads, LDS writes and loads
    // interleave one per MFMA.
    auto body = [&](int kt, u32x4 (&S)[RL]) {
      const half* cur = lds + (kt & 1) * STAGE;
      half* nxt = lds + ((kt + 1) & 1) * STAGE;
      frags(0, 0, cur);
#pragma unroll
      for (int kk = 0; kk < KSUB; ++kk) {
        __builtin_amdgcn_sched_barrier(0);
        if (kk + 1 < KSUB) frags((kk + 1) & 1, kk + 1, cur);
        constexpr int PER = (RL + 1) / 2;
        const int lo = kk < 2 ? kk * PER : RL, hi = kk < 2 ? min(RL, (kk + 1) * PER) : RL;
#pragma unroll
        for (int i = lo; i < hi; ++i) {
          *(u32x4*)(nxt + dst0 + i * 32 * LDR) = S[i];
          S[i] = ld(i, kt + 3);
        }
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = mfma32x32x16(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);
        if (kk + 1 < KSUB) {
#pragma unroll
          for (int t = 0; t < FN + FM; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
#pragma unroll
        for (int t = lo; t < hi; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, FN * FM, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      lds_barrier();
    };
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
      body(kt, sb);
      body(kt + 1, sa);
    }
    if (kt < nk) body(kt, sb);
  }

  // ---- Epilogue ----
  // acc[i][j][4g+e] = C[m][n] with m = row j*32 + lane%32 of the wave tile and
  // n = i*32 + 8g + 4*(lane/32) + e.  Each wave stages its WM x WN tile of fp16(acc + bias
  // [, GELU]) in its own LDS area and then writes whole rows with 16-byte stores (residual and
  // mask applied on the way out), so every store instruction writes full 128-byte lines.
  // Row-major staging is swizzled in 8-byte units: unit u of row r lives at u ^ (r & SWM), which
  // keeps the 8-byte writes of 32 consecutive rows and the 16-byte row reads conflict-free.  The
  // V part of the QKV projection is staged transposed ([n][m]) and written as V^T rows.
  __syncthreads();  // every wave is done with the last stage's fragments
  half* cst = lds + wave * (WM * WN);
  constexpr int UNITS = WN / 4;
  constexpr int SWM = (UNITS >= 16 ? 16 : UNITS) - 1;
  const int mw = m0 + wm * WM, nw = n0 + wn * WN;  // wave tile origin
  bool vt_mode = false, vt_scalar = false;
  if constexpr (MODE == TT_EPI_QKV) {
    vt_mode = n0 >= 2 * ep.d_model;   // tiles never straddle the Q / K / V boundaries
    vt_scalar = vt_mode && ep.rowmap == nullptr && (ep.seq % 8 != 0);
  }
  // Modes without a residual write masked rows as +0.0 (the residual modes handle the mask
  // when they store).
  float qs = 1.f;  // Q columns of the QKV projection carry ep.q_scale
  if constexpr (MODE == TT_EPI_QKV) qs = n0 < ep.d_model ? ep.q_scale : 1.f;
  bool keep[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    keep[j] = true;
    if constexpr (ZERO_MASKED)
      keep[j] = ep.valid == nullptr || ep.valid[min(mw + j * 32 + (lane & 31), M - 1)] != 0;
  }
  // Columns outermost: each lane reads its 4 bias values of a column group once for all FM rows.
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = i * 32 + 8 * g + 4 * (lane >> 5);
      const floatx4 bv = *(const floatx4*)(sbias + wn * WN + nl);
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int ml = j * 32 + (lane & 31);
        half4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[i][j][4 * g + e] + bv[e];
          if constexpr (MODE == TT_EPI_BIAS_GELU) v = gelu_erf(v);
          if constexpr (MODE == TT_EPI_QKV) v *= qs;
          h[e] = keep[j] ? (half)v : (half)0.f;
        }
        if (vt_scalar) {
          if (mw + ml < M) store_vt4(ep, mw + ml, nw + nl, h);
        } else if (vt_mode) {
#pragma unroll
          for (int e = 0; e < 4; ++e) cst[(nl + e) * WM + ml] = h[e];
        } else {
          const int u = nl >> 2;
          *(half4*)(cst + ml * WN + ((u ^ (ml & SWM)) << 2)) = h;
        }
      }
    }
  }
  if (vt_scalar) return;
  __builtin_amdgcn_s_waitcnt(0);  // wave-local staging: the LDS writes above precede the reads

  if (vt_mode) {
    // V^T rows: staged row nl holds WM consecutive tokens of feature nw + nl.  S % 8 == 0 here,
    // so an aligned group of 8 tokens lies in one sequence and M is a multiple of 8.
    // The lane's 8 tokens (m .. m + 7) are fixed, so their (sequence, position) is one division;
    // the feature row advances by RPI per iteration and its (head, feature) pair is stepped
    // instead of divided (integer division is a ~20-instruction VALU sequence).
    constexpr int CPR = WM / 8, RPI = 64 / CPR;
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
    const size_t plane = (size_t)ep.batch * S * D;
    const size_t ldv = (size_t)(S + 63) / 64 * 64;
    const int c = lane % CPR, m = mw + 8 * c;
    if (m >= M) return;
    half* vbase;
    // Packed rows: the lane's 8 rows are 8 consecutive tokens of one sequence, starting on an
    // 8-token boundary (the packed layout pads every sequence to 8 rows), unless the batch's mask
    // is not a prefix or the packed rows end inside the group; then each token is stored alone.
    bool vec = true;
    int voffs[8];
    if (ep.rowmap != nullptr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) voffs[e] = ep.rowmap[min(m + e, M - 1)].y;
      vec = m + 8 <= M && voffs[7] == voffs[0] + 7 && voffs[0] % 8 == 0;
      vbase = ep.y + 2 * plane + voffs[0];
    } else {
      const int bb = m / S, sq = m - bb * S;
      vbase = ep.y + 2 * plane + (size_t)bb * ep.heads * hd * ldv + sq;
    }
    const int nn0 = nw + lane / CPR - 2 * D;
    int hh = nn0 / hd, d = nn0 - hh * hd;
#pragma unroll 4
    for (int it = 0; it < WN / RPI; ++it) {
      const int r = it * RPI + lane / CPR;
      const half8 t = *(const half8*)(cst + r * WM + 8 * c);
      const size_t frow = ((size_t)hh * hd + d) * ldv;
      if (vec) {
        *(half8*)(vbase + frow) = t;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (m + e < M) ep.y[2 * plane + (size_t)voffs[e] + frow] = t[e];
      }
      d += RPI;
      while (d >= hd) {  // at most RPI / hd + 1 steps
        d -= hd;
        ++hh;
      }
    }
    return;
  }

  // Row-major tile: CPR 16-byte chunks per row, RPI rows per wave instruction, processed in
  // batches of NB instructions whose residual / mask loads are all issued before any store.
  constexpr int CPR = WN / 8, RPI = 64 / CPR, NIT = WM / RPI;
  constexpr int NB = NIT < 8 ? NIT : 8;
  constexpr bool RESID = MODE == TT_EPI_RESID_MASKED || MODE == TT_EPI_MASKED_RESID;
  const int c = lane % CPR;
  // Q / K destinations, [B, H, S, hd]: the lane's 8 features (one head) are fixed, so the column
  // part is one base pointer; the row m = mw + r advances by RPI per store and its (sequence,
  // position) pair is stepped (one wrap per store once S >= RPI) instead of divided.
  [[maybe_unused]] half* qk_col = nullptr;
  [[maybe_unused]] int qk_sq = 0;
  [[maybe_unused]] size_t qk_row = 0;  // ((b H) S + sq) hd for the current row
  if constexpr (MODE == TT_EPI_QKV) {
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
    const int n = nw + 8 * c;
    const int which = n / D, nn = n - which * D;
    const int hh = nn / hd, d = nn - hh * hd;
    qk_col = ep.y + which * ((size_t)ep.batch * S * D) + (size_t)hh * S * hd + d;
    const int m = mw + lane / CPR;
    const int bb = m / S;
    qk_sq = m - bb * S;
    qk_row = ((size_t)bb * ep.heads * S + qk_sq) * hd;
  }
#pragma unroll
  for (int b0 = 0; b0 < NIT; b0 += NB) {
    half8 rv[NB];
    bool ok[NB];
    if constexpr (RESID) {
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        const int m = min(mw + (b0 + q) * RPI + lane / CPR, M - 1);
        ok[q] = ep.valid == nullptr || ep.valid[m] != 0;
        rv[q] = *(const half8*)(ep.resid + (size_t)m * ep.ldy + nw + 8 * c);
      }
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int r = (b0 + q) * RPI + lane / CPR;
      const int m = mw + r;
      const int sw = r & SWM;
      half8 t = *(const half8*)(cst + r * WN + (((2 * c) ^ (sw & ~1)) << 2));
      if (sw & 1) t = swap_halves(t);
      [[maybe_unused]] size_t row_off = 0;
      if constexpr (MODE == TT_EPI_QKV) {
        if (ep.rowmap != nullptr) {  // packed rows: the token's row offset from the map
          row_off = (size_t)ep.rowmap[min(m, M - 1)].x;
        } else {
          row_off = qk_row;
          const int S = ep.seq, hd = ep.head_dim;
          qk_sq += RPI;
          qk_row += (size_t)RPI * hd;
          while (qk_sq >= S) {  // next row crosses into the next sequence
            qk_sq -= S;
            qk_row += (size_t)(ep.heads - 1) * S * hd;
          }
        }
      }
      if constexpr (RESID) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (MODE == TT_EPI_RESID_MASKED)
            t[e] = ok[q] ? (half)((float)rv[q][e] + (float)t[e]) : rv[q][e];
          else
            t[e] = ok[q] ? (half)((float)rv[q][e] + (float)t[e]) : (half)0.f;
        }
        if (ep.part_out != nullptr) {
          // partial (mean, M2) of this row over the wave's WN columns (CPR lanes, aligned):
          // the statistics of the next LayerNorm, folded into the next projection
          float f[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = (float)t[e];
          const float2 st = slot_stats<CPR, 8>(f);
          if (c == 0 && m < M) ep.part_out[(size_t)m * ep.ln_stride + nw / WN] = st;
        }
      }
      if (m >= M) continue;
      half* dst;
      if constexpr (MODE == TT_EPI_QKV) {
        dst = qk_col + row_off;  // Q or K: 8 features of one head of token m
      } else {
        dst = ep.y + (size_t)m * ep.ldy + nw + 8 * c;
      }
      *(half8*)dst = t;
    }
  }
}

// Epilogue of 4 consecutive outputs n .. n + 3 of row m from their fp32 sums (the semantics of
// gemm_kernel's epilogue, element by element), for the small-shape and narrow-tile kernels.
// G lanes (aligned) share a row and hold consecutive 4-column groups of it: with ep.part_out,
// they write the partial statistics slot of their 4 G columns; with ep.ln_part, K is the row
// length of the folded LayerNorm.
// Folded-LayerNorm inputs of one thread's 4 outputs, loaded before the GEMM's K loop so their
// latency overlaps it: the row's (mean, rstd) and the 4 columns' c and b'.
struct LnPre {
  float2 rs;
  floatx4 c, b;
};

template <int MODE, int G>
__device__ __forceinline__ LnPre ln_pre4(const EpiArgs& ep, int m, int n, int K) {
  LnPre p{};
  constexpr bool ZERO_MASKED = MODE == TT_EPI_BIAS || MODE == TT_EPI_BIAS_GELU || MODE == TT_EPI_QKV;
  if (ZERO_MASKED && ep.ln_part != nullptr) {
    p.rs = combine_row_stats_group<G>(ep.ln_part + (size_t)m * ep.ln_stride, ep.ln_slots, K);
    p.c = *(const floatx4*)(ep.ln_colsum + n);
    p.b = *(const floatx4*)(ep.ln_bias + n);
  }
  return p;
}

template <int MODE, int G>
__device__ __forceinline__ void epilogue4(const EpiArgs& ep, int m, int n, const float acc[4],
                                          const LnPre& pre) {
  const bool keep = ep.valid == nullptr || ep.valid[m] != 0;
  half4 hv;
  constexpr bool ZERO_MASKED = MODE == TT_EPI_BIAS || MODE == TT_EPI_BIAS_GELU || MODE == TT_EPI_QKV;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v;
    if (ZERO_MASKED && ep.ln_part != nullptr)
      v = fmaf(pre.rs.y, fmaf(-pre.rs.x, pre.c[e], acc[e]), pre.b[e]);
    else
      v = acc[e] + (float)ep.bias[n + e];
    if constexpr (MODE == TT_EPI_BIAS_GELU) v = gelu_erf(v);
    if constexpr (MODE == TT_EPI_QKV) v *= n < ep.d_model ? ep.q_scale : 1.f;
    hv[e] = (half)v;
  }
  if constexpr (MODE == TT_EPI_QKV) {
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq;
    const size_t plane = (size_t)ep.batch * S * D;
    const int bb = m / S, sq = m - bb * S;
    if (!keep) hv = half4{(half)0.f, (half)0.f, (half)0.f, (half)0.f};
    const int which = n / D, nn = n - which * D;
    const int hh = nn / hd, d = nn - hh * hd;  // hd % 4 == 0: the 4 outputs share a head
    if (which < 2) {
      *(half4*)(ep.y + which * plane + (((size_t)bb * ep.heads + hh) * S + sq) * hd + d) = hv;
    } else {
      const size_t ldv = (size_t)(S + 63) / 64 * 64;
      half* vt = ep.y + 2 * plane + (((size_t)bb * ep.heads + hh) * hd + d) * ldv + sq;
#pragma unroll
      for (int e = 0; e < 4; ++e) vt[(size_t)e * ldv] = hv[e];
    }
  } else {
    half* dst = ep.y + (size_t)m * ep.ldy + n;
    if constexpr (MODE == TT_EPI_RESID_MASKED || MODE == TT_EPI_MASKED_RESID) {
      const half4 rv = *(const half4*)(ep.resid + (size_t)m * ep.ldy + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (MODE == TT_EPI_RESID_MASKED)
          hv[e] = keep ? (half)((float)rv[e] + (float)hv[e]) : rv[e];
        else
          hv[e] = keep ? (half)((float)rv[e] + (float)hv[e]) : (half)0.f;
      }
      if (ep.part_out != nullptr) {
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = (float)hv[e];
        const float2 st = slot_stats<G, 4>(f);
        if ((threadIdx.x & (G - 1)) == 0) ep.part_out[(size_t)m * ep.ln_stride + n / (4 * G)] = st;
      }
    } else if (!keep) {
      hv = half4{(half)0.f, (half)0.f, (half)0.f, (half)0.f};
    }
    *(half4*)dst = hv;
  }
}

// Small-shape GEMM for projections whose N or K is not a multiple of 64 (d_model 32 and the
// like): one thread computes 4 consecutive outputs of one row with fp32 FMAs, 16-byte loads of
// X and W rows (K % 8 == 0), and the same epilogue semantics as gemm_kernel, element by element.
// These shapes are a few MFLOP; the MFMA tiles are kept for everything else.
template <int MODE>
__global__ __launch_bounds__(256) void gemm_small_kernel(const half* __restrict__ X,
                                                         const half* __restrict__ W, int M, int N,
                                                         int K, EpiArgs ep) {
  const int ngroups = N / 4;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long)M * ngroups) return;
  const int m = (int)(g / ngroups), n = (int)(g - (long)m * ngroups) * 4;
  const LnPre pre = ln_pre4<MODE, 1>(ep, m, n, K);
  const half* xr = X + (size_t)m * K;
  const half* wr = W + (size_t)n * K;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < K; k += 8) {
    const half8 xv = *(const half8*)(xr + k);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const half8 wv = *(const half8*)(wr + (size_t)e * K + k);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[e] = fmaf((float)xv[t], (float)wv[t], acc[e]);
    }
  }
  epilogue4<MODE, 1>(ep, m, n, acc, pre);
}

static int run_small(int mode, const half* x, const half* w, int m, int n, int k,
                     const EpiArgs& ep, hipStream_t stream) {
  const long threads = (long)m * (n / 4);
  const long blocks = (threads + 255) / 256;
  TT_REQUIRE(blocks < (1L << 31), "linear: grid too large");
  const dim3 grid((unsigned)blocks), block(256);
  switch (mode) {
    case TT_EPI_BIAS:
      hipLaunchKernelGGL(gemm_small_kernel<TT_EPI_BIAS>, grid, block, 0, stream, x, w, m, n, k, ep);
      break;
    case TT_EPI_BIAS_GELU:
      hipLaunchKernelGGL(gemm_small_kernel<TT_EPI_BIAS_GELU>, grid, block, 0, stream, x, w, m, n, k, ep);
      break;
    case TT_EPI_RESID_MASKED:
      hipLaunchKernelGGL(gemm_small_kernel<TT_EPI_RESID_MASKED>, grid, block, 0, stream, x, w, m, n, k, ep);
      break;
    case TT_EPI_MASKED_RESID:
      hipLaunchKernelGGL(gemm_small_kernel<TT_EPI_MASKED_RESID>, grid, block, 0, stream, x, w, m, n, k, ep);
      break;
    default:
      hipLaunchKernelGGL(gemm_small_kernel<TT_EPI_QKV>, grid, block, 0, stream, x, w, m, n, k, ep);
      break;
  }
  return launch_status("gemm_small_kernel");
}

// Narrow-tile GEMM for grids that would leave most CUs idle (few tokens): 32 x 32 output tiles, so
// four times as many blocks as 64 x 64 tiles pull operands (each CU's streaming rate is set by the
// bytes it keeps in flight), with the K range split over the block's NW waves.  Each wave loads
// its W and X fragments straight into registers (lane l: row l % 32, 8 K values at 8 (l / 32)),
// NPF K steps ahead, and accumulates one 32 x 32 MFMA tile; the NW partial tiles are summed in
// LDS in wave order (deterministic) and the epilogue runs 4 outputs per thread on the first 256
// threads.  Long K (few blocks, each streaming many bytes) uses 8 waves with 8 steps per buffer,
// so a block keeps 128 KiB of operands in flight.
constexpr int kNarrow = 32;
template <int MODE, int NW, int NPF>
__global__ __launch_bounds__(64 * NW) void gemm_narrow_kernel(const half* __restrict__ X,
                                                              const half* __restrict__ W, int M,
                                                              int N, int K, EpiArgs ep) {
  const int tiles_n = N / kNarrow;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const int m0 = tm * kNarrow, n0 = tn * kNarrow;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, kh = 8 * (lane >> 5);
  const half* xr = X + (size_t)min(m0 + r, M - 1) * K + kh;
  const half* wr = W + (size_t)(n0 + r) * K + kh;
  const int steps = K / 16 / NW;         // K steps of this wave (K % (16 NW) == 0)
  const int kbeg = wave * steps * 16;
  // epilogue mapping (below): thread -> row ml, 4 columns nl; 8 aligned threads per row
  const int et = threadIdx.x & 255;
  const int ml = et >> 3, nl = 4 * (et & 7);
  const LnPre pre = ln_pre4<MODE, 8>(ep, min(m0 + ml, M - 1), n0 + nl, K);
  floatx16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  half8 a[2][NPF], b[2][NPF];
  auto load = [&](int buf, int s0) {
#pragma unroll
    for (int j = 0; j < NPF; ++j) {
      const int k = kbeg + 16 * min(s0 + j, steps - 1);  // past the end: reload the last step
      a[buf][j] = *(const half8*)(wr + k);
      b[buf][j] = *(const half8*)(xr + k);
    }
  };
  auto mma = [&](int buf, int s0) {
#pragma unroll
    for (int j = 0; j < NPF; ++j)
      if (s0 + j < steps) acc = mfma32x32x16(a[buf][j], b[buf][j], acc);
  };
  // Two buffers, alternated by a loop unrolled twice (register arrays need compile-time indices).
  load(0, 0);
  for (int s0 = 0; s0 < steps; s0 += 2 * NPF) {
    if (s0 + NPF < steps) load(1, s0 + NPF);
    mma(0, s0);
    if (s0 + NPF >= steps) break;
    if (s0 + 2 * NPF < steps) load(0, s0 + 2 * NPF);
    mma(1, s0 + NPF);
  }
  // acc[4g + e] = C[m0 + r][n0 + 8g + 4 (lane / 32) + e]
  __shared__ __align__(16) float part[NW][kNarrow][kNarrow];
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *(floatx4*)&part[wave][r][8 * g + 4 * (lane >> 5)] =
        floatx4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
  __syncthreads();
  if (threadIdx.x >= 256 || m0 + ml >= M) return;
  float sum[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = part[0][ml][nl + e];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += part[w][ml][nl + e];
    sum[e] = v;
  }
  epilogue4<MODE, 8>(ep, m0 + ml, n0 + nl, sum, pre);
}

// Long K: 8 waves (K % 128 == 0 and more than two 4-step buffers per wave at 4 waves).
static bool narrow_long_k(int k) { return k % 128 == 0 && k / 64 > 8; }

template <int MODE>
static void launch_narrow_mode(dim3 grid, const half* x, const half* w, int m, int n, int k,
                               const EpiArgs& ep, hipStream_t stream) {
  if (narrow_long_k(k))
    hipLaunchKernelGGL((gemm_narrow_kernel<MODE, 8, 8>), grid, dim3(512), 0, stream, x, w, m, n, k, ep);
  else
    hipLaunchKernelGGL((gemm_narrow_kernel<MODE, 4, 4>), grid, dim3(256), 0, stream, x, w, m, n, k, ep);
}

static int run_narrow(int mode, const half* x, const half* w, int m, int n, int k,
                      const EpiArgs& ep, hipStream_t stream) {
  const long blocks = (long)((m + kNarrow - 1) / kNarrow) * (n / kNarrow);
  TT_REQUIRE(blocks < (1L << 31), "linear: grid too large");
  const dim3 grid((unsigned)blocks);
  switch (mode) {
    case TT_EPI_BIAS: launch_narrow_mode<TT_EPI_BIAS>(grid, x, w, m, n, k, ep, stream); break;
    case TT_EPI_BIAS_GELU: launch_narrow_mode<TT_EPI_BIAS_GELU>(grid, x, w, m, n, k, ep, stream); break;
    case TT_EPI_RESID_MASKED: launch_narrow_mode<TT_EPI_RESID_MASKED>(grid, x, w, m, n, k, ep, stream); break;
    case TT_EPI_MASKED_RESID: launch_narrow_mode<TT_EPI_MASKED_RESID>(grid, x, w, m, n, k, ep, stream); break;
    default: launch_narrow_mode<TT_EPI_QKV>(grid, x, w, m, n, k, ep, stream); break;
  }
  return launch_status("gemm_narrow_kernel");
}

// ---- host-side tile selection ----
struct TileCfg {
  int bm, bn;
};

template <int BM, int BN, int MODE, int PATH, int NW = 4>
static int run_tile(const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                    hipStream_t stream) {
  // the K-stage ring; the epilogue stages the whole BM x BN tile in the same memory
  constexpr size_t NS = gemm_stages(BM, BN, PATH, NW);
  const size_t lds = std::max(NS * (BM + BN) * (size_t)gemm_ldr(PATH), (size_t)BM * BN) *
                     sizeof(half);
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    attr_err = hipFuncSetAttribute((const void*)gemm_kernel<BM, BN, MODE, PATH, NW>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  });
  if (attr_err != hipSuccess)
    return fail(TT_ERR_HIP, "hipFuncSetAttribute(gemm %dx%d): %s", BM, BN, hipGetErrorString(attr_err));
  int tiles = ((m + BM - 1) / BM) * (n / BN);
  // with a device row count the kernel deals the live tiles, rounded up to the 8 XCDs, over the
  // first blocks of the grid: the grid covers that rounding (extra blocks leave at once)
  if (ep.m_dev != nullptr) tiles = (tiles + 7) & ~7;
  hipLaunchKernelGGL((gemm_kernel<BM, BN, MODE, PATH, NW>), dim3(tiles), dim3(64 * NW), lds,
                     stream, x, w, m, n, k, ep);
  return launch_status("gemm_kernel");
}

template <int MODE>
static int run_mode(int tile, const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                    hipStream_t stream) {
  switch (tile) {
    case 0: return run_tile<256, 256, MODE, 0, 8>(x, w, m, n, k, ep, stream);
    case 1: return run_tile<256, 128, MODE, 0>(x, w, m, n, k, ep, stream);
    case 2: return run_tile<128, 128, MODE, 0>(x, w, m, n, k, ep, stream);
    case 3: return run_tile<128, 64, MODE, 0>(x, w, m, n, k, ep, stream);
    case 6: return run_tile<128, 256, MODE, 1>(x, w, m, n, k, ep, stream);
    case 7: return run_tile<128, 128, MODE, 1>(x, w, m, n, k, ep, stream);
    case 8: return run_tile<128, 64, MODE, 1>(x, w, m, n, k, ep, stream);
    case 9: return run_tile<256, 128, MODE, 1>(x, w, m, n, k, ep, stream);
    case 10: return run_tile<256, 128, MODE, 0, 8>(x, w, m, n, k, ep, stream);
    default: return run_tile<64, 64, MODE, 0>(x, w, m, n, k, ep, stream);
  }
}

// index 0: 256 x 256 on 8 waves; index 5: 32 x 32 narrow tiles (gemm_narrow_kernel), chosen for
// grids that leave most CUs idle; indices 6-9: 128 x 256, 128 x 128, 128 x 64, 256 x 128 on the
// register path; index 10: 256 x 128 on 8 waves with a three-stage ring
static const TileCfg kTiles[] = {{256, 256}, {256, 128}, {128, 128}, {128, 64}, {64, 64},
                                 {32, 32},   {128, 256}, {128, 128}, {128, 64}, {256, 128},
                                 {256, 128}};
constexpr int kNumTiles = (int)(sizeof(kTiles) / sizeof(kTiles[0]));

static int g_tile_override = -1;  // test hook: force one tile configuration

// Tile choice, from measurements on MI355X (M = 8192, N in {1024, 3072, 4096}, K in {1024,
// 4096}; round-robin medians of interleaved runs in one process): the 8-wave 256 x 256 block
// (two waves per SIMD, half the operand traffic per FLOP of 128 x 128) wins when its tiles fill
// whole rounds of the chip, at least two (ffn_in, 8192 x 4096 x 1024: 85 against 87 us with
// GELU, 71 against 76 us with bias only); with 1.5 rounds (QKV, N = 3072) or half a round (N =
// 1024) two 128 x 128 blocks per CU are faster (QKV 57 against 63 us, ffn_out 65 against 95 us).
// Narrower tiles are used when a wider one would leave CUs idle, down to the 32x32 narrow kernel
// for few-token grids.  Exactly one round of 8-wave 256 x 128 tiles with the three-stage ring
// (N = 1024 at M = 8192) beats two 128 x 128 blocks per CU inside the forward, with or without a
// row mask (same-process A/B of whole forwards: C5 -2.5%, C4 with 20% padded rows -3.4%), although
// a GEMM repeated on its own favours the 128-row tiles for out_proj and for padded rows.  The QKV
// projection takes the same tile for whole rounds of it (C5, 8192 x 3072 x 1024: three rounds;
// forward -2.0%) unless its live row count is read on the device (packed rows, whose live tiles
// end inside a round: C4 +0.4 / +0.8% with it).
static int pick_tile(int m, int n, int k, int mode, int cus, bool packed = false) {
  if (g_tile_override >= 0 && g_tile_override < kNumTiles && n % kTiles[g_tile_override].bn == 0)
    return g_tile_override;
  auto tiles = [&](int i) { return (long)((m + kTiles[i].bm - 1) / kTiles[i].bm) * (n / kTiles[i].bn); };
  if (n % 256 == 0 && tiles(0) >= 2 * cus && tiles(0) % cus == 0) return 0;
  if (n % 128 == 0 && k >= 1024 &&
      (tiles(10) == cus || (mode == TT_EPI_QKV && !packed && tiles(10) % cus == 0)))
    return 10;
  // One round of 128 x 64 tiles streaming a long K is latency-bound: each CU moves only the bytes
  // it keeps in flight, and the register path keeps two more K stages in flight than the direct
  // copies (measured on MI355X, 4096 x 512 x 2048: 22.3 -> 15.8 us).  On grids of several tiles
  // per CU the direct path is as fast or faster (M = 8192 projections), so it stays there.
  for (int i = 2; i < 4; ++i)
    if (n % kTiles[i].bn == 0 && tiles(i) >= cus) return (i == 3 && k >= 1024) ? 8 : i;
  // Few tokens: 64 x 64 tiles that would fill at most half the CUs become 32 x 32 narrow tiles
  // (measured on MI355X: C1 77 -> 68 us, C2 138 -> 106 us; C1 / C2 ffn_out has 32 / 4 tiles of
  // K = 1024 at 64 x 64, 10-11 us, each CU limited by the bytes it keeps in flight).
  if (2 * tiles(4) <= cus) return 5;
  return 4;  // 64x64: every N that is a multiple of 64
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

bool linear_is_narrow(int m, int n, int k, int mode) {
  if (k % kBK != 0 || n % 64 != 0) return true;
  return pick_tile(m, n, k, mode, device_cus()) == 5;
}

int linear_stats_width(int m, int n, int k, int mode) {
  if (k % kBK != 0 || n % 64 != 0) return 4;  // gemm_small_kernel: one thread per 4 columns
  const int tile = pick_tile(m, n, k, mode, device_cus());
  if (tile == 5) return kNarrow;               // gemm_narrow_kernel: 8 threads per 32 columns
  return kTiles[tile].bn / 2;                  // MFMA tiles: the column range of one wave
}

int launch_linear(const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                  hipStream_t stream) {
  TT_REQUIRE(m >= 0 && n > 0 && k > 0, "linear: bad shape m=%d n=%d k=%d", m, n, k);
  TT_REQUIRE(k % 8 == 0 && n % 8 == 0, "linear: N=%d and K=%d must be multiples of 8", n, k);
  TT_REQUIRE((int64_t)n * k < (1LL << 31), "linear: weight of more than 2^31 elements (n=%d k=%d)",
             n, k);
  if (ep.mode == TT_EPI_RESID_MASKED || ep.mode == TT_EPI_MASKED_RESID || ep.mode == TT_EPI_BIAS ||
      ep.mode == TT_EPI_BIAS_GELU)
    TT_REQUIRE(ep.ldy >= n && ep.ldy % 8 == 0, "linear: ldy=%d must be >= N=%d and a multiple of 8",
               ep.ldy, n);
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
  if (ep.ln_part != nullptr) {
    TT_REQUIRE(ep.mode == TT_EPI_QKV || ep.mode == TT_EPI_BIAS_GELU || ep.mode == TT_EPI_BIAS,
               "linear: a folded LayerNorm needs a bias / GELU / QKV epilogue");
    TT_REQUIRE(linear_is_narrow(m, n, k, ep.mode),
               "linear: a folded LayerNorm runs on the narrow / small kernels only (m=%d n=%d)", m, n);
    TT_REQUIRE(ep.ln_colsum != nullptr && ep.ln_bias != nullptr && ep.ln_slots > 0 &&
                   k % ep.ln_slots == 0 && ep.ln_stride >= ep.ln_slots,
               "linear: bad folded-LayerNorm arguments (slots %d, stride %d, K %d)", ep.ln_slots,
               ep.ln_stride, k);
  }
  if (ep.part_out != nullptr) {
    TT_REQUIRE(ep.mode == TT_EPI_RESID_MASKED || ep.mode == TT_EPI_MASKED_RESID,
               "linear: row statistics are written by the residual epilogues only");
    TT_REQUIRE(ep.ln_stride >= n / linear_stats_width(m, n, k, ep.mode),
               "linear: statistics row stride %d < %d slots", ep.ln_stride,
               n / linear_stats_width(m, n, k, ep.mode));
  }
  if (ep.m_dev != nullptr || ep.rowmap != nullptr) {
    TT_REQUIRE(!linear_is_narrow(m, n, k, ep.mode),
               "linear: packed variable-length rows run on the MFMA tiles only (m=%d n=%d k=%d)", m,
               n, k);
    TT_REQUIRE(ep.ln_part == nullptr && ep.part_out == nullptr,
               "linear: packed rows take no folded LayerNorm");
    TT_REQUIRE(ep.mode != TT_EPI_QKV || (ep.m_dev != nullptr && ep.rowmap != nullptr),
               "linear(qkv): packed rows need both the row count and the row map");
  }
  if (m == 0) return TT_OK;
  if (k % kBK != 0 || n % 64 != 0) return run_small(ep.mode, x, w, m, n, k, ep, stream);
  const int tile = pick_tile(m, n, k, ep.mode, device_cus(), ep.m_dev != nullptr);
  if (tile == 5) return run_narrow(ep.mode, x, w, m, n, k, ep, stream);
  switch (ep.mode) {
    case TT_EPI_BIAS: return run_mode<TT_EPI_BIAS>(tile, x, w, m, n, k, ep, stream);
    case TT_EPI_BIAS_GELU: return run_mode<TT_EPI_BIAS_GELU>(tile, x, w, m, n, k, ep, stream);
    case TT_EPI_RESID_MASKED: return run_mode<TT_EPI_RESID_MASKED>(tile, x, w, m, n, k, ep, stream);
    case TT_EPI_MASKED_RESID: return run_mode<TT_EPI_MASKED_RESID>(tile, x, w, m, n, k, ep, stream);
    default: return run_mode<TT_EPI_QKV>(tile, x, w, m, n, k, ep, stream);
  }
}

}  // namespace tt

extern "C" int tt_gemm_tile_override(int index) {
  TT_REQUIRE(index >= -1 && index < tt::kNumTiles, "gemm_tile_override: index %d out of [-1, %d)",
             index, tt::kNumTiles);
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
