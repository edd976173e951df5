// Flash-attention block for head_dim 32 and 64 on gfx950 (device code shared by the standalone
// attention kernel and the persistent megakernel).
//
// One 256-thread block owns (sequence b, head h, 128-query tile); each of its four waves owns 32
// queries.  Key/value tiles of 64 keys are staged in LDS (double-buffered, or a ring of three for
// long sequences) by buffer -> LDS dwordx4 copies issued one (two) tiles ahead, so no registers
// hold in-flight tiles; each lane's source offset is fixed and the tile start moves the
// wave-uniform buffer base.
// Per wave and tile:
//   S^T = K Q^T   with v_mfma_f32_32x32x16_f16 (K from LDS as the A operand, Q^T held in
//                 registers as the B operand), so lane l holds one query (l % 32) and 32 of the 64
//                 keys: the row max and sum need one cross-half exchange (v_permlane32_swap);
//   O^T += V^T P^T with V^T tiles from LDS (the QKV projection writes V transposed, [hd, S]).
// To make the probabilities a lane already holds line up with 8 consecutive keys of V^T, K rows
// are placed in LDS with bits 2 and 3 of the row index swapped: S^T row r then holds key pi(r),
// and lane l of key block kb holds keys 32kb + 16(j/8) + 8(l/32) + (j%8), j = 0..15.
// Softmax runs in the exp2 domain: Q arrives multiplied by scale*log2(e) (from the forward's QKV
// epilogue, with one fp16 rounding as unscaled Q would have; through the C ABI, multiplied and
// rounded again when the block loads it), and the S^T MFMA chains start from minus the row's
// reference max instead of zero, so each score leaves the MFMA ready for v_exp_f32.  The reference max is refreshed lazily: the output is rescaled
// only when some row's max grows by more than 2^8 over the reference in use (exp2 of a score
// minus a stale reference is then at most 256, exact in fp32 and in the fp16 probabilities).
// Row sums add the fp16 probabilities that feed the P V MFMA (v_dot2_f32_f16), so numerator and
// denominator use the same rounded values.
// Masking: keys are dropped when key >= kv_end (last valid key + 1), when causal && key > query,
// and, for masks that are not right-padded prefixes, when mask[b, key] == 0.  Query rows that are
// padded are written as +0.0.  Causal query tiles are scheduled heaviest-first.
#pragma once

#include "common.hpp"

#include <mutex>

namespace tt {

constexpr int kBQ = 128;
constexpr int kBKV = 64;

__host__ __device__ constexpr int round_up(int v, int m) { return (v + m - 1) / m * m; }

__device__ __forceinline__ int pi23(int r) {  // swap bits 2 and 3
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

// Chunk swizzles of the LDS tiles.  One ds_read_b128 phase serves 16 lanes, which read 16
// consecutive rows at one logical 16-byte chunk; the physical chunk is XORed with row bits chosen so
// that those 16 rows land in 16 different 16-byte bank groups (64 banks x 4 bytes = 256 bytes):
// 64-byte rows (HD 32) pair the 4 chunks with bits 2-3 of the row, 128-byte rows (HD 64, and the
// 64-key V^T rows) the 8 chunks with bits 1-3, 256- and 512-byte rows (HD 128, 256) 16 chunks with
// bits 0-3.  The global -> LDS copies fetch logical chunk c ^ swizzle into physical chunk c, so any
// per-row XOR works with them.
template <int HD>
__device__ __forceinline__ int kswz(int row, int c) {
  if constexpr (HD >= 128) return c ^ (row & 15);
  else if constexpr (HD == 64) return c ^ ((row >> 1) & 7);
  else return c ^ ((row >> 2) & 3);
}
__device__ __forceinline__ int vswz(int row, int c) { return c ^ ((row >> 1) & 7); }

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float xhalf_max(float v) {  // max over lanes l and l ^ 32
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float xhalf_sum(float v) {  // sum over lanes l and l ^ 32
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}


// Arguments shared by every attention block of one launch (see attention_block).
struct AttnArgs {
  const half* Q;       // [B, H, S, hd]
  const half* K;       // [B, H, S, hd]
  const half* Vt;      // [B, H, hd, Sp], Sp = S rounded up to 64
  const uint8_t* mask; // [B, S] or nullptr
  half* ctx;           // [B, S, H * hd]
  int B, S, H;
  float scale_log2;    // hd^-1/2 * log2(e)
  // Q already multiplied by scale_log2 (rounded to fp16 once, by the QKV projection's epilogue);
  // otherwise the block multiplies and rounds it when it loads it.
  int q_prescaled;
  // Packed context rows (variable-length batches): out_row[b * S + s] is the row of token (b, s)
  // in a context of only the valid tokens, -1 for a padded token (not stored).  nullptr: the
  // context is token-major [B, S, D] and padded rows are written as +0.0.
  const int* out_row = nullptr;
};

// One (sequence b, head h, 128-query tile qt) attention block on 256 threads.  kv_end is
// 1 + the index of the last valid key of sequence b (S without a mask) and `prefix` says whether
// the valid keys form a prefix; sk_base / sv_base are 2 * 64 * HD halfs of LDS each, or 3 * 64 *
// HD with RING3 (three key tiles in flight, so a tile's copies are issued two tiles before it is
// read; a compile-time choice: with a run-time buffer index the compiler can no longer tell the
// in-flight copies from the tile being read and waits for all of them before its first MFMA).
// POLICY is the cache policy of the Q, K and V^T loads (kLoadDevice when other workgroups of the
// same launch wrote them).
template <int HD, bool CAUSAL, int POLICY = kLoadDefault, bool RING3 = false>
__device__ __forceinline__ void attention_block(const AttnArgs& a, int bh, int qt, int kv_end,
                                                bool prefix, half* sk_base, half* sv_base) {
  static_assert(HD == 32 || HD == 64 || HD == 128 || HD == 256, "MFMA attention head_dim");
  constexpr int KSTEPS = HD / 16;  // k-steps of the S^T MFMA
  constexpr int DB = HD / 32;      // 32-row blocks of O^T
  constexpr int KCH = HD / 8;      // 16-byte chunks per K row
  constexpr int KRPC = 64 / KCH;   // K rows per 1 KiB copy
  constexpr int KCOPIES = kBKV * HD * 2 / 1024 / 4;  // K copies per wave per tile
  constexpr int VCOPIES = HD * kBKV * 2 / 1024 / 4;  // V^T copies per wave per tile
  constexpr float kLazy = 8.0f;    // log2 growth of the row max that forces a rescale

  half (*sk)[kBKV * HD] = reinterpret_cast<half (*)[kBKV * HD]>(sk_base);
  half (*sv)[HD * kBKV] = reinterpret_cast<half (*)[HD * kBKV]>(sv_base);
  const half* __restrict__ Q = a.Q;
  const half* __restrict__ K = a.K;
  const half* __restrict__ Vt = a.Vt;
  const uint8_t* __restrict__ mask = a.mask;
  half* __restrict__ ctx = a.ctx;
  const int S = a.S, H = a.H;
  const float scale_log2 = a.scale_log2;
  const int b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, col = lane & 31;
  const int ldv = round_up(S, kBKV);

  const bool keymask = (mask != nullptr) && !prefix;
  constexpr bool r3 = RING3;

  const int q0 = qt * kBQ;
  const int qw = q0 + wave * 32;
  const int q = qw + col;
  const int block_end = CAUSAL ? min(kv_end, q0 + kBQ) : kv_end;
  const int ntiles = (block_end + kBKV - 1) / kBKV;
  const bool wave_active = qw < kv_end;  // queries >= kv_end are padded
  const int wave_end = CAUSAL ? min(kv_end, qw + 32) : kv_end;

  const size_t D = (size_t)H * HD;
  const half* Qbh = Q + (size_t)bh * S * HD;
  const half* Kbh = K + (size_t)bh * S * HD;
  const half* Vbh = Vt + (size_t)bh * HD * ldv;

  // Copy sources (per lane; the tile start is added per tile).  K copy c of this wave fills LDS
  // rows p = (wave * KCOPIES + c) * KRPC + lane / KCH with key pi(p) at logical chunk
  // (lane % KCH) ^ swizzle(p); V^T copy c fills row d = (wave * VCOPIES + c) * 8 + lane / 8 with
  // keys 8 ((lane % 8) ^ (d % 8)) .. +7 of feature row d.
  // Key rows at or past S lie outside the K buffer's range, so those lanes read no memory (their
  // LDS rows hold whatever the buffer check leaves there); the scores of such keys are always
  // masked, by selection, so no value of those rows can reach the output.
  uint32_t koff[KCOPIES], voff[VCOPIES];
#pragma unroll
  for (int c = 0; c < KCOPIES; ++c) {
    const int p = (wave * KCOPIES + c) * KRPC + lane / KCH;
    koff[c] = (uint32_t)(((p & ~31) | pi23(p & 31)) * HD + kswz<HD>(p, lane % KCH) * 8) * 2;
  }
#pragma unroll
  for (int c = 0; c < VCOPIES; ++c) {
    const int d = (wave * VCOPIES + c) * 8 + (lane >> 3);
    voff[c] = (uint32_t)(d * ldv + vswz(d, lane & 7) * 8) * 2;
  }
  auto issue_tile = [&](int t0, int st) {
    const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(Kbh + (size_t)t0 * HD, (uint32_t)(S - t0) * HD * 2);
#pragma unroll
    for (int c = 0; c < KCOPIES; ++c)
      lds_copy16_buf<POLICY>(kr, koff[c], &sk[st][(wave * KCOPIES + c) * 512]);
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(Vbh + t0, (uint32_t)(HD * ldv - t0) * 2);
#pragma unroll
    for (int c = 0; c < VCOPIES; ++c)
      lds_copy16_buf<POLICY>(vr, voff[c], &sv[st][(wave * VCOPIES + c) * 512]);
  };
  // V^T columns of keys >= S (padding of the last, partial tile) are cleared in LDS so that
  // 0-probability keys contribute 0 * 0, whatever the padding memory holds.
  auto clear_vt_tail = [&](int t0, int st) {
    const int first = S - t0;  // first invalid column of this tile, in (0, 64)
    for (int e = tid; e < HD * kBKV; e += 256) {
      const int d = e / kBKV, k = e % kBKV;
      if (k >= first) sv[st][d * kBKV + vswz(d, k / 8) * 8 + (k & 7)] = (half)0.f;
    }
  };

  // Q is held multiplied by scale * log2(e) (in fp16), so the MFMA yields scores in the log2
  // domain directly.
  half8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    if (q < S) {
      if constexpr (POLICY == kLoadDefault) {
        qf[kk] = *(const half8*)(Qbh + (size_t)q * HD + 16 * kk + 8 * hf);
      } else {  // one (b, h) plane of Q is S * HD halfs, far below 4 GiB
        const __amdgpu_buffer_rsrc_t qr = buffer_rsrc(Qbh, (uint32_t)S * HD * 2);
        qf[kk] = __builtin_bit_cast(half8, load16<POLICY>(qr, (uint32_t)(q * HD + 16 * kk + 8 * hf) * 2));
      }
      if (!a.q_prescaled) {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[kk][e] = (half)((float)qf[kk][e] * scale_log2);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[kk][e] = (half)0.f;
    }
  }

  floatx16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.f;
  float m_ref = -INFINITY;  // reference max (log2 domain) the running sums are scaled to
  float l_run = 0.f;        // this lane's half of the row sum
  // The S^T MFMA chains start from -m_ref (0 while no key of the row has been seen), so the
  // scores come out relative to the reference max and exp2 applies to them directly.  thr is
  // the relative tile max above which the reference moves.
  float thr = -INFINITY;
  floatx16 sinit;
#pragma unroll
  for (int e = 0; e < 16; ++e) sinit[e] = 0.f;

  // Non-prefix masks: this lane's key-mask byte.  Ring of two: the next tile's byte is loaded
  // when its copies are issued, so the end-of-tile wait covers it.  Ring of three: each tile's
  // byte is loaded at the start of that tile (a byte carried over two tiles would make its
  // register moves wait for every load issued before it).  The raw byte is kept (address
  // clamped, bound applied at use) so the load's wait lands at the use, not at the load.
  auto mask_byte = [&](int t0) -> int {
    const int key = min(t0 + lane, S - 1);
    return mask[(size_t)b * S + key];
  };
  int mcur = 0, mnext = 0;
  if (ntiles > 0) {
    issue_tile(0, 0);
    if (!r3 && keymask) mcur = mask_byte(0);
    // Both first tiles land before the loop: with copies still in flight on entry, the compiler
    // adds a wait for the next tile's copies before every tile's first MFMA.
    if (r3 && ntiles > 1) issue_tile(kBKV, 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (kBKV > S) {
      clear_vt_tail(0, 0);
      __syncthreads();
    }
  }
  for (int t = 0; t < ntiles; ++t) {
    const int st = r3 ? t % 3 : (t & 1);
    const int t0 = t * kBKV;
    if (!r3 && t + 1 < ntiles) {
      issue_tile(t0 + kBKV, st ^ 1);
      if (keymask) mnext = mask_byte(t0 + kBKV);
    }
    // Ring of three: the copies of tile t + 2 go to the buffer tile t - 1 used.
    if (r3) {
      if (keymask) mcur = mask_byte(t0);
      if (t + 2 < ntiles) issue_tile(t0 + 2 * kBKV, st == 0 ? 2 : st - 1);
    }
    if (wave_active && t0 < wave_end) {
      floatx16 s[2];
      // The S^T MFMAs issue at raised wave priority: the SIMD's other waves are mostly in their
      // softmax (vector ALU), so a wave that reaches its MFMAs gets the matrix unit first
      // (measured on MI355X: -3% at B 2, S 4096, head_dim 64; +2% at head_dim 32, not used there).
      if constexpr (HD == 64) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int row = kb * 32 + col;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
          const half8 a = *(const half8*)(&sk[st][row * HD + kswz<HD>(row, 2 * kk + hf) * 8]);
          s[kb] = mfma32x32x16(a, qf[kk], kk == 0 ? sinit : s[kb]);
        }
      }
      if constexpr (HD == 64) __builtin_amdgcn_s_setprio(0);
      const bool need_mask = (t0 + kBKV > kv_end) || (CAUSAL && t0 + kBKV - 1 > qw) || keymask;
      if (need_mask) {
        // Lane-local 32-bit "allowed" word, bit 16 kb + j for score s[kb][j] (key offset
        // kr = 16 g + 8 hf + (j % 8) with g = 2 kb + j / 8): a range part (kr < lim - t0) and,
        // for non-prefix masks, the bytes 2 g + hf of the tile's 64-key mask ballot.
        const int lim = CAUSAL ? min(kv_end, q + 1) : kv_end;  // keys < lim may be valid
        const int rem = lim - t0;
        uint32_t allowed = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = min(max(rem - (16 * g + 8 * hf), 0), 8);
          allowed |= ((1u << n) - 1u) << (8 * g);
        }
        if (keymask) {
          const uint64_t kbits = __ballot(mcur != 0 && t0 + lane < S);
          allowed &= __builtin_amdgcn_perm((uint32_t)(kbits >> 32), (uint32_t)kbits,
                                           hf ? 0x07050301u : 0x06040200u);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (!((allowed >> (16 * kb + j)) & 1u)) s[kb][j] = -INFINITY;
      }
      float mx = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[kb][j]);
      const float mt = xhalf_max(mx);  // tile row max relative to the reference in use
      if (__builtin_amdgcn_ballot_w64(mt > thr) != 0) {
        // Rescale: the new reference is the true running max (lanes whose max did not grow
        // get corr = 1 and shift 0).  A row with no valid key so far keeps m_ref = -inf and
        // o = l = 0.
        const float mc = (m_ref == -INFINITY) ? 0.f : m_ref;  // offset the scores carry
        const float m_new = fmaxf(m_ref, mt + mc);
        const float corr = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_ref - m_new);
        const float shift = (m_new == -INFINITY) ? 0.f : m_new - mc;
        m_ref = m_new;
        thr = (m_new == -INFINITY) ? -INFINITY : kLazy;
        l_run *= corr;
#pragma unroll
        for (int i = 0; i < DB; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[i][e] *= corr;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[kb][e] -= shift;
#pragma unroll
        for (int e = 0; e < 16; ++e) sinit[e] = (m_new == -INFINITY) ? 0.f : -m_new;
      }
      half8 p16[2][2];
      const half2v ones = {(half)1.f, (half)1.f};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
          const float p0 = __builtin_amdgcn_exp2f(s[kb][j]);
          const float p1 = __builtin_amdgcn_exp2f(s[kb][j + 1]);
          const half2v pp = {(half)p0, (half)p1};
          l_run = __builtin_amdgcn_fdot2(pp, ones, l_run, false);
          p16[kb][j >> 3][j & 7] = pp[0];
          p16[kb][j >> 3][(j & 7) + 1] = pp[1];
        }
#pragma unroll
      for (int i = 0; i < DB; ++i) {
        const int row = i * 32 + col;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const half8 a = *(const half8*)(&sv[st][row * kBKV + vswz(row, 4 * kb + 2 * c + hf) * 8]);
            o[i] = mfma32x32x16(a, p16[kb][c], o[i]);
          }
      }
    }
    if (!r3) mcur = mnext;
    if (t + 1 < ntiles) {
      const int sn = r3 ? (st == 2 ? 0 : st + 1) : (st ^ 1);
      if (r3 && t + 2 < ntiles) {
        // The next tile's copies have landed (those of tile t + 2, issued after them, may stay
        // in flight) ...
        wait_vmcnt<KCOPIES + VCOPIES>();
        raw_barrier();                  // ... and every wave is done with this one (the LDS
                                        // reads fed this tile's MFMAs, so they have returned)
      } else {
        __builtin_amdgcn_s_waitcnt(0);  // the next tile's copies have landed ...
        __syncthreads();                // ... and every wave is done with this one
      }
      if (t0 + 2 * kBKV > S) {        // next tile is the partial last one
        clear_vt_tail(t0 + kBKV, sn);
        __syncthreads();
      }
    }
  }

  if (q >= S) return;
  size_t orow = (size_t)b * S + q;
  if (a.out_row != nullptr) {  // lanes l and l ^ 32 hold the same query: they leave together
    const int r = a.out_row[orow];
    if (r < 0) return;
    orow = (size_t)r;
  }
  const float l_tot = xhalf_sum(l_run);
  const bool qvalid = wave_active && q < kv_end && (mask == nullptr || mask[(size_t)b * S + q] != 0);
  const float inv = (qvalid && l_tot > 0.f) ? 1.0f / l_tot : 0.f;
  half* dst = ctx + orow * D + (size_t)h * HD;
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * i + 8 * g + 4 * hf;
      half4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = qvalid ? (half)(o[i][4 * g + e] * inv) : (half)0.f;
      *(half4*)(dst + d) = v;
    }
}

// Key tiles in flight in the standalone kernel: three for long sequences up to head_dim 64
// (48 KiB per block at 64, still three blocks per CU), two otherwise (a third 32 / 64 KiB tile
// would cost a block per CU above head_dim 64).  Measured on MI355X: the ring of three is 2-4%
// faster at B 2, S 4096 (causal) but 1-3% slower at S 512 / 1024, where blocks run few tiles.
constexpr bool attention_ring3_hd(int hd) { return hd <= 64; }
inline bool attention_ring3(int hd, int seq) { return attention_ring3_hd(hd) && seq >= 2048; }

// Standalone launch: one block per (b, h, 128-query tile).  `info` (or nullptr without a mask)
// holds kv_end per sequence and whether its valid keys form a prefix (mask_info_kernel).
template <int HD, bool CAUSAL, bool RING3>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a, const int32_t* __restrict__ info) {
  // Dynamic LDS: with statically declared tiles the compiler makes the first K-fragment read of
  // every tile wait (vmcnt(0)) for the next tile's in-flight global -> LDS copies, serialising
  // the prefetch; from the dynamic area it relies on the explicit waits, as intended.
  extern __shared__ __align__(16) half att_lds[];
  half* sk = att_lds;
  half* sv = att_lds + (RING3 ? 3 : 2) * kBKV * HD;
  const int BH = a.B * a.H;
  const int nqt = (a.S + kBQ - 1) / kBQ;
  const int bh = blockIdx.x % BH;
  int qt = blockIdx.x / BH;
  if (CAUSAL) qt = nqt - 1 - qt;  // heaviest causal tiles first
  const int b = bh / a.H;
  int kv_end = a.S;
  bool prefix = true;
  if (info != nullptr) {
    kv_end = info[b];
    prefix = info[a.B + b] != 0;
  }
  // A query tile at or past the last valid key holds only padded rows: they are +0.0 (or, with a
  // packed output map, not stored at all), and the key loop -- whose copies and barriers such a
  // block would otherwise run without any MFMA work, over the longest key range of the sequence --
  // is skipped.
  const int q0 = qt * kBQ;
  if (q0 >= kv_end) {
    if (a.out_row != nullptr) return;
    constexpr int CPR = HD / 8;  // 16-byte chunks per context row
    const size_t D = (size_t)a.H * HD;
    const int h = bh - b * a.H;
    for (int e = threadIdx.x; e < kBQ * CPR; e += 256) {
      const int q = q0 + e / CPR;
      if (q < a.S)
        *(u32x4*)(a.ctx + ((size_t)b * a.S + q) * D + (size_t)h * HD + 8 * (e % CPR)) =
            u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  attention_block<HD, CAUSAL, kLoadDefault, RING3>(a, bh, qt, kv_end, prefix, sk, sv);
}

constexpr size_t attention_lds_bytes(int hd, bool ring3 = false) {
  return 2 * (size_t)(ring3 ? 3 : 2) * kBKV * hd * sizeof(half);
}

// Host side: one launch of attention_kernel<HD, CAUSAL, RING3> over every (b, h, query tile);
// the dynamic LDS limit is raised once per instantiation (above 64 KiB for HD 256).
template <int HD, bool CAUSAL, bool RING3>
int launch_attention_ring(const AttnArgs& args, const int32_t* info, hipStream_t stream) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute((const void*)attention_kernel<HD, CAUSAL, RING3>,
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)attention_lds_bytes(HD, RING3));
  });
  if (attr != hipSuccess)
    return fail(TT_ERR_HIP, "hipFuncSetAttribute(attention hd %d): %s", HD, hipGetErrorString(attr));
  const long blocks = (long)args.B * args.H * ((args.S + kBQ - 1) / kBQ);
  TT_REQUIRE(blocks < (1L << 31), "attention: grid too large");
  hipLaunchKernelGGL((attention_kernel<HD, CAUSAL, RING3>), dim3((unsigned)blocks), dim3(256),
                     attention_lds_bytes(HD, RING3), stream, args, info);
  return launch_status("attention_kernel");
}

// The key-tile ring chosen for the sequence length.
template <int HD, bool CAUSAL>
int launch_attention_hd(const AttnArgs& args, const int32_t* info, hipStream_t stream) {
  if constexpr (attention_ring3_hd(HD)) {
    if (attention_ring3(HD, args.S)) return launch_attention_ring<HD, CAUSAL, true>(args, info, stream);
  }
  return launch_attention_ring<HD, CAUSAL, false>(args, info, stream);
}

}  // namespace tt
