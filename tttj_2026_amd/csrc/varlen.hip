// Packed variable-length rows for masked batches.
//
// With a mask, the layer-wise plan runs LayerNorms and GEMMs only over the valid tokens: the
// valid tokens of every sequence, in order, are packed into rows 0 .. n - 1 of the residual
// stream, the LayerNorm output, the attention context and the FFN hidden activations, and the
// kernels read n from device memory (no host synchronisation), so the tiles of padded tokens
// never run.  Q / K / V^T stay in their [B, H, S, hd] / [B, H, hd, Sp] token layout (the QKV
// epilogue scatters packed rows to their tokens), so the attention kernel is unchanged apart from
// where it stores the context.  The final LayerNorm scatters the packed rows back to [B, S, D]
// and writes +0.0 for padded tokens (torch_transformer_benchmark.py:169-171).  Masked rows
// never feed valid ones (keys with mask 0 get probability 0 and every other op is row-wise), so
// the packed forward computes the same valid rows as the padded one.
//
// Packed layout: sequence b owns rows [P_b, P_b + L_b), P_b = sum of L_b' for b' < b.  For a
// right-padded prefix mask of length l_b, L_b = min(l_b rounded up to 8, S): the up to 7 rows
// past l_b stand for padded tokens (their first LayerNorm input is +0.0, their context is +0.0,
// and the QKV projection writes +0.0 into those padded tokens' Q / K / V^T slots, pvalid = 0), so
// a sequence starts on an 8-row boundary and the V^T part of the QKV epilogue stores 8
// consecutive tokens with one 16-byte store.  For any other mask L_b is the number of valid
// tokens.  Every padded token's Q / K / V^T is then +0.0, as in the padded forward: the
// attention's lazy-rescale decision is taken per wave, over valid and padded query rows alike,
// so the same inputs there keep a sequence's result independent of the batch it runs in and of
// which of the two forwards runs it.
#include "common.hpp"
#include "kernels.hpp"

namespace tt {

// Packed rows of sequence b (the layout above), from its mask_info entry and valid count.
__device__ __forceinline__ int packed_len(const int32_t* info, const int32_t* counts, int B, int S,
                                          int b) {
  const int kv_end = info[b];
  if (info[B + b] != 0) return min((kv_end + 7) & ~7, S);
  return counts[b];
}

// One block per sequence: its row offset (a block-wide sum over the earlier sequences), then the
// maps of its tokens.  Prefix masks map position s < L_b to row P_b + s directly; other masks
// rank the valid tokens with a block-wide scan, 256 tokens at a time.
__global__ __launch_bounds__(256) void varlen_map_kernel(
    const uint8_t* __restrict__ mask, const int32_t* __restrict__ info,
    const int32_t* __restrict__ counts, int32_t* __restrict__ n_dev, int32_t* __restrict__ row_tok,
    int32_t* __restrict__ slot, int2* __restrict__ rowmap, uint8_t* __restrict__ pvalid,
    half* __restrict__ q, half* __restrict__ k, int B, int S, int H, int hd) {
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int sred[4];
  __shared__ int swave[4];
  int part = 0;
  for (int j = tid; j < b; j += 256) part += packed_len(info, counts, B, S, j);
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) sred[wave] = part;
  __syncthreads();
  const int P = sred[0] + sred[1] + sred[2] + sred[3];
  const int L = packed_len(info, counts, B, S, b);
  if (b == B - 1 && tid == 0) *n_dev = P + L;
  const int kv_end = info[b];
  const int ldv = (S + 63) / 64 * 64;
  const size_t tok0 = (size_t)b * S;
  const int qk_base = b * H * S * hd, v_base = b * H * hd * ldv;
  const bool prefix = info[B + b] != 0;
  if (prefix) {
    for (int s = tid; s < S; s += 256) {
      if (s < L) {
        const int r = P + s;
        slot[tok0 + s] = r;
        row_tok[r] = s < kv_end ? (int)(tok0 + s) : -1;
        pvalid[r] = s < kv_end ? 1 : 0;
        rowmap[r] = make_int2(qk_base + s * hd, v_base + s);
      } else {
        slot[tok0 + s] = -1;
      }
    }
  }
  int base = P;
  for (int s0 = 0; !prefix && s0 < S; s0 += 256) {
    const int s = s0 + tid;
    const bool v = s < S && mask[tok0 + s] != 0;
    const uint64_t bal = __ballot(v);
    const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                               __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    __syncthreads();  // the previous chunk's wave totals have been read
    if (lane == 0) swave[wave] = __popcll(bal);
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += swave[w];
    if (s < S) {
      if (v) {
        const int r = base + before + rank;
        slot[tok0 + s] = r;
        row_tok[r] = (int)(tok0 + s);
        pvalid[r] = 1;
        rowmap[r] = make_int2(qk_base + s * hd, v_base + s);
      } else {
        slot[tok0 + s] = -1;
      }
    }
    base += swave[0] + swave[1] + swave[2] + swave[3];
  }
  // Q and K of the padded tokens below the sequence's last key tile: +0.0, as the padded
  // forward's QKV projection writes them (a key tile's padded keys are masked by selection, but a
  // padded query row shares its wave's rescale decision with valid rows).  The packed QKV
  // projection writes only the packed rows, so once per forward is enough.
  const int end = min(S, (kv_end + 63) & ~63);
  const int first = prefix ? kv_end : 0;
  const int cpr = hd / 8, span = end - first;
  for (int e = tid; e < H * span * cpr; e += 256) {
    const int c = e % cpr, rest = e / cpr;
    const int s = first + rest % span, h = rest / span;
    if (prefix || mask[tok0 + s] == 0) {
      const size_t off = (((size_t)b * H + h) * S + s) * hd + 8 * c;
      *(u32x4*)(q + off) = u32x4{0u, 0u, 0u, 0u};
      *(u32x4*)(k + off) = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// V^T entries of padded keys that the attention's 64-key tiles read, keys < min(S, kv_end rounded
// up to 64): +0.0, so that a key with probability 0 contributes exactly 0 whatever the workspace
// held.  One wave per V^T row (b, h, d); 8 keys (16 bytes) per lane step, rewritten only when one
// of them is padded.  For a prefix mask only keys >= kv_end can be padded.
__global__ __launch_bounds__(256) void varlen_vt_clear_kernel(const uint8_t* __restrict__ mask,
                                                              const int32_t* __restrict__ info,
                                                              half* __restrict__ vt, int B, int S,
                                                              int D) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= B * D) return;
  const int b = row / D;
  const int kv_end = info[b];
  const int end = min(S, (kv_end + 63) & ~63);
  const int first = info[B + b] != 0 ? kv_end & ~7 : 0;
  const int ldv = (S + 63) / 64 * 64;
  half* vrow = vt + (size_t)row * ldv;
  const uint8_t* mrow = mask + (size_t)b * S;
  for (int c = first + 8 * lane; c < end; c += 8 * 64) {
    uint32_t keep = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) keep |= (c + e < end && mrow[c + e] != 0) ? (1u << e) : 0u;
    if (keep == 0xFFu) continue;
    half8 v = *(const half8*)(vrow + c);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (!((keep >> e) & 1u) && c + e < end) v[e] = (half)0.f;
    *(half8*)(vrow + c) = v;
  }
}

// The mask summary (mask_info_kernel's info and the valid counts), the maps and the clears in one
// launch: kPrepSplit blocks per sequence.  Every block first sums up its own sequence's mask
// (one wave per 64-byte stripe round); block 0 of sequence b also scans sequences 0 .. b - 1 for
// the packed rows before it (one wave per sequence) and writes the sequence's info, count and
// maps (as varlen_map_kernel); all blocks of the sequence share out the clears of its padded Q /
// K rows and V^T entries below its last key tile (as varlen_map_kernel / varlen_vt_clear_kernel).
constexpr int kPrepSplit = 16;

// Last valid position and valid count among mask bytes [0, n) of one sequence, over the lanes
// i = idx, idx + stride, ...: 16 bytes per lane and step when the row is 16-byte aligned (one
// load round for n <= 16 stride), bytes otherwise.
__device__ __forceinline__ void scan_mask(const uint8_t* __restrict__ m, int n, int idx, int stride,
                                          int& last, int& cnt) {
  last = -1;
  cnt = 0;
  if ((n & 15) == 0 && ((uintptr_t)m & 15) == 0) {
    for (int c = idx; c < n / 16; c += stride) {
      const u32x4 w = *(const u32x4*)(m + 16 * c);
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        if ((w[x >> 2] >> (8 * (x & 3))) & 0xFFu) {
          last = 16 * c + x;
          ++cnt;
        }
      }
    }
  } else {
    for (int s = idx; s < n; s += stride) {
      if (m[s] != 0) {
        last = s;
        ++cnt;
      }
    }
  }
}

// kv_end (1 + last valid position), valid count and prefix flag of a sequence's mask, reduced
// over the block (every thread gets them).
__device__ __forceinline__ void seq_summary(const uint8_t* __restrict__ mj, int S, int& kv_end,
                                            int& cnt, bool& prefix) {
  __shared__ int s_red[2][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int last, c;
  scan_mask(mj, S, tid, 256, last, c);
  for (int off = 32; off > 0; off >>= 1) {
    last = max(last, __shfl_xor(last, off));
    c += __shfl_xor(c, off);
  }
  if (lane == 0) {
    s_red[0][wave] = last;
    s_red[1][wave] = c;
  }
  __syncthreads();
  last = max(max(s_red[0][0], s_red[0][1]), max(s_red[0][2], s_red[0][3]));
  cnt = s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3];
  kv_end = last + 1;
  prefix = cnt == kv_end;
}

__global__ __launch_bounds__(256) void varlen_prep_kernel(
    const uint8_t* __restrict__ mask, int32_t* __restrict__ info, int32_t* __restrict__ counts,
    int32_t* __restrict__ n_dev, int32_t* __restrict__ row_tok, int32_t* __restrict__ slot,
    int2* __restrict__ rowmap, uint8_t* __restrict__ pvalid, half* __restrict__ q,
    half* __restrict__ k, half* __restrict__ vt, int B, int S, int H, int hd) {
  const int b = blockIdx.x / kPrepSplit, y = blockIdx.x % kPrepSplit;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t tok0 = (size_t)b * S;
  int kv_end, cnt;
  bool prefix;
  seq_summary(mask + tok0, S, kv_end, cnt, prefix);
  const int ldv = (S + 63) / 64 * 64;
  const int end = min(S, (kv_end + 63) & ~63);  // keys the attention's tiles read
  if (y == 0) {
    // packed rows of the earlier sequences, one wave per sequence
    __shared__ int s_part[4];
    int part = 0;
    for (int j = wave; j < b; j += 4) {
      int last, c;
      scan_mask(mask + (size_t)j * S, S, lane, 64, last, c);
      for (int off = 32; off > 0; off >>= 1) {
        last = max(last, __shfl_xor(last, off));
        c += __shfl_xor(c, off);
      }
      part += c == last + 1 ? min((last + 1 + 7) & ~7, S) : c;
    }
    if (lane == 0) s_part[wave] = part;
    __syncthreads();
    const int P = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const int L = prefix ? min((kv_end + 7) & ~7, S) : cnt;
    if (tid == 0) {
      info[b] = kv_end;
      info[B + b] = prefix ? 1 : 0;
      counts[b] = cnt;
      if (b == B - 1) *n_dev = P + L;
    }
    const int qk_base = b * H * S * hd, v_base = b * H * hd * ldv;
    if (prefix) {
      for (int s = tid; s < S; s += 256) {
        if (s < L) {
          const int r = P + s;
          slot[tok0 + s] = r;
          row_tok[r] = s < kv_end ? (int)(tok0 + s) : -1;
          pvalid[r] = s < kv_end ? 1 : 0;
          rowmap[r] = make_int2(qk_base + s * hd, v_base + s);
        } else {
          slot[tok0 + s] = -1;
        }
      }
    } else {
      __shared__ int swave[4];
      int base = P;
      for (int s0 = 0; s0 < S; s0 += 256) {
        const int s = s0 + tid;
        const bool v = s < S && mask[tok0 + s] != 0;
        const uint64_t bal = __ballot(v);
        const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        __syncthreads();  // the previous chunk's wave totals have been read
        if (lane == 0) swave[wave] = __popcll(bal);
        __syncthreads();
        int before = 0;
        for (int w = 0; w < wave; ++w) before += swave[w];
        if (s < S) {
          if (v) {
            const int r = base + before + rank;
            slot[tok0 + s] = r;
            row_tok[r] = (int)(tok0 + s);
            pvalid[r] = 1;
            rowmap[r] = make_int2(qk_base + s * hd, v_base + s);
          } else {
            slot[tok0 + s] = -1;
          }
        }
        base += swave[0] + swave[1] + swave[2] + swave[3];
      }
    }
  }
  // Q / K of padded tokens below the last key tile (shared out over the sequence's blocks).
  {
    const int first = prefix ? kv_end : 0;
    const int cpr = hd / 8, span = end - first;
    for (int e = y * 256 + tid; e < H * span * cpr; e += 256 * kPrepSplit) {
      const int c = e % cpr, rest = e / cpr;
      const int s = first + rest % span, h = rest / span;
      if (prefix || mask[tok0 + s] == 0) {
        const size_t off = (((size_t)b * H + h) * S + s) * hd + 8 * c;
        *(u32x4*)(q + off) = u32x4{0u, 0u, 0u, 0u};
        *(u32x4*)(k + off) = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  // V^T entries of padded keys below the last key tile: the sequence's H * hd rows, 8 keys per
  // item, rewritten only when one of the 8 is padded.
  {
    const int first = prefix ? kv_end & ~7 : 0;
    const int nch = (end - first + 7) / 8, D = H * hd;
    const uint8_t* mrow = mask + tok0;
    for (int e = y * 256 + tid; e < D * nch; e += 256 * kPrepSplit) {
      const int row = e / nch, c = first + 8 * (e % nch);
      uint32_t keep = 0;
#pragma unroll
      for (int x = 0; x < 8; ++x) keep |= (c + x < end && mrow[c + x] != 0) ? (1u << x) : 0u;
      if (keep == 0xFFu) continue;
      half* vrow = vt + ((size_t)b * D + row) * ldv;
      half8 v = *(const half8*)(vrow + c);
#pragma unroll
      for (int x = 0; x < 8; ++x)
        if (!((keep >> x) & 1u) && c + x < end) v[x] = (half)0.f;
      *(half8*)(vrow + c) = v;
    }
  }
}

int launch_varlen_prep(const uint8_t* mask, int32_t* info, int32_t* counts, int32_t* n_dev,
                       int32_t* row_tok, int32_t* slot, int2* rowmap, uint8_t* pvalid, half* q,
                       half* k, half* vt, int B, int S, int H, int hd, hipStream_t stream) {
  TT_REQUIRE(mask && info && counts && n_dev && row_tok && slot && rowmap && pvalid && q && k && vt,
             "varlen: null pointer");
  TT_REQUIRE(B > 0 && S > 0 && H > 0 && hd > 0, "varlen: bad shape");
  const int64_t ldv = (S + 63) / 64 * 64;
  TT_REQUIRE((int64_t)B * H * S * hd < (1LL << 31) && (int64_t)B * H * hd * ldv < (1LL << 31),
             "varlen: Q / V^T planes of more than 2^31 elements");
  if ((int64_t)B * S > (1LL << 20) || B > (1 << 16)) {  // long scans: three launches
    int rc = launch_mask_info(mask, info, B, S, stream, counts);
    if (rc != TT_OK) return rc;
    return launch_varlen_maps(mask, info, counts, n_dev, row_tok, slot, rowmap, pvalid, q, k, vt, B,
                              S, H, hd, stream);
  }
  hipLaunchKernelGGL(varlen_prep_kernel, dim3(B * kPrepSplit), dim3(256), 0, stream, mask, info,
                     counts, n_dev, row_tok, slot, rowmap, pvalid, q, k, vt, B, S, H, hd);
  return launch_status("varlen_prep_kernel");
}

int launch_varlen_maps(const uint8_t* mask, const int32_t* info, int32_t* counts, int32_t* n_dev,
                       int32_t* row_tok, int32_t* slot, int2* rowmap, uint8_t* pvalid, half* q,
                       half* k, half* vt, int B, int S, int H, int hd, hipStream_t stream) {
  TT_REQUIRE(mask && info && counts && n_dev && row_tok && slot && rowmap && pvalid && q && k && vt,
             "varlen: null pointer");
  TT_REQUIRE(B > 0 && S > 0 && H > 0 && hd > 0, "varlen: bad shape");
  const int64_t ldv = (S + 63) / 64 * 64;
  TT_REQUIRE((int64_t)B * H * S * hd < (1LL << 31) && (int64_t)B * H * hd * ldv < (1LL << 31),
             "varlen: Q / V^T planes of more than 2^31 elements");
  hipLaunchKernelGGL(varlen_map_kernel, dim3(B), dim3(256), 0, stream, mask, info, counts, n_dev,
                     row_tok, slot, rowmap, pvalid, q, k, B, S, H, hd);
  int rc = launch_status("varlen_map_kernel");
  if (rc != TT_OK) return rc;
  const int D = H * hd;
  hipLaunchKernelGGL(varlen_vt_clear_kernel, dim3((B * D + 3) / 4), dim3(256), 0, stream, mask,
                     info, vt, B, S, D);
  return launch_status("varlen_vt_clear_kernel");
}

}  // namespace tt
