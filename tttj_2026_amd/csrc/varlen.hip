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
