// Attention for head_dim 8 and 16 (the reference's D = 32 / 4-head and D = 128 / 16-head model
// shapes).  At these widths a 32x32x16 MFMA would be mostly padding and the work is the softmax,
// so one lane owns one query and everything runs on the vector ALUs:
//   block = (b, h, 128 queries), 128 threads; key tiles of 128 keys are staged in LDS as fp32
//   (K rows and V rows -- V read from the transposed V^T [B, H, hd, Sp] layout the QKV projection
//   writes), and every lane reads each key with an LDS broadcast.
//   Online softmax in the exp2 domain (scale * log2(e) folded into Q), 16 keys at a time: the
//   chunk's scores, one max, one rescale of (o, l) when the max grows, then p = 2^(s - m),
//   l += p, o += p v.  Probabilities stay fp32 (no fp16 rounding before P V).
// Masking as in attention_block.hpp: keys >= kv_end, keys > query (causal) and, for masks that
// are not right-padded prefixes, keys whose mask byte is 0 get no weight; padded query rows are
// written as +0.0.  Causal query tiles are dispatched heaviest first.
#include "attention_block.hpp"
#include "kernels.hpp"

namespace tt {

constexpr int kSmallBQ = 128;   // queries per block (one per lane)
constexpr int kSmallBKV = 128;  // keys per LDS tile
constexpr int kSmallChunk = 16; // keys per softmax update

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(kSmallBQ) void attention_small_kernel(AttnArgs a,
                                                                   const int32_t* __restrict__ info) {
  __shared__ float sk[kSmallBKV][HD];
  __shared__ float sv[kSmallBKV][HD];
  __shared__ uint8_t sok[kSmallBKV];
  const int S = a.S, H = a.H;
  const int BH = a.B * H;
  const int nqt = (S + kSmallBQ - 1) / kSmallBQ;
  const int bh = blockIdx.x % BH;
  int qt = blockIdx.x / BH;
  if (CAUSAL) qt = nqt - 1 - qt;
  const int b = bh / H, h = bh - b * H;
  int kv_end = S;
  bool prefix = true;
  if (info != nullptr) {
    kv_end = info[b];
    prefix = info[a.B + b] != 0;
  }
  const bool keymask = a.mask != nullptr && !prefix;
  const int tid = threadIdx.x;
  const int q0 = qt * kSmallBQ, q = q0 + tid;
  if (q0 >= kv_end) {  // only padded queries: +0.0 rows (none with a packed context), no key loop
    if (a.out_row == nullptr && q < S) {
      half* dst = a.ctx + ((size_t)b * S + q) * ((size_t)H * HD) + (size_t)h * HD;
#pragma unroll
      for (int d0 = 0; d0 < HD; d0 += 8) *(u32x4*)(dst + d0) = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const int ldv = round_up(S, 64);
  const half* Qbh = a.Q + (size_t)bh * S * HD;
  const half* Kbh = a.K + (size_t)bh * S * HD;
  const half* Vbh = a.Vt + (size_t)bh * HD * ldv;

  float qf[HD], o[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) {
    qf[d] = q < S ? (float)Qbh[(size_t)q * HD + d] * (a.q_prescaled ? 1.f : a.scale_log2) : 0.f;
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int lim = CAUSAL ? min(kv_end, q + 1) : kv_end;  // keys < lim may be valid for q
  const int block_end = CAUSAL ? min(kv_end, q0 + kSmallBQ) : kv_end;

  for (int t0 = 0; t0 < block_end; t0 += kSmallBKV) {
    __syncthreads();  // the previous tile is no longer read
    {
      const int key = t0 + tid;
#pragma unroll
      for (int d = 0; d < HD; ++d) {
        sk[tid][d] = key < S ? (float)Kbh[(size_t)key * HD + d] : 0.f;
        sv[tid][d] = key < S ? (float)Vbh[(size_t)d * ldv + key] : 0.f;
      }
      sok[tid] = key < S && (!keymask || a.mask[(size_t)b * S + key] != 0);
    }
    __syncthreads();
    const int nk = min(max(lim - t0, 0), kSmallBKV);  // this lane's keys in range
    for (int j0 = 0; j0 < nk; j0 += kSmallChunk) {
      float s[kSmallChunk];
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < kSmallChunk; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < HD; ++d) acc = fmaf(qf[d], sk[j0 + j][d], acc);
        const bool ok = j0 + j < nk && sok[j0 + j];
        s[j] = ok ? acc : -INFINITY;
        mx = fmaxf(mx, s[j]);
      }
      if (mx > m) {  // the running max grows: rescale what was accumulated against the old one
        const float corr = __builtin_amdgcn_exp2f(m - mx);  // m = -inf: 0 (nothing accumulated)
        l *= corr;
#pragma unroll
        for (int d = 0; d < HD; ++d) o[d] *= corr;
        m = mx;
      }
      if (m == -INFINITY) continue;  // no allowed key yet
#pragma unroll
      for (int j = 0; j < kSmallChunk; ++j) {
        const float p = __builtin_amdgcn_exp2f(s[j] - m);  // 0 for masked keys
        l += p;
#pragma unroll
        for (int d = 0; d < HD; ++d) o[d] = fmaf(p, sv[j0 + j][d], o[d]);
      }
    }
  }

  if (q >= S) return;
  size_t orow = (size_t)b * S + q;
  if (a.out_row != nullptr) {  // packed context: padded tokens have no row
    const int r = a.out_row[orow];
    if (r < 0) return;
    orow = (size_t)r;
  }
  const bool qvalid = q < kv_end && (a.mask == nullptr || a.mask[(size_t)b * S + q] != 0);
  const float inv = (qvalid && l > 0.f) ? 1.0f / l : 0.f;
  half* dst = a.ctx + orow * ((size_t)H * HD) + (size_t)h * HD;
#pragma unroll
  for (int d0 = 0; d0 < HD; d0 += 8) {
    half8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = qvalid ? (half)(o[d0 + e] * inv) : (half)0.f;
    *(half8*)(dst + d0) = v;
  }
}

int launch_attention_small(const AttnArgs& args, const int32_t* info, int head_dim, int causal,
                           hipStream_t stream) {
  TT_REQUIRE(head_dim == 8 || head_dim == 16, "attention_small: head_dim %d not in {8, 16}",
             head_dim);
  const long blocks = (long)args.B * args.H * ((args.S + kSmallBQ - 1) / kSmallBQ);
  TT_REQUIRE(blocks < (1L << 31), "attention: grid too large");
  const dim3 grid((unsigned)blocks), block(kSmallBQ);
#define TT_ATT_SMALL(HD, C) \
  hipLaunchKernelGGL((attention_small_kernel<HD, C>), grid, block, 0, stream, args, info)
  if (head_dim == 8) {
    if (causal) TT_ATT_SMALL(8, true); else TT_ATT_SMALL(8, false);
  } else {
    if (causal) TT_ATT_SMALL(16, true); else TT_ATT_SMALL(16, false);
  }
#undef TT_ATT_SMALL
  return launch_status("attention_small_kernel");
}

}  // namespace tt
