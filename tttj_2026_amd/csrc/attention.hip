// Standalone flash-attention kernel (one block per (b, h, 128-query tile)) and the per-sequence
// mask summary; the block itself is attention_block() in attention_block.hpp.
#include "attention_block.hpp"
#include "kernels.hpp"

namespace tt {

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a, const int32_t* __restrict__ info) {
  // Dynamic LDS: with statically declared tiles the compiler makes the first K-fragment read of
  // every tile wait (vmcnt(0)) for the next tile's in-flight global -> LDS copies, serialising
  // the prefetch; from the dynamic area it relies on the explicit waits, as intended.
  extern __shared__ __align__(16) half att_lds[];
  half* sk = att_lds;
  half* sv = att_lds + 2 * kBKV * HD;
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
  attention_block<HD, CAUSAL>(a, bh, qt, kv_end, prefix, sk, sv);
}

__global__ __launch_bounds__(256) void mask_info_kernel(const uint8_t* __restrict__ mask,
                                                        int32_t* __restrict__ info, int B, int S) {
  const int b = blockIdx.x;
  int last = -1, count = 0;
  if (mask == nullptr) {
    last = S - 1;
    count = S;
  } else {
    for (int s = threadIdx.x; s < S; s += 256)
      if (mask[(size_t)b * S + s]) {
        last = s;
        ++count;
      }
  }
  __shared__ int sl[256], sc[256];
  sl[threadIdx.x] = last;
  sc[threadIdx.x] = count;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) {
      sl[threadIdx.x] = max(sl[threadIdx.x], sl[threadIdx.x + off]);
      sc[threadIdx.x] += sc[threadIdx.x + off];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (mask == nullptr) {
      info[b] = S;
      info[B + b] = 1;
    } else {
      info[b] = sl[0] + 1;
      info[B + b] = (sc[0] == sl[0] + 1) ? 1 : 0;
    }
  }
}

int launch_mask_info(const uint8_t* mask, int32_t* info, int batch, int seq, hipStream_t stream) {
  TT_REQUIRE(batch > 0 && seq > 0 && info != nullptr, "mask_info: bad arguments");
  hipLaunchKernelGGL(mask_info_kernel, dim3(batch), dim3(256), 0, stream, mask, info, batch, seq);
  return launch_status("mask_info_kernel");
}

int launch_attention(const half* q, const half* k, const half* vt, const uint8_t* mask,
                     const int32_t* info, half* ctx, int batch, int seq, int heads, int head_dim,
                     int causal, hipStream_t stream) {
  TT_REQUIRE(batch > 0 && seq > 0 && heads > 0, "attention: bad shape");
  TT_REQUIRE(head_dim == 32 || head_dim == 64, "attention: head_dim %d not in {32, 64}", head_dim);
  TT_REQUIRE(mask == nullptr || info != nullptr, "attention: a mask needs its mask_info");
  const long blocks = (long)batch * heads * ((seq + kBQ - 1) / kBQ);
  TT_REQUIRE(blocks < (1L << 31), "attention: grid too large");
  const float scale_log2 = (1.0f / sqrtf((float)head_dim)) * 1.4426950408889634f;
  const dim3 grid((unsigned)blocks), block(256);
  const AttnArgs args{q, k, vt, mask, ctx, batch, seq, heads, scale_log2};
#define TT_ATT(HD, C)                                                                          \
  hipLaunchKernelGGL((attention_kernel<HD, C>), grid, block, 4 * kBKV * HD * sizeof(half), stream, \
                     args, info)
  if (head_dim == 64) {
    if (causal) TT_ATT(64, true); else TT_ATT(64, false);
  } else {
    if (causal) TT_ATT(32, true); else TT_ATT(32, false);
  }
#undef TT_ATT
  return launch_status("attention_kernel");
}

}  // namespace tt

extern "C" int tt_mask_info(const uint8_t* mask, int32_t* info, int batch, int seq, void* stream) {
  return tt::launch_mask_info(mask, info, batch, seq, (hipStream_t)stream);
}

extern "C" int tt_attention_fwd(const void* q, const void* k, const void* vt, const uint8_t* mask,
                                const int32_t* info, void* ctx, int batch, int seq, int heads,
                                int head_dim, int causal, void* stream) {
  TT_REQUIRE(q && k && vt && ctx, "attention: null pointer");
  return tt::launch_attention((const tt::half*)q, (const tt::half*)k, (const tt::half*)vt, mask,
                              info, (tt::half*)ctx, batch, seq, heads, head_dim, causal,
                              (hipStream_t)stream);
}
