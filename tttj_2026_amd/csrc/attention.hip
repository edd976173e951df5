// Flash-attention launches for head_dim 32, 64 and 128 (attention_kernel, one block per (b, h,
// 128-query tile); the block itself is attention_block() in attention_block.hpp), the head_dim
// dispatch (8 / 16: attention_small.hip, 256: attention_wide.hip) and the per-sequence mask
// summary.  Built with the VGPR-form MFMA flag (accumulators in architectural VGPRs: 138-140 VGPRs
// at head_dim 64, three waves per SIMD; 199-203 at 128, two).
#include "attention_block.hpp"
#include "kernels.hpp"

namespace tt {

__global__ __launch_bounds__(256) void mask_info_kernel(const uint8_t* __restrict__ mask,
                                                        int32_t* __restrict__ info,
                                                        int32_t* __restrict__ counts, int B,
                                                        int S) {
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
    if (counts != nullptr) counts[b] = sc[0];
  }
}

int launch_mask_info(const uint8_t* mask, int32_t* info, int batch, int seq, hipStream_t stream,
                     int32_t* counts) {
  TT_REQUIRE(batch > 0 && seq > 0 && info != nullptr, "mask_info: bad arguments");
  hipLaunchKernelGGL(mask_info_kernel, dim3(batch), dim3(256), 0, stream, mask, info, counts,
                     batch, seq);
  return launch_status("mask_info_kernel");
}

int attention_head_dim_supported(int head_dim) {
  TT_REQUIRE(head_dim == 8 || head_dim == 16 || head_dim == 32 || head_dim == 64 ||
                 head_dim == 128 || head_dim == 256,
             "attention: head_dim %d not in {8, 16, 32, 64, 128, 256}", head_dim);
  return TT_OK;
}

float attention_q_scale(int head_dim) {
  return (1.0f / sqrtf((float)head_dim)) * 1.4426950408889634f;
}

int launch_attention(const half* q, const half* k, const half* vt, const uint8_t* mask,
                     const int32_t* info, half* ctx, int batch, int seq, int heads, int head_dim,
                     int causal, hipStream_t stream, bool q_prescaled, const int* out_row) {
  TT_REQUIRE(batch > 0 && seq > 0 && heads > 0, "attention: bad shape");
  int rc = attention_head_dim_supported(head_dim);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(mask == nullptr || info != nullptr, "attention: a mask needs its mask_info");
  const AttnArgs args{q, k, vt, mask, ctx, batch, seq, heads, attention_q_scale(head_dim),
                      q_prescaled ? 1 : 0, out_row};
  if (head_dim <= 16) return launch_attention_small(args, info, head_dim, causal, stream);
  if (head_dim == 256) return launch_attention_wide(args, info, head_dim, causal, stream);
  switch (head_dim) {
    case 32: return causal ? launch_attention_hd<32, true>(args, info, stream)
                           : launch_attention_hd<32, false>(args, info, stream);
    case 64: return causal ? launch_attention_hd<64, true>(args, info, stream)
                           : launch_attention_hd<64, false>(args, info, stream);
    default: return causal ? launch_attention_hd<128, true>(args, info, stream)
                           : launch_attention_hd<128, false>(args, info, stream);
  }
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

extern "C" int tt_attention_fwd_prescaled(const void* q, const void* k, const void* vt,
                                          const uint8_t* mask, const int32_t* info, void* ctx,
                                          int batch, int seq, int heads, int head_dim, int causal,
                                          void* stream) {
  TT_REQUIRE(q && k && vt && ctx, "attention: null pointer");
  return tt::launch_attention((const tt::half*)q, (const tt::half*)k, (const tt::half*)vt, mask,
                              info, (tt::half*)ctx, batch, seq, heads, head_dim, causal,
                              (hipStream_t)stream, true);
}
