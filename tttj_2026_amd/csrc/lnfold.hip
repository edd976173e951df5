// LayerNorm folded into the projection that follows it (layer-wise plan).
//
// With LN(x) = (x - mean) rstd gamma + beta and Y = LN(x) W^T + b,
//   Y[m, n] = rstd_m (sum_k x[m, k] W'[n, k] - mean_m c_n) + b'_n,
//   W' = W diag(gamma),  c_n = sum_k W'[n, k],  b'_n = b_n + sum_k W[n, k] beta_k,
// so the GEMM runs on the raw residual stream and the norm costs two FMAs per output in the
// epilogue.  The per-row (mean, rstd) come from partial statistics that the GEMM producing the
// residual stream writes in its epilogue (gemm.hip); this file derives W', c and b' from the
// packed weights once per model (tt_pack_derived).
#include "common.hpp"
#include "kernels.hpp"

namespace tt {

struct DerivedArgs {
  half* w;
  int64_t stride;
  int64_t off[TT_LAYER_SEGMENTS];
  int D, F;
};

// One block per (output row n of [Wqkv; W1], layer): W' row, c_n and b'_n.
__global__ __launch_bounds__(256) void pack_derived_kernel(DerivedArgs a) {
  const int n = blockIdx.x, l = blockIdx.y;
  half* wl = a.w + (size_t)l * a.stride;
  const bool qkv = n < 3 * a.D;
  const int r = qkv ? n : n - 3 * a.D;
  const half* W = wl + (qkv ? a.off[2] : a.off[8]) + (size_t)r * a.D;
  const half* gamma = wl + (qkv ? a.off[0] : a.off[6]);
  const half* beta = wl + (qkv ? a.off[1] : a.off[7]);
  const half bias = wl[(qkv ? a.off[3] : a.off[9]) + r];
  half* Wp = wl + (qkv ? a.off[12] : a.off[15]) + (size_t)r * a.D;
  float* c = (float*)(wl + (qkv ? a.off[13] : a.off[16]));
  float* bp = (float*)(wl + (qkv ? a.off[14] : a.off[17]));
  float cs = 0.f, bs = 0.f;
  for (int k = threadIdx.x; k < a.D; k += blockDim.x) {
    const float w = (float)W[k];
    const half wp = (half)(w * (float)gamma[k]);
    Wp[k] = wp;
    cs += (float)wp;
    bs = fmaf(w, (float)beta[k], bs);
  }
  __shared__ float red[2][4];
  cs = wave_sum(cs);
  bs = wave_sum(bs);
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = cs;
    red[1][threadIdx.x >> 6] = bs;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    c[r] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    bp[r] = (float)bias + ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
  }
}

int launch_pack_derived(half* w, int64_t stride, const int64_t* off, int D, int F, int L,
                        hipStream_t stream) {
  TT_REQUIRE(w != nullptr && D > 0 && F > 0 && L > 0, "pack_derived: bad arguments");
  DerivedArgs a{};
  a.w = w;
  a.stride = stride;
  for (int i = 0; i < TT_LAYER_SEGMENTS; ++i) a.off[i] = off[i];
  a.D = D;
  a.F = F;
  hipLaunchKernelGGL(pack_derived_kernel, dim3(3 * D + F, L), dim3(256), 0, stream, a);
  return launch_status("pack_derived_kernel");
}

}  // namespace tt
