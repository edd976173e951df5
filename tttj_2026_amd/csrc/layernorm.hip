// Row LayerNorm for the pre-LN block stack (norm1 / norm2 / final_norm) on gfx950.
//
// One 64-lane wave owns one row of D fp16 values (D <= 8192): every lane loads its 16-byte chunks
// once into registers, the wave reduces the mean, then the centred second moment (two-pass, fp32),
// and writes (x - mean) * rsqrt(var + eps) * gamma + beta as fp16.  Rows whose mask byte is zero
// are written as +0.0 (the final_norm + masked_fill of torch_transformer_benchmark.py:169-171).
// HBM-bound: 4*D bytes per row (+4*D for gamma/beta, cached).
#include "common.hpp"
#include "kernels.hpp"

namespace tt {

// Packed variable-length rows: output row r reads input row in_row[r] (negative: +0.0), only
// rows below *n_dev run, and copy_out receives the gathered input row (the residual stream of
// the first layer).
struct LnRows {
  const int* in_row;
  const int* n_dev;
  half* copy_out;
};

template <int NV>
__global__ __launch_bounds__(256) void layernorm_kernel(const half* __restrict__ x,
                                                        const half* __restrict__ gamma,
                                                        const half* __restrict__ beta,
                                                        const uint8_t* __restrict__ valid,
                                                        half* __restrict__ y, int rows, int d,
                                                        float eps, LnRows pk) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (pk.n_dev != nullptr) rows = min(rows, *pk.n_dev);
  if (row >= rows) return;
  const int nch = d >> 3;
  const size_t base = (size_t)row * d;
  const int src = pk.in_row != nullptr ? pk.in_row[row] : row;
  if ((valid != nullptr && valid[row] == 0) || src < 0) {
    for (int c = lane; c < nch; c += 64) {
      *(uint4*)(y + base + 8 * c) = make_uint4(0, 0, 0, 0);
      if (pk.copy_out != nullptr) *(uint4*)(pk.copy_out + base + 8 * c) = make_uint4(0, 0, 0, 0);
    }
    return;
  }
  const size_t sbase = (size_t)src * d;
  // The row and the affine chunks are loaded together, so gamma / beta do not add a memory round
  // trip after the reductions (the kernel is latency-bound for small row counts).
  half8 v[NV], g[NV], bt[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      v[i] = *(const half8*)(x + sbase + 8 * c);
      if (pk.copy_out != nullptr) *(half8*)(pk.copy_out + base + 8 * c) = v[i];
      g[i] = *(const half8*)(gamma + 8 * c);
      bt[i] = *(const half8*)(beta + 8 * c);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s += (float)v[i][e];
    }
  }
  const float mean = wave_sum(s) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = (float)v[i][e] - mean;
        q += t * t;
      }
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)d + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = (half)(((float)v[i][e] - mean) * rstd * (float)g[i][e] + (float)bt[i][e]);
      *(half8*)(y + base + 8 * c) = o;
    }
  }
}

int launch_layernorm_rows(const half* x, const half* gamma, const half* beta, const uint8_t* valid,
                          const int* in_row, const int* n_dev, half* copy_out, half* y, int rows,
                          int d, float eps, hipStream_t stream) {
  TT_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && d <= 8192,
             "layernorm: need d %% 8 == 0 and 0 < d <= 8192 (got d=%d)", d);
  if (rows == 0) return TT_OK;
  const dim3 grid((rows + 3) / 4), block(256);
  const int nv = (d / 8 + 63) / 64;
  const LnRows pk{in_row, n_dev, copy_out};
  if (nv <= 1)
    hipLaunchKernelGGL(layernorm_kernel<1>, grid, block, 0, stream, x, gamma, beta, valid, y, rows, d, eps, pk);
  else if (nv <= 2)
    hipLaunchKernelGGL(layernorm_kernel<2>, grid, block, 0, stream, x, gamma, beta, valid, y, rows, d, eps, pk);
  else if (nv <= 4)
    hipLaunchKernelGGL(layernorm_kernel<4>, grid, block, 0, stream, x, gamma, beta, valid, y, rows, d, eps, pk);
  else if (nv <= 8)
    hipLaunchKernelGGL(layernorm_kernel<8>, grid, block, 0, stream, x, gamma, beta, valid, y, rows, d, eps, pk);
  else
    hipLaunchKernelGGL(layernorm_kernel<16>, grid, block, 0, stream, x, gamma, beta, valid, y, rows, d, eps, pk);
  return launch_status("layernorm_kernel");
}

int launch_layernorm(const half* x, const half* gamma, const half* beta, const uint8_t* valid,
                     half* y, int rows, int d, float eps, hipStream_t stream) {
  return launch_layernorm_rows(x, gamma, beta, valid, nullptr, nullptr, nullptr, y, rows, d, eps,
                               stream);
}

}  // namespace tt

extern "C" int tt_layernorm_fwd(const void* x, const void* gamma, const void* beta,
                                const uint8_t* valid, void* y, int rows, int d, float eps,
                                void* stream) {
  TT_REQUIRE(x && gamma && beta && y, "layernorm: null pointer");
  return tt::launch_layernorm((const tt::half*)x, (const tt::half*)gamma, (const tt::half*)beta,
                              valid, (tt::half*)y, rows, d, eps, (hipStream_t)stream);
}
