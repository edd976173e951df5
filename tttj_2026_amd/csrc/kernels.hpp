// Internal launch functions shared by the C-ABI entry points and the forward executor.
#pragma once

#include "common.hpp"

namespace tt {

struct EpiArgs {
  const half* bias;      // [N]
  const half* resid;     // [M, ldy] (may alias y)
  const uint8_t* valid;  // [M] or nullptr
  half* y;
  int ldy;
  int mode;              // TT_EPI_*
  int batch, seq, heads, head_dim, d_model;  // TT_EPI_QKV only
};

int launch_layernorm(const half* x, const half* gamma, const half* beta, const uint8_t* valid,
                     half* y, int rows, int d, float eps, hipStream_t stream);

int launch_linear(const half* x, const half* w, int m, int n, int k, const EpiArgs& ep,
                  hipStream_t stream);

int launch_mask_info(const uint8_t* mask, int32_t* info, int batch, int seq, hipStream_t stream);

int launch_attention(const half* q, const half* k, const half* vt, const uint8_t* mask,
                     const int32_t* info, half* ctx, int batch, int seq, int heads, int head_dim,
                     int causal, hipStream_t stream);

}  // namespace tt
