// Flash attention for head_dim 256 (the reference's D = 1024, 4-head shape): the same block as
// head_dim 32 / 64 / 128 (attention_block.hpp: 128 queries per block, 64-key K / V^T tiles
// double-buffered in LDS by global -> LDS copies, S^T = K Q^T and O^T += V^T P^T on
// v_mfma_f32_32x32x16_f16, lazy online softmax in the exp2 domain).
//
// Built without the VGPR-form MFMA flag of attention.hip: at head_dim 256 the output accumulators
// (128 floats per lane) and the Q^T fragments (64 VGPRs) do not fit the 256 architectural VGPRs
// together, so the accumulators live in AGPRs (one wave per SIMD).  LDS: 4 * 64 * 256 * 2 bytes =
// 128 KiB per block.
#include "attention_block.hpp"
#include "kernels.hpp"

namespace tt {

int launch_attention_wide(const AttnArgs& args, const int32_t* info, int head_dim, int causal,
                          hipStream_t stream) {
  TT_REQUIRE(head_dim == 256, "attention_wide: head_dim %d is not 256", head_dim);
  return causal ? launch_attention_hd<256, true>(args, info, stream)
                : launch_attention_hd<256, false>(args, info, stream);
}

}  // namespace tt
