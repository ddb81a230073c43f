// Internal interface of the residual-add + RMSNorm kernels (norm.hip), the MoE layer's serving neighbours.
#pragma once

#include "common.h"

namespace janus {

constexpr int kMaxNormH = 4096;  // 16 four-column groups per lane

int check_norm_sizes(int T, int H);
// x_out = bf16(residual + h) (h null: residual), n_out = Qwen3_5RMSNorm(x_out) with weight w, 0 where valid[t] == 0
// (valid null: every row). x_out may be null, or alias residual; n_out may alias h.
int launch_add_rmsnorm(const uint16_t* residual, const uint16_t* h, const uint16_t* w, float eps, const uint8_t* valid,
                       int T, int H, uint16_t* x_out, uint16_t* n_out, hipStream_t stream);
// The combine (moe = bf16 of the slot sum, the slot format of gemm.h; 0 where moe_valid[t] == 0) followed by
// x_res = bf16(x_res + moe) in place and n_out = Qwen3_5RMSNorm(x_res), 0 where valid[t] == 0.
int launch_combine_add_rmsnorm(const int16_t* slots, const float* slot_scale, int nslots, const uint8_t* moe_valid,
                               uint16_t* x_res, const uint16_t* w, float eps, const uint8_t* valid, int T, int H,
                               uint16_t* n_out, hipStream_t stream);

}  // namespace janus
