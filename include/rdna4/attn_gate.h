// The attention output gate and the row RMSNorm of rdna4-infer's
// include/rdna4/nn.cuh (sigmoid_gate_launch, nn.cuh:405-420; rms_norm_launch,
// nn.cuh:239-243) with the reference's signatures, forwarding to librdna4attn.
// nn.cuh holds many unrelated kernels; a build that takes this library
// replaces those two launchers with these.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "../rdna4attn.h"

namespace rdna4 {

inline bool sigmoid_gate_launch(float *d_g_io, float *d_y_io, std::int64_t n,
                                hipStream_t stream = nullptr) {
  return rd4_sigmoid_gate_launch(d_g_io, d_y_io, n, (void *)stream) == RD4_OK;
}

inline bool rms_norm_launch(const float *d_x, const float *d_w, float *d_y, std::int64_t nrows,
                            std::int64_t ncols, float eps, hipStream_t stream = nullptr) {
  return rd4_rms_norm_launch(d_x, d_w, d_y, nrows, ncols, eps, (void *)stream) == RD4_OK;
}

}  // namespace rdna4
