// The attention output gate of rdna4-infer's include/rdna4/nn.cuh:405-420
// (sigmoid_gate_launch) with the reference's signature, forwarding to
// librdna4attn. nn.cuh holds many unrelated kernels; a build that takes this
// library replaces its sigmoid_gate_launch with this one.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "../rdna4attn.h"

namespace rdna4 {

inline bool sigmoid_gate_launch(float *d_g_io, float *d_y_io, std::int64_t n,
                                hipStream_t stream = nullptr) {
  return rd4_sigmoid_gate_launch(d_g_io, d_y_io, n, (void *)stream) == RD4_OK;
}

}  // namespace rdna4
