// Device half of the include/rdna4/kv.h shim check: kernels that read stored
// rows through rdna4::kv_load<> (one element per call) and rdna4::kv_load8<>
// (8 dims per lane, kv.h:247-368 lane mapping), exported for the GPU tests.
#include "rdna4/kv.h"

using rdna4::KvType;

template <KvType CT>
__global__ void read_rows(const std::uint8_t *rows, float *out, int head_dim, int use8) {
  const std::uint64_t rb = rdna4::kv_row_bytes(CT, head_dim);
  const std::uint8_t *row = rows + (std::uint64_t)blockIdx.x * rb;
  float *o = out + (std::int64_t)blockIdx.x * head_dim;
  if (use8) {
    const int lane = threadIdx.x;
    if (lane * 8 < head_dim) {
      float v[8];
      rdna4::kv_load8<CT>(row, lane, v);
      for (int i = 0; i < 8; ++i) o[lane * 8 + i] = v[i];
    }
  } else {
    for (int d = threadIdx.x; d < head_dim; d += blockDim.x) o[d] = rdna4::kv_load<CT>(row, d);
  }
}

extern "C" int shim_kv_read_rows(int type, const void *rows, float *out, int n_rows, int head_dim,
                                 int use8, void *stream) {
  if (n_rows < 1 || head_dim < 32 || head_dim % 32 || head_dim > 512) return -1;
  const dim3 grid(n_rows), block(64);
  hipStream_t st = (hipStream_t)stream;
  const std::uint8_t *r = (const std::uint8_t *)rows;
  switch ((KvType)type) {
    case KvType::F32: read_rows<KvType::F32><<<grid, block, 0, st>>>(r, out, head_dim, use8); break;
    case KvType::F16: read_rows<KvType::F16><<<grid, block, 0, st>>>(r, out, head_dim, use8); break;
    case KvType::Q8_0: read_rows<KvType::Q8_0><<<grid, block, 0, st>>>(r, out, head_dim, use8); break;
    case KvType::Q4_0: read_rows<KvType::Q4_0><<<grid, block, 0, st>>>(r, out, head_dim, use8); break;
    case KvType::Q5_0: read_rows<KvType::Q5_0><<<grid, block, 0, st>>>(r, out, head_dim, use8); break;
    case KvType::Q4_1: read_rows<KvType::Q4_1><<<grid, block, 0, st>>>(r, out, head_dim, use8); break;
    default: return -2;
  }
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
