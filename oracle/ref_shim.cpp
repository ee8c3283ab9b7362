// Exposes the reference's host-side fp16 conversion and KV tables through a C
// ABI so tests can pin the oracle against them. Compiled against the headers at
// their original location (/root/reference/include); output oracle/_ref/.
// TEST INFRASTRUCTURE ONLY.
#include "rdna4/kv.h"

extern "C" {
unsigned short ref_f32_to_f16(float f) { return rdna4::float_to_fp16(f); }
float ref_f16_to_f32(unsigned short h) { return rdna4::fp16_to_float(h); }
long long ref_row_bytes(int t, int head_dim) {
  return (long long)rdna4::kv_row_bytes((rdna4::KvType)t, head_dim);
}
double ref_bytes_per_elem(int t) { return rdna4::kv_bytes_per_elem((rdna4::KvType)t); }
int ref_type_parse(const char *name) {
  rdna4::KvType t = rdna4::KvType::F16;
  return rdna4::kv_type_parse(name, &t) == nullptr ? (int)t : -1;
}
const char *ref_type_name(int t) { return rdna4::kv_type_name((rdna4::KvType)t); }
}
