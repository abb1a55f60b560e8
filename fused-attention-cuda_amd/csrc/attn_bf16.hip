// attn_bf16.hip -- bf16 instantiations of the matrix-core kernels (stages 4 and 5).
#include "attn_decode.h"
#include "attn_mfma16.h"

namespace fa {
VariantList variants_s5_bf16() { return m16::s5_table<__bf16>(); }
VariantList variants_s4_bf16() { return m16::s4_table<__bf16>(); }
VariantList variants_s5sync_bf16() { return m16::s5_table<__bf16, 4>(); }
LaunchFn combine_s5_bf16(int D) {
  if (D == 64) return &m16::launch_combine<__bf16, 64>;
  if (D == 128) return &m16::launch_combine<__bf16, 128>;
  return nullptr;
}
DecodeFn decode_bf16(int D) {
  if (D == 64) return &m16::launch_decode<__bf16, 64>;
  if (D == 128) return &m16::launch_decode<__bf16, 128>;
  return nullptr;
}
}  // namespace fa
