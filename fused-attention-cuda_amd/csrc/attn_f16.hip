// attn_f16.hip -- fp16 instantiations of the matrix-core kernels (stages 4 and 5).
#include "attn_decode.h"
#include "attn_mfma16.h"

namespace fa {
VariantList variants_s5_f16() { return m16::s5_table<_Float16>(); }
VariantList variants_s4_f16() { return m16::s4_table<_Float16>(); }
VariantList variants_s5sync_f16() { return m16::s5_table<_Float16, 4>(); }
LaunchFn combine_s5_f16(int D) {
  if (D == 64) return &m16::launch_combine<_Float16, 64>;
  if (D == 128) return &m16::launch_combine<_Float16, 128>;
  return nullptr;
}
DecodeFn decode_f16(int D) {
  if (D == 64) return &m16::launch_decode<_Float16, 64>;
  if (D == 128) return &m16::launch_decode<_Float16, 128>;
  return nullptr;
}
}  // namespace fa
