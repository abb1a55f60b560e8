// attn_bf16.hip -- bf16 instantiations of the matrix-core kernels (stages 4 and 5).
#include "attn_kernel.h"

namespace fa {
VariantList variants_s5_bf16() { return kern::s5_table<__bf16>(); }
VariantList variants_s4_bf16() { return kern::s4_table<__bf16>(); }
}  // namespace fa
