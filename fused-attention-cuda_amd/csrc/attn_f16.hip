// attn_f16.hip -- fp16 instantiations of the matrix-core kernels (stages 4 and 5).
#include "attn_kernel.h"

namespace fa {
VariantList variants_s5_f16() { return kern::s5_table<_Float16>(); }
VariantList variants_s4_f16() { return kern::s4_table<_Float16>(); }
}  // namespace fa
