// attn_f32.hip -- the fp32-compute rung (stage 3) for fp32 and fp16 inputs.
#include "attn_kernel.h"

namespace fa {
VariantList variants_s3_f32() { return kern::s3_table<float>(); }
VariantList variants_s3_f16() { return kern::s3_table<_Float16>(); }
}  // namespace fa
