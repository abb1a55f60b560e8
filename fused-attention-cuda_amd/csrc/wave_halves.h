// wave_halves.h -- reductions across the two 32-lane halves of a wave64.
//
// In the MFMA accumulator layouts the kernels use, lane l and lane l ^ 32 hold the two halves of
// one query row, so a row's max or sum is the lane's own partial combined with its partner's.
// v_permlane32_swap exchanges the two halves on the VALU, with no trip through the LDS crossbar
// that a ds_bpermute (__shfl_xor) takes. Called with the same value in both operands, it returns
// the low half's value and the high half's value in every lane. max and + are commutative, so
// each lane gets the same bits as from its own value combined with its partner's.
#pragma once

#include <hip/hip_runtime.h>

namespace fa {

__device__ __forceinline__ float halves_max(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<unsigned>(sw[0])),
               __builtin_bit_cast(float, static_cast<unsigned>(sw[1])));
}

__device__ __forceinline__ float halves_sum(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, static_cast<unsigned>(sw[0])) +
         __builtin_bit_cast(float, static_cast<unsigned>(sw[1]));
}

}  // namespace fa
