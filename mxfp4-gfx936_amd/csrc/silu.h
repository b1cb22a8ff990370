// SiLU rounded to the activation type, by table lookup.
//
// The gate_up epilogue rounds the gate to T (bf16 / fp16) before SiLU and
// the SiLU result to T after it (vllm:249-252 on tensors of T), so SiLU is
// a function of the 65536 bit patterns of T.  build.py generates both
// tables (mxfp4-gfx936_amd/silu_table.py: torch's FP32 steps x / (1 +
// exp(-x)), exp correctly rounded, then round-to-nearest-even to T) into
// _build/gen/silu_table.inc; one 2-byte load replaces an FP32 exp and an
// IEEE division per output, ~2/3 of the gate_up epilogue's VALU work.
#pragma once
#include <type_traits>

#include "common.h"

namespace mx {

#include "silu_table.inc"

// silu(g) rounded to T; FP32 (no rounding step to tabulate) evaluates it
template <typename T>
__device__ __forceinline__ T silu_round(T g) {
  if constexpr (std::is_same<T, __bf16>::value) {
    return __builtin_bit_cast(T, kSiluBf16[__builtin_bit_cast(uint16_t, g)]);
  } else if constexpr (std::is_same<T, _Float16>::value) {
    return __builtin_bit_cast(T, kSiluF16[__builtin_bit_cast(uint16_t, g)]);
  } else {
    return from_f32<T>(silu_f32(to_f32(g)));
  }
}

}  // namespace mx
