// MXFP4 activation quantizer: x [rows, k] -> packed E2M1 [rows, k/2] + E8M0
// [rows, k/32].  The step before the W4A4 GEMM.
//
// MXFP4_QUANT_TIES_AWAY restates the reference test quantizer
// torch_dynamic_mxfp4_quant (test:28-60) operation by operation: the block
// amax is rounded to a power of two by adding 0x200000 to its FP32 bits and
// masking the mantissa, E = clamp(floor(log2 amax') - 2, -127, 127), and each
// x * 2^-E is truncated to three bits and rounded half away from zero in the
// integer domain, saturating at 6; the scale byte is (E + 127) mod 256.
// MXFP4_QUANT_RNE is the OCP MX rule: E = floor(log2 amax) - 2, E2M1 round
// to nearest even, saturating at +-6.  In both, the sign bit follows the input
// (negative values that round to 0 give code 8, -0).
#include "common.h"

namespace mx {
namespace {

__device__ __forceinline__ float pow2_f32(int e) {  // 2^e for e in [-127, 127]
  return e >= -126 ? __uint_as_float((uint32_t)(e + 127) << 23) : __uint_as_float(0x00400000u);
}

// floor(log2(v)) for finite v > 0, from the bits
__device__ __forceinline__ int floor_log2(float v) {
  const uint32_t b = __float_as_uint(v);
  const int ex = (int)((b >> 23) & 0xFF);
  if (ex) return ex - 127;
  return (31 - __builtin_clz(b & 0x7FFFFF)) - 149;
}

__device__ __forceinline__ int clamp_e(int e) { return e < -127 ? -127 : (e > 127 ? 127 : e); }

__device__ __forceinline__ uint32_t code_ties_away(float q) {
  const uint32_t qi = __float_as_uint(q);
  const uint32_t sign = qi & 0x80000000u;
  int32_t ex = (int32_t)((qi >> 23) & 0xFF);
  int32_t mant = (int32_t)(qi & 0x7FFFFF);
  if (ex < 127) {
    const int sh = 127 - ex - 1;
    mant = sh < 32 ? ((0x400000 | (mant >> 1)) >> sh) : 0;
  }
  ex = (ex > 126 ? ex : 126) - 126;
  const int32_t comb = (((ex << 2) | (mant >> 21)) + 1) >> 1;
  const int32_t mag = comb < 7 ? comb : 7;
  return ((sign >> 28) & 0xFu) | (uint32_t)mag;
}

__device__ __forceinline__ uint32_t code_rne(float q) {
  const float m = fabsf(q);
  const uint32_t c = (uint32_t)(m > 0.25f) + (uint32_t)(m >= 0.75f) + (uint32_t)(m > 1.25f) +
                     (uint32_t)(m >= 1.75f) + (uint32_t)(m > 2.5f) + (uint32_t)(m >= 3.5f) +
                     (uint32_t)(m > 5.0f);
  return c | ((__float_as_uint(q) >> 28) & 8u);
}

template <typename T, int MODE>
__global__ __launch_bounds__(256) void quant_kernel(const T* __restrict__ x, int64_t rows,
                                                    int64_t k, int64_t ldx,
                                                    uint8_t* __restrict__ packed,
                                                    uint8_t* __restrict__ scales) {
  const int64_t bpr = k >> 5;
  const int64_t total = rows * bpr;
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < total;
       u += (int64_t)gridDim.x * 256) {
    const int64_t r = u / bpr;
    const int64_t b = u - r * bpr;
    const T* src = x + r * ldx + b * 32;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = (float)src[j];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    int e;
    if (MODE == MXFP4_QUANT_TIES_AWAY) {
      const uint32_t ab = (__float_as_uint(amax) + 0x200000u) & 0xFF800000u;
      const float ar = __uint_as_float(ab);
      if (ar == 0.f) e = -127;
      else if (isinf(ar)) e = 127;
      else e = clamp_e(floor_log2(ar) - 2);
    } else {
      if (amax == 0.f) e = -127;
      else if (isinf(amax)) e = 127;
      else e = clamp_e(floor_log2(amax) - 2);
    }
    const float inv = pow2_f32(-e);
    uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const float q = v[j] * inv;
      const uint32_t c = MODE == MXFP4_QUANT_TIES_AWAY ? code_ties_away(q) : code_rne(q);
      words[j >> 3] |= (c & 15u) << ((j & 7) * 4);
    }
    *reinterpret_cast<i32x4*>(packed + r * (k >> 1) + b * 16) =
        i32x4{(int)words[0], (int)words[1], (int)words[2], (int)words[3]};
    scales[r * bpr + b] = (uint8_t)((e + 127) & 0xFF);
  }
}

// RNE quantizer for 16-bit inputs on gfx950's FP4 encoder.
// v_cvt_scalef32_pk_fp4_{bf16,f16}(pair, 2^E) equals code_rne(x * 2^-E) for
// every non-NaN bf16 / f16 value and every E in [-127, 127] (checked on the
// device, exhaustively), and writes its two nibbles into a chosen byte of
// the destination, so one instruction handles two elements and packs them.
// Four consecutive lanes share a 32-block (16 bytes of input each: 1 KB per
// wave load, 256 contiguous output bytes per wave store); the block amax is
// an integer max of the magnitude bits (their order is the float order
// below NaN), reduced over the four lanes.  A block holding a NaN takes the
// scalar path above, so NaN handling is unchanged (ignored by the amax, code
// = its sign).  Needs 16-byte aligned rows.
template <typename T>
__global__ __launch_bounds__(256) void quant_rne16(const T* __restrict__ x, int64_t rows, int64_t k,
                                                   int64_t ldx, uint8_t* __restrict__ packed,
                                                   uint8_t* __restrict__ scales) {
  static_assert(sizeof(T) == 2, "16-bit inputs");
  constexpr uint32_t kInf = std::is_same<T, __bf16>::value ? 0x7F80u : 0x7C00u;
  typedef T T2 __attribute__((ext_vector_type(2)));
  const int64_t bpr = k >> 5;
  const int64_t total = rows * bpr;
  const int q = threadIdx.x & 3;
  for (int64_t u = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 2; u < total;
       u += (int64_t)gridDim.x * 64) {
    const int64_t r = u / bpr;
    const int64_t b = u - r * bpr;
    const T* src = x + r * ldx + b * 32 + q * 8;
    const i32x4 w = *reinterpret_cast<const i32x4*>(src);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = (uint32_t)w[j] & 0x7FFF7FFFu;
      const uint32_t lo = a & 0xFFFFu, hi = a >> 16;
      m = m > lo ? m : lo;
      m = m > hi ? m : hi;
    }
    uint32_t o = (uint32_t)__shfl_xor((int)m, 1);
    m = m > o ? m : o;
    o = (uint32_t)__shfl_xor((int)m, 2);
    m = m > o ? m : o;
    uint32_t word = 0;
    int e;
    if (m <= kInf) {
      const float amax = std::is_same<T, __bf16>::value
                             ? __uint_as_float(m << 16)
                             : (float)__builtin_bit_cast(_Float16, (uint16_t)m);
      if (amax == 0.f) e = -127;
      else if (isinf(amax)) e = 127;
      else e = clamp_e(floor_log2(amax) - 2);
      const float sc = pow2_f32(e);
      static_for<0, 4>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        // (int) first: this clang bit-casts an element of a vector lvalue as
        // element 0, whatever the index
        const T2 v = __builtin_bit_cast(T2, (int)w[j]);
        if constexpr (std::is_same<T, __bf16>::value)
          word = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(word, v, sc, j);
        else
          word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f16(word, v, sc, j);
      });
    } else {  // a NaN in the block: the scalar rule
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (float)src[j];
      float amax = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      if (amax == 0.f) e = -127;
      else if (isinf(amax)) e = 127;
      else e = clamp_e(floor_log2(amax) - 2);
      const float inv = pow2_f32(-e);
#pragma unroll
      for (int j = 0; j < 8; ++j) word |= (code_rne(v[j] * inv) & 15u) << (j * 4);
    }
    *reinterpret_cast<uint32_t*>(packed + r * (k >> 1) + b * 16 + q * 4) = word;
    if (q == 0) scales[r * bpr + b] = (uint8_t)((e + 127) & 0xFF);
  }
}

template <typename T>
void launch_quant_typed(const void* x, int64_t rows, int64_t k, int64_t ldx, int mode,
                        uint8_t* packed, uint8_t* scales, int grid, hipStream_t st) {
  if (mode == MXFP4_QUANT_TIES_AWAY)
    quant_kernel<T, MXFP4_QUANT_TIES_AWAY><<<grid, 256, 0, st>>>(static_cast<const T*>(x), rows, k,
                                                                 ldx, packed, scales);
  else
    quant_kernel<T, MXFP4_QUANT_RNE><<<grid, 256, 0, st>>>(static_cast<const T*>(x), rows, k, ldx,
                                                           packed, scales);
}

}  // namespace
}  // namespace mx

extern "C" int mxfp4_quant(const void* x, int x_dtype, int64_t rows, int64_t k,
                           int64_t x_row_stride, int mode, uint8_t* packed, uint8_t* scales,
                           void* stream) {
  using namespace mx;
  if (x_dtype != MXFP4_DT_BF16 && x_dtype != MXFP4_DT_F16 && x_dtype != MXFP4_DT_F32) {
    set_error("quant: unsupported input dtype %d", x_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (mode != MXFP4_QUANT_TIES_AWAY && mode != MXFP4_QUANT_RNE) {
    set_error("quant: unknown mode %d", mode);
    return MXFP4_ERR_VALUE;
  }
  if (rows < 0 || k < 0 || k % 32 != 0 || x_row_stride < k) {
    set_error("quantizer requires K divisible by 32, got %lld", (long long)k);
    return MXFP4_ERR_VALUE;
  }
  if ((reinterpret_cast<uintptr_t>(packed) & 15) != 0) {
    set_error("quant: packed output must be 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  const int64_t total = rows * (k / 32);
  if (total == 0) return MXFP4_OK;
  const int grid = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // 16-bit inputs with 16-byte aligned rows: the RNE rule on the FP4 encoder
  const bool rows16 = ((reinterpret_cast<uintptr_t>(x) | (uintptr_t)(x_row_stride * 2)) & 15) == 0;
  if (mode == MXFP4_QUANT_RNE && x_dtype != MXFP4_DT_F32 && rows16) {
    const int g16 = (int)((total + 63) / 64 < 16384 ? (total + 63) / 64 : 16384);
    if (x_dtype == MXFP4_DT_BF16)
      quant_rne16<__bf16><<<g16, 256, 0, st>>>(static_cast<const __bf16*>(x), rows, k, x_row_stride,
                                               packed, scales);
    else
      quant_rne16<_Float16><<<g16, 256, 0, st>>>(static_cast<const _Float16*>(x), rows, k,
                                                 x_row_stride, packed, scales);
    return launch_status("quant launch");
  }
  switch (x_dtype) {
    case MXFP4_DT_BF16:
      launch_quant_typed<__bf16>(x, rows, k, x_row_stride, mode, packed, scales, grid, st);
      break;
    case MXFP4_DT_F16:
      launch_quant_typed<_Float16>(x, rows, k, x_row_stride, mode, packed, scales, grid, st);
      break;
    default:
      launch_quant_typed<float>(x, rows, k, x_row_stride, mode, packed, scales, grid, st);
      break;
  }
  return launch_status("quant launch");
}
