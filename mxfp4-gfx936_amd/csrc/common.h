// Shared device helpers and host status plumbing for libmxfp4_gfx950.
//
// Formats (OCP MX v1.0, as used by the moe_op_mxfp4_soft operator surface):
//   * weights/activations: E2M1 nibbles packed two per byte, the low nibble is
//     the even K index;
//   * one E8M0 byte per 32 consecutive K values, value 2^(s-127), s = 255 NaN.
// gfx950 converts a byte of two E2M1 codes times an FP32 scale to two
// bf16/fp16 values in one instruction (v_cvt_scalef32_pk_{bf16,f16}_fp4);
// fed the scale 2^(s-127) (the FP32 subnormal 2^-127 for s = 0, a quiet NaN
// for s = 255) it returns exactly the reference's dequantized value rounded to
// bf16/fp16, for all 16 codes x 256 scales.
#pragma once

#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxfp4_gfx950.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

namespace mx {

// ---------------------------------------------------------------- host side
// Thread-local message for the last failing call; see mxfp4_last_error().
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);  // 0 or MXFP4_ERR_HIP
int launch_status(const char* what);             // checks hipGetLastError()

// ---------------------------------------------------------------- device side

// Raw (MUBUF) buffer loads through a 128-bit resource {base, byte size,
// raw-buffer flags}: a lane whose byte offset lies at or past the size reads
// zero instead of memory.  Kernels use kOOB for padding rows and K tails,
// so their loads need no branches; every resource they build is at most
// 2 GiB, which keeps kOOB out of range.
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ i32x4 make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return i32x4{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)bytes, 0x00020000};
}

extern "C" __device__ i32x4 llvm_amdgcn_raw_buffer_load_v4i32(i32x4 rsrc, uint32_t voffset,
                                                               int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");
extern "C" __device__ i32x2 llvm_amdgcn_raw_buffer_load_v2i32(i32x4 rsrc, uint32_t voffset,
                                                               int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v2i32");
extern "C" __device__ int llvm_amdgcn_raw_buffer_load_i32(i32x4 rsrc, uint32_t voffset,
                                                           int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");
extern "C" __device__ uint8_t llvm_amdgcn_raw_buffer_load_i8(i32x4 rsrc, uint32_t voffset,
                                                             int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i8");

__device__ __forceinline__ i32x4 buf_load16(i32x4 rsrc, uint32_t off) {
  return llvm_amdgcn_raw_buffer_load_v4i32(rsrc, off, 0, 0);
}
__device__ __forceinline__ i32x2 buf_load8(i32x4 rsrc, uint32_t off) {
  return llvm_amdgcn_raw_buffer_load_v2i32(rsrc, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load4(i32x4 rsrc, uint32_t off) {
  return (uint32_t)llvm_amdgcn_raw_buffer_load_i32(rsrc, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load_u8(i32x4 rsrc, uint32_t off) {
  return llvm_amdgcn_raw_buffer_load_i8(rsrc, off, 0, 0);
}

// Direct-to-LDS buffer loads: each lane's `size` bytes land at the wave's
// LDS base (taken from M0) + size x lane, without passing through VGPRs.
// The compiler does not order later LDS reads after these writes: callers
// wait with wait_vmcnt and a barrier.
typedef __attribute__((address_space(3))) uint32_t lds_u32;

extern "C" __device__ void llvm_amdgcn_raw_buffer_load_lds(i32x4 rsrc, lds_u32* lds, int size,
                                                           int voffset, int soffset, int offset,
                                                           int aux)
    __asm("llvm.amdgcn.raw.buffer.load.lds");

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Calls f(std::integral_constant<int, I>{}) for I = B .. E-1 (compile-time
// indices for register arrays and template arguments inside loops).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// s_barrier without __syncthreads' release / acquire fences (which would
// wait for every outstanding global load).  The empty asm statements with
// memory clobbers keep the compiler from moving memory accesses across it;
// callers wait for the LDS traffic the barrier publishes themselves.
__device__ __forceinline__ void barrier_only() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ lds_u32* lds_ptr(uint8_t* p) {
  return (lds_u32*)(__attribute__((address_space(3))) uint8_t*)p;
}

// E8M0 byte -> scale operand of v_cvt_scalef32_pk_*_fp4.  The converter
// reads only the exponent field of that operand (verified on the device for
// every scale byte x every code pair: a mantissa of 0.5 changes no output
// bit), so the byte goes straight into the exponent.  The 0x400000 mantissa
// bit makes s = 0 the subnormal 2^-127 and s = 255 a quiet NaN, the two
// encodings the converter is known to treat as 2^-127 and NaN.  One
// v_lshl_or_b32.  The result is only meaningful as the converter's operand.
__device__ __forceinline__ float e8m0_scale(uint32_t s) {
  return __uint_as_float((s << 23) | 0x00400000u);
}

// Eight E2M1 codes (one dword, low nibble first) times scale -> 8 x T.
template <typename T>
struct Decode;

template <>
struct Decode<__bf16> {
  typedef bf16x8 vec8;
  __device__ __forceinline__ static bf16x8 run(uint32_t p, float scale) {
    bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, scale, 0);
    bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, scale, 1);
    bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, scale, 2);
    bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, scale, 3);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
  }
};

template <>
struct Decode<_Float16> {
  typedef f16x8 vec8;
  __device__ __forceinline__ static f16x8 run(uint32_t p, float scale) {
    f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(p, scale, 0);
    f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(p, scale, 1);
    f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(p, scale, 2);
    f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(p, scale, 3);
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
  }
};

// 16x16x32 MFMA, FP32 accumulate.  Lane l holds A[l%16][(l/16)*8 + 0..7],
// B[(l/16)*8 + 0..7][l%16]; the result lane l holds D[(l/16)*4 + i][l%16].
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Scalar conversions with round-to-nearest-even.
template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }

template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

}  // namespace mx
