// dequant_mxfp4 (soft:277-307) as one HBM-streaming kernel.
//
// The reference builds ~10 full-size temporaries (codes, int64 gather
// indices, repeated scales, exp2, where) per call; here each thread turns one
// packed dword (8 codes) and its E8M0 byte into 8 outputs with four
// v_cvt_scalef32_pk_* instructions: 4 B + 1/4 B read, 16 B (bf16/f16) or
// 32 B (f32) written, consecutive lanes on consecutive 16-byte chunks.
#include "common.h"

namespace mx {
namespace {

template <int DT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ packed,
                                                      int64_t pstride,
                                                      const uint8_t* __restrict__ scales,
                                                      int64_t sstride, int64_t rows, int64_t k,
                                                      void* __restrict__ out) {
  const int64_t units_per_row = k >> 3;  // 8 values per unit
  // a workgroup takes 256 consecutive units of one row, so the row index is
  // one scalar division per workgroup step, not a 64-bit division per lane
  const int64_t chunks = (units_per_row + 255) >> 8;  // per row
  const int64_t total = rows * chunks;
  for (int64_t gch = blockIdx.x; gch < total; gch += gridDim.x) {
    const int64_t r = gch / chunks;
    const int64_t c = (gch - r * chunks) * 256 + threadIdx.x;
    if (c >= units_per_row) continue;
    const uint32_t p = *reinterpret_cast<const uint32_t*>(packed + r * pstride + c * 4);
    const uint32_t s = scales[r * sstride + (c >> 2)];
    const int64_t o = r * k + c * 8;
    if (DT == MXFP4_DT_F32) {
      // bf16 holds every product exactly (at most two significant bits and
      // the FP32 exponent range), so widening it gives the FP32 value.
      bf16x8 v = Decode<__bf16>::run(p, e8m0_scale(s));
      f32x4 lo, hi;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = (float)v[i];
        hi[i] = (float)v[i + 4];
      }
      if (s == 255u) {  // canonical NaN of the reference (0x7FC00000)
        const float nan = __uint_as_float(0x7FC00000u);
        lo = f32x4{nan, nan, nan, nan};
        hi = lo;
      }
      f32x4* dst = reinterpret_cast<f32x4*>(static_cast<float*>(out) + o);
      dst[0] = lo;
      dst[1] = hi;
    } else if (DT == MXFP4_DT_BF16) {
      bf16x8 v = Decode<__bf16>::run(p, e8m0_scale(s));
      u16x8 bits = __builtin_bit_cast(u16x8, v);
      if (s == 255u) bits = u16x8{0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0};
      *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(out) + o) = bits;
    } else {
      f16x8 v = Decode<_Float16>::run(p, e8m0_scale(s));
      u16x8 bits = __builtin_bit_cast(u16x8, v);
      if (s == 255u) bits = u16x8{0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00};
      *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(out) + o) = bits;
    }
  }
}

}  // namespace
}  // namespace mx

extern "C" int mxfp4_dequant(const uint8_t* packed, int64_t packed_row_stride,
                             const uint8_t* scales, int64_t scale_row_stride, int64_t rows,
                             int64_t k, void* out, int out_dtype, void* stream) {
  using namespace mx;
  if (out_dtype != MXFP4_DT_F32 && out_dtype != MXFP4_DT_BF16 && out_dtype != MXFP4_DT_F16) {
    set_error("dequant: unsupported output dtype %d", out_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (rows < 0 || k < 0 || k % 32 != 0) {
    set_error("logical K must be divisible by 32, got %lld", (long long)k);
    return MXFP4_ERR_VALUE;
  }
  if (packed_row_stride < k / 2 || scale_row_stride < k / 32 || (packed_row_stride % 4) != 0 ||
      (reinterpret_cast<uintptr_t>(packed) % 4) != 0 || (reinterpret_cast<uintptr_t>(out) % 16) != 0) {
    set_error("dequant: packed rows must be 4-byte aligned and out 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  const int64_t total = rows * (k / 8);
  if (total == 0) return MXFP4_OK;
  const int64_t want = rows * ((k / 8 + 255) / 256);  // workgroup steps
  const int grid = (int)(want < 16384 ? want : 16384);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case MXFP4_DT_F32:
      dequant_kernel<MXFP4_DT_F32><<<grid, 256, 0, st>>>(packed, packed_row_stride, scales,
                                                         scale_row_stride, rows, k, out);
      break;
    case MXFP4_DT_BF16:
      dequant_kernel<MXFP4_DT_BF16><<<grid, 256, 0, st>>>(packed, packed_row_stride, scales,
                                                          scale_row_stride, rows, k, out);
      break;
    default:
      dequant_kernel<MXFP4_DT_F16><<<grid, 256, 0, st>>>(packed, packed_row_stride, scales,
                                                         scale_row_stride, rows, k, out);
      break;
  }
  return launch_status("dequant launch");
}
