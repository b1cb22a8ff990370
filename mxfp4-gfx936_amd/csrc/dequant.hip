// dequant_mxfp4 (soft:277-307) as one HBM-streaming kernel.
//
// The reference builds ~10 full-size temporaries (codes, int64 gather
// indices, repeated scales, exp2, where) per call; here the codes go through
// v_cvt_scalef32_pk_* (two values per instruction, the E8M0 byte as the
// scale operand's exponent) straight from the packed bytes.
//
// dequant_wide (rows of 16-byte aligned packed bytes): a wave takes blocks
// of 2048 values of one row (1 KB of packed input, one E8M0 block of 32
// values per lane).  Each lane loads its block's 16 bytes and scale byte,
// kWideUnroll blocks per wave before any is used, and stages them in the
// wave's LDS slot; it then reads them back in store order -- for bf16 / f16
// dword j*64 + l at step j, for f32 half-dword j*64 + l -- so every output
// store instruction writes 64 consecutive 16-byte chunks (1 KB).  The kernel
// moves 0.53 B in and 2 (4) B out per value.  Measured (MI355X, 128 x 1536
// x 2048 -> 805 MB of bf16): 4-byte loads, one unit per lane and step 211
// us (60% of HBM); 16-byte loads through LDS 184 us; one pass of waves
// instead of a grid capped at 8192 workgroups 175 us; non-temporal stores
// 145 us (88%; f32 out 286 us, 80%, against 430 us with each lane's 32
// bytes as two 16-byte stores).  Non-temporal stores are used for outputs
// of at least the 256 MiB MALL, which cannot keep them anyway: a smaller
// output stays cache-resident for the consumer that reads it next.
// dequant_kernel (any 4-byte aligned rows): one packed dword (8 codes) and
// its E8M0 byte per lane and step.
#include "common.h"

namespace mx {
namespace {

// Eight codes (one dword) times scale byte s -> the output type's bits,
// written as 16 (bf16 / f16) or 32 (f32) bytes at `dst`.  s = 255 gives the
// reference's canonical NaN (0x7FC0 / 0x7E00 / 0x7FC00000).
template <int DT>
__device__ __forceinline__ void decode_store(uint32_t p, uint32_t s, void* dst) {
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
    if (s == 255u) {
      const float nan = __uint_as_float(0x7FC00000u);
      lo = f32x4{nan, nan, nan, nan};
      hi = lo;
    }
    reinterpret_cast<f32x4*>(dst)[0] = lo;
    reinterpret_cast<f32x4*>(dst)[1] = hi;
  } else if (DT == MXFP4_DT_BF16) {
    u16x8 bits = __builtin_bit_cast(u16x8, Decode<__bf16>::run(p, e8m0_scale(s)));
    if (s == 255u) bits = u16x8{0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0};
    *reinterpret_cast<u16x8*>(dst) = bits;
  } else {
    u16x8 bits = __builtin_bit_cast(u16x8, Decode<_Float16>::run(p, e8m0_scale(s)));
    if (s == 255u) bits = u16x8{0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00};
    *reinterpret_cast<u16x8*>(dst) = bits;
  }
}

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
    constexpr int OB = (DT == MXFP4_DT_F32) ? 4 : 2;  // output bytes per value
    decode_store<DT>(p, s, static_cast<uint8_t*>(out) + (r * k + c * 8) * OB);
  }
}

constexpr int kWideUnroll = 2;  // blocks of 2048 values a wave loads before using any

template <int DT, bool NT>
__global__ __launch_bounds__(256) void dequant_wide(const uint8_t* __restrict__ packed,
                                                    int64_t pstride,
                                                    const uint8_t* __restrict__ scales,
                                                    int64_t sstride, int64_t rows, int64_t k,
                                                    void* __restrict__ out) {
  constexpr int U = kWideUnroll;
  constexpr int OB = (DT == MXFP4_DT_F32) ? 4 : 2;  // output bytes per value
  __shared__ i32x4 s_data[4][U][64];
  __shared__ uint8_t s_scale[4][U][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t chunks_per_row = k >> 5;         // 16-byte chunks (32 values, one scale)
  const int64_t bpr = (chunks_per_row + 63) >> 6;  // blocks of 64 chunks per row
  const int64_t total = rows * bpr;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t w0 = ((int64_t)blockIdx.x * 4 + wave) * U; w0 < total; w0 += nwaves * U) {
    int64_t row[U], blk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t w = w0 + u;
      row[u] = w / bpr;
      blk[u] = w - row[u] * bpr;
    }
    // every load of the U blocks first
    i32x4 d[U];
    uint32_t sb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = blk[u] * 64 + lane;  // chunk of the row
      const bool ok = w0 + u < total && q < chunks_per_row;
      d[u] = ok ? *reinterpret_cast<const i32x4*>(packed + row[u] * pstride + q * 16)
                : i32x4{0, 0, 0, 0};
      sb[u] = ok ? scales[row[u] * sstride + q] : 0u;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      s_data[wave][u][lane] = d[u];
      s_scale[wave][u][lane] = (uint8_t)sb[u];
    }
    // (the wave's own LDS slot: its accesses are ordered, no barrier)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (w0 + u >= total) break;  // the same for the whole wave
      const uint32_t* dw = reinterpret_cast<const uint32_t*>(&s_data[wave][u][0]);
      uint8_t* const orow = static_cast<uint8_t*>(out) + row[u] * k * OB;
      if constexpr (DT == MXFP4_DT_F32) {
        // 16-byte chunks of 4 values: chunk c is half c & 1 of dword c >> 1
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int c = j * 64 + lane;
          const int64_t v0 = blk[u] * 2048 + c * 4;  // first value of the chunk
          if (v0 >= k) continue;
          const uint32_t sb = s_scale[wave][u][c >> 3];
          const uint32_t d = dw[c >> 1] >> ((c & 1) * 16);
          // bf16 holds every product exactly, so widening it gives the FP32 value
          const bf16x2 x = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, e8m0_scale(sb), 0);
          const bf16x2 y = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, e8m0_scale(sb), 1);
          f32x4 o = f32x4{(float)x[0], (float)x[1], (float)y[0], (float)y[1]};
          if (sb == 255u) {
            const float nan = __uint_as_float(0x7FC00000u);
            o = f32x4{nan, nan, nan, nan};
          }
          f32x4* dst = reinterpret_cast<f32x4*>(orow + v0 * 4);
          if (NT) __builtin_nontemporal_store(o, dst);
          else *dst = o;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = j * 64 + lane;            // dword of the block
          const int64_t unit = blk[u] * 256 + c;  // 8-value unit of the row
          if (unit * 8 >= k) continue;
          const uint32_t sb = s_scale[wave][u][c >> 2];
          u16x8 bits;
          if (DT == MXFP4_DT_BF16) {
            bits = __builtin_bit_cast(u16x8, Decode<__bf16>::run(dw[c], e8m0_scale(sb)));
            if (sb == 255u) bits = u16x8{0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0, 0x7FC0};
          } else {
            bits = __builtin_bit_cast(u16x8, Decode<_Float16>::run(dw[c], e8m0_scale(sb)));
            if (sb == 255u) bits = u16x8{0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00, 0x7E00};
          }
          i32x4* dst = reinterpret_cast<i32x4*>(orow + unit * 8 * OB);
          if (NT) __builtin_nontemporal_store(__builtin_bit_cast(i32x4, bits), dst);
          else *dst = __builtin_bit_cast(i32x4, bits);
        }
      }
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((reinterpret_cast<uintptr_t>(packed) % 16) == 0 && (packed_row_stride % 16) == 0) {
    // 16-byte chunks: k % 32 == 0 makes every row a whole number of them
    const int64_t blocks = rows * ((k / 32 + 63) / 64);  // wave blocks of 2048 values
    const int64_t want = (blocks + 4 * kWideUnroll - 1) / (4 * kWideUnroll);
    const unsigned grid = (unsigned)(want < (1 << 30) ? want : (1 << 30));
    const int64_t out_bytes = total * 8 * (out_dtype == MXFP4_DT_F32 ? 4 : 2);
    const bool nt = out_bytes >= ((int64_t)256 << 20);  // non-temporal stores
#define MX_DQ_WIDE(DTV)                                                                       \
  do {                                                                                        \
    if (nt)                                                                                   \
      dequant_wide<DTV, true><<<grid, 256, 0, st>>>(packed, packed_row_stride, scales,       \
                                                   scale_row_stride, rows, k, out);          \
    else                                                                                      \
      dequant_wide<DTV, false><<<grid, 256, 0, st>>>(packed, packed_row_stride, scales,      \
                                                    scale_row_stride, rows, k, out);         \
  } while (0)
    switch (out_dtype) {
      case MXFP4_DT_F32: MX_DQ_WIDE(MXFP4_DT_F32); break;
      case MXFP4_DT_BF16: MX_DQ_WIDE(MXFP4_DT_BF16); break;
      default: MX_DQ_WIDE(MXFP4_DT_F16); break;
    }
#undef MX_DQ_WIDE
    return launch_status("dequant launch");
  }
  const int64_t want = rows * ((k / 8 + 255) / 256);  // workgroup steps
  const int grid = (int)(want < 16384 ? want : 16384);
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
