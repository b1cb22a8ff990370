// FP32 compute path of the routed / dense W4A16 GEMM (C in FP32).
//
// soft:405-407 lets C, and with it the compute dtype, be FP32: the reference
// then widens A to FP32, dequantizes B to FP32 and runs an FP32 GEMM
// (soft:487-494).  Every E2M1 x 2^(s-127) weight is exact in bf16 (two
// significant bits, FP32's exponent range), so the decode goes through the
// bf16 converter and widens exactly; A (FP32, bf16 or fp16) is widened
// exactly.  The products then run on gfx950's FP32 MFMA
// (v_mfma_f32_16x16x4_f32), FP32 accumulation, one scaling step:
// C = (acc * a_scale * b_scale[e]) [* route weight].
//
// Tile BM x 128 (BM = 16, 32 or 64: routed tiles must not straddle an
// expert block of block_m rows), 4 waves side by side on columns, each wave
// all BM rows x 32 columns (BM/16 x 2 MFMA blocks); K in 32-deep steps
// staged in LDS as FP32 (rows padded to 33 floats: the column-wise fragment
// reads of 16 rows fall on 16 different banks).  MFMA operand layout
// (16x16x4): lane l supplies row / column l % 16 at k = l / 16; the result
// lane l holds rows 4 * (l / 16) + 0..3 of column l % 16.
#include "gemm.h"

namespace mx {
namespace {

constexpr int kF32BN = 128;
constexpr int kF32BK = 32;
constexpr int kF32LD = kF32BK + 1;

template <typename TA, int BM>
__global__ __launch_bounds__(256) void f32_tiled(GemmArgs g, int nbn) {
  constexpr int MB = BM / 16;  // MFMA row blocks per wave
  __shared__ float sA[BM * kF32LD];
  __shared__ float sB[kF32BN * kF32LD];
  __shared__ int64_t s_arow[BM], s_orow[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int bm = (int)(blockIdx.x / nbn), bn = (int)(blockIdx.x % nbn);
  const int64_t pos0 = (int64_t)bm * BM;
  if (pos0 >= rows_in_use(g)) return;  // past the padded rows in use
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = bn * kF32BN;

  if (tid < BM) {
    const RowInfo r = row_info(g, pos0 + tid);
    s_arow[tid] = r.valid ? r.a_row : -1;
    s_orow[tid] = r.valid ? r.out_row : -1;
  }
  __syncthreads();
  float* const c = static_cast<float*>(g.c);
  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    for (int idx = tid; idx < BM * kF32BN; idx += 256) {
      const int64_t orow = s_orow[idx / kF32BN];
      const int col = ncol0 + idx % kF32BN;
      if (orow >= 0 && col < g.n) c[orow * g.ldc + col] = 0.f;
    }
    return;
  }

  const TA* const a = static_cast<const TA*>(g.a);
  // B: thread t stages 16 K values of weight row t / 2 (bytes 8 * (t & 1)
  // .. +7 of the row's 16-byte K step); rows past N stage zeros
  const int brow = tid >> 1, bhalf = tid & 1;
  const int64_t wrow = (int64_t)ncol0 + brow;
  const bool b_ok = wrow < g.n;
  const uint8_t* const bp = g.b + expert * g.b_e + (b_ok ? wrow : 0) * g.b_n + bhalf * 8;
  const uint8_t* const sp = g.bs + expert * g.bs_e + (b_ok ? wrow : 0) * g.bs_n;

  f32x4 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < g.k; k0 += kF32BK) {
    // A: BM rows x 32 K as chunks of 4 values
    for (int ch = tid; ch < BM * (kF32BK / 4); ch += 256) {
      const int row = ch / (kF32BK / 4), kk = (ch % (kF32BK / 4)) * 4;
      const int64_t ar = s_arow[row];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sA[row * kF32LD + kk + j] = ar >= 0 ? (float)a[ar * g.lda + k0 + kk + j] : 0.f;
    }
    {
      float w[16];
      if (b_ok) {
        const float sc = e8m0_scale(sp[k0 >> 5]);
        const uint32_t* p = reinterpret_cast<const uint32_t*>(bp + (k0 >> 1));
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const bf16x8 v = Decode<__bf16>::run(p[d], sc);
#pragma unroll
          for (int j = 0; j < 8; ++j) w[d * 8 + j] = (float)v[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) w[j] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) sB[brow * kF32LD + bhalf * 16 + j] = w[j];
    }
    __syncthreads();
#pragma unroll
    for (int k4 = 0; k4 < kF32BK / 4; ++k4) {
      const int kk = k4 * 4 + (lane >> 4);
      float af[MB], bf[2];
#pragma unroll
      for (int i = 0; i < MB; ++i) af[i] = sA[(i * 16 + (lane & 15)) * kF32LD + kk];
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = sB[(wave * 32 + j * 16 + (lane & 15)) * kF32LD + kk];
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  const float alpha = scalar_alpha(g, expert);
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t orow = s_orow[i * 16 + (lane >> 4) * 4 + r];
      if (orow < 0) continue;
      const float rw = g.route_w ? g.route_w[orow] : 1.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = ncol0 + wave * 32 + j * 16 + (lane & 15);
        if (col >= g.n) continue;
        float o = acc[i][j][r] * alpha;
        if (g.route_w) o *= rw;
        c[orow * g.ldc + col] = o;
      }
    }
}

template <typename TA>
int launch_f32_typed(const GemmArgs& g, int bm, int64_t nwg, int nbn, hipStream_t st) {
  switch (bm) {
    case 64: f32_tiled<TA, 64><<<(unsigned)nwg, 256, 0, st>>>(g, nbn); break;
    case 32: f32_tiled<TA, 32><<<(unsigned)nwg, 256, 0, st>>>(g, nbn); break;
    default: f32_tiled<TA, 16><<<(unsigned)nwg, 256, 0, st>>>(g, nbn); break;
  }
  return launch_status("f32 gemm launch");
}

}  // namespace

int launch_f32_reference(const GemmArgs& g, int a_dtype, hipStream_t st) {
  if (g.k % kF32BK != 0) {
    set_error("f32 gemm: K must be a multiple of %d", kF32BK);
    return MXFP4_ERR_VALUE;
  }
  // tile rows: as many as fit an expert block (routed) and the rows in use
  int bm = 64;
  if (g.sorted_ids) {
    while (bm > 16 && g.block_m % bm != 0) bm /= 2;
  } else {
    while (bm > 16 && g.m <= bm / 2) bm /= 2;
  }
  const int nbn = (g.n + kF32BN - 1) / kF32BN;
  const int64_t nbm = (g.m + bm - 1) / bm;
  const int64_t nwg = nbm * nbn;
  if (nwg <= 0 || nwg > 0x7FFFFFFF) {
    set_error("f32 gemm: bad grid");
    return MXFP4_ERR_VALUE;
  }
  switch (a_dtype) {
    case MXFP4_DT_F32: return launch_f32_typed<float>(g, bm, nwg, nbn, st);
    case MXFP4_DT_BF16: return launch_f32_typed<__bf16>(g, bm, nwg, nbn, st);
    case MXFP4_DT_F16: return launch_f32_typed<_Float16>(g, bm, nwg, nbn, st);
    default:
      set_error("f32 gemm: unsupported activation dtype %d", a_dtype);
      return MXFP4_ERR_TYPE;
  }
}

}  // namespace mx
