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
// all BM rows x 32 columns (BM/16 x 2 MFMA blocks).  K runs in 32-deep
// stages through two LDS buffers.  During stage s the global loads of
// stage s + 2 go out (16-byte activation chunks of the gathered rows; 8
// packed weight bytes and the stage's E8M0 byte per thread, into one of two
// register sets), the MFMAs of stage s run, and stage s + 1 (loaded during
// stage s - 1) lands in the other buffer (activations widened to FP32,
// weights decoded to FP32); one barrier per stage.  LDS rows are 36 floats (144
// bytes), so the 16-byte fragment reads of 8 consecutive rows fall in 8
// different bank groups.
//
// MFMA operand layout (16x16x4): lane l supplies row / column l % 16 at k =
// l / 16; the result lane l holds rows 4 * (l / 16) + 0..3 of column l % 16.
// Within a 16-deep K chunk, lane group q = l / 16 supplies K = 4q + j to
// MFMA j (j = 0..3) for both operands, so one 16-byte read gives a lane its
// values for four MFMAs; the four MFMAs together sum every K of the chunk
// once (an FP32 sum in another order than K order).
#include "gemm.h"

namespace mx {
namespace {

constexpr int kF32BN = 128;
constexpr int kF32BK = 32;
constexpr int kF32LD = kF32BK + 4;

template <typename TA>
__device__ __forceinline__ void widen_store(float* dst, const i32x4 v) {
  if constexpr (sizeof(TA) == 4) {
    *reinterpret_cast<i32x4*>(dst) = v;
  } else {
    const TA* e = reinterpret_cast<const TA*>(&v);
    *reinterpret_cast<f32x4*>(dst) = f32x4{(float)e[0], (float)e[1], (float)e[2], (float)e[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{(float)e[4], (float)e[5], (float)e[6], (float)e[7]};
  }
}

template <typename TA, int BM>
__global__ __launch_bounds__(256) void f32_pipe(GemmArgs g, int nbm, int nbn) {
  constexpr int MB = BM / 16;              // MFMA row blocks per wave
  constexpr int V = 16 / (int)sizeof(TA);  // activation values per 16-byte chunk
  constexpr int CPR = kF32BK / V;          // chunks per activation row and stage
  constexpr int ACH = BM * CPR;            // activation chunks per stage
  constexpr int APT = (ACH + 255) / 256;   // ... per thread
  __shared__ __attribute__((aligned(16))) float sA[2][BM * kF32LD];
  __shared__ __attribute__((aligned(16))) float sB[2][kF32BN * kF32LD];
  __shared__ int64_t s_arow[BM], s_orow[BM];
  __shared__ int s_live;  // bit i: MFMA row block i holds a valid row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int bm, bn;
  if (!tile_of(g, BM, nbm, nbn, bm, bn, blockIdx.x, gridDim.x)) return;
  const int64_t pos0 = (int64_t)bm * BM;
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = bn * kF32BN;

  if (wave == 0) {  // BM <= 64: one lane per tile row
    bool valid = false;
    if (lane < BM) {
      const RowInfo r = row_info(g, pos0 + lane);
      valid = r.valid;
      s_arow[lane] = r.valid ? r.a_row : -1;
      s_orow[lane] = r.valid ? r.out_row : -1;
    }
    const uint64_t v = __ballot(valid);
    if (lane == 0) {
      int live = 0;
#pragma unroll
      for (int i = 0; i < MB; ++i) live |= ((v >> (16 * i)) & 0xFFFFull) ? 1 << i : 0;
      s_live = live;
    }
  }
  __syncthreads();
  // row blocks of padding only (a routed block's tail) skip their fragment
  // reads and MFMAs: the FP32 MFMA is the bound here
  const int live = __builtin_amdgcn_readfirstlane(s_live);
  float* const c = static_cast<float*>(g.c);
  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    for (int idx = tid; idx < BM * kF32BN; idx += 256) {
      const int64_t orow = s_orow[idx / kF32BN];
      const int col = ncol0 + idx % kF32BN;
      if (orow >= 0 && col < g.n) c[orow * g.ldc + col] = 0.f;
    }
    return;
  }

  // activation chunk q = tid + 256 j: row q / CPR, K q % CPR * V of the stage
  const TA* const a = static_cast<const TA*>(g.a);
  const TA* a_src[APT];
  int a_dst[APT];
#pragma unroll
  for (int j = 0; j < APT; ++j) {
    const int q = tid + 256 * j;
    const int row = q / CPR;
    const int64_t ar = (q < ACH) ? s_arow[row] : -1;
    a_src[j] = ar >= 0 ? a + ar * g.lda + (q % CPR) * V : nullptr;
    a_dst[j] = q < ACH ? row * kF32LD + (q % CPR) * V : -1;
  }
  // weights: thread t stages 16 K values of weight row t / 2 (bytes 8 * (t &
  // 1) .. +7 of the row's 16-byte stage); rows past N stage zeros
  const int brow = tid >> 1, bhalf = tid & 1;
  const int64_t wrow = (int64_t)ncol0 + brow;
  const bool b_ok = wrow < g.n;
  const uint8_t* const bp = g.b + expert * g.b_e + (b_ok ? wrow : 0) * g.b_n + bhalf * 8;
  const uint8_t* const sp = g.bs + expert * g.bs_e + (b_ok ? wrow : 0) * g.bs_n;
  const int b_dst = brow * kF32LD + bhalf * 16;

  // two register sets: stage s + 2's loads are issued while stage s + 1's
  // (issued a stage earlier) wait to be stored
  struct Regs {
    i32x4 a[APT];
    uint2 b;
    uint32_t s;
  };
  auto load = [&](Regs& r, int kt) {
    const int k0 = kt * kF32BK;
#pragma unroll
    for (int j = 0; j < APT; ++j)
      r.a[j] = a_src[j] ? *reinterpret_cast<const i32x4*>(a_src[j] + k0) : i32x4{0, 0, 0, 0};
    if (b_ok) {
      r.b = *reinterpret_cast<const uint2*>(bp + (k0 >> 1));
      r.s = sp[k0 >> 5];
    }
  };
  auto store = [&](const Regs& r, int buf) {
    const i32x4* ra = r.a;
    const uint2 rb = r.b;
    const uint32_t rs = r.s;
#pragma unroll
    for (int j = 0; j < APT; ++j)
      if (a_dst[j] >= 0) widen_store<TA>(&sA[buf][a_dst[j]], ra[j]);
    float* const db = &sB[buf][b_dst];
    if (b_ok) {
      const float sc = e8m0_scale(rs);
      const bf16x8 lo = Decode<__bf16>::run(rb.x, sc);
      const bf16x8 hi = Decode<__bf16>::run(rb.y, sc);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        *reinterpret_cast<f32x4*>(db + 4 * q) =
            f32x4{(float)lo[4 * q], (float)lo[4 * q + 1], (float)lo[4 * q + 2], (float)lo[4 * q + 3]};
        *reinterpret_cast<f32x4*>(db + 8 + 4 * q) =
            f32x4{(float)hi[4 * q], (float)hi[4 * q + 1], (float)hi[4 * q + 2], (float)hi[4 * q + 3]};
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<f32x4*>(db + 4 * q) = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  f32x4 acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = g.k / kF32BK;
  const int ar_rd = (lane & 15) * kF32LD + 4 * (lane >> 4);
  const int br_rd = (wave * 32 + (lane & 15)) * kF32LD + 4 * (lane >> 4);
  Regs r0, r1;
  load(r0, 0);
  if (nk > 1) load(r1, 1);
  store(r0, 0);
  __syncthreads();
  // stage kt: loads of stage kt + 2 go out, the MFMAs of stage kt run from
  // buffer kt & 1, stage kt + 1 (loaded during stage kt - 1) is stored into
  // the other buffer; unrolled by two so each register set is fixed
  auto step = [&](int kt, Regs& next, Regs& later) {
    const int buf = kt & 1;
    if (kt + 2 < nk) load(later, kt + 2);
    const float* const As = sA[buf];
    const float* const Bs = sB[buf];
#pragma unroll
    for (int ch = 0; ch < kF32BK / 16; ++ch) {
      f32x4 af[MB], bf[2];
#pragma unroll
      for (int i = 0; i < MB; ++i)
        if (live & (1 << i))
          af[i] = *reinterpret_cast<const f32x4*>(As + ar_rd + i * 16 * kF32LD + ch * 16);
#pragma unroll
      for (int jn = 0; jn < 2; ++jn)
        bf[jn] = *reinterpret_cast<const f32x4*>(Bs + br_rd + jn * 16 * kF32LD + ch * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          if (!(live & (1 << i))) continue;
#pragma unroll
          for (int jn = 0; jn < 2; ++jn)
            acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][j], bf[jn][j], acc[i][jn], 0,
                                                               0, 0);
        }
    }
    // buffer buf ^ 1 was last read in stage kt - 1, before the previous
    // barrier; the barrier below publishes it for stage kt + 1
    if (kt + 1 < nk) store(next, buf ^ 1);
    __syncthreads();
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, r1, r0);
    if (kt + 1 < nk) step(kt + 1, r0, r1);
  }

  float alpha = scalar_alpha(g, expert);
  if (g.ref_round) {
    ref_pass<float>(g, expert, acc);
    alpha = 1.0f;
  }
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
int launch_f32_typed(const GemmArgs& g, int bm, int64_t nbm, int nbn, hipStream_t st) {
  const int64_t nwg = nbm * nbn;
  switch (bm) {
    case 64: f32_pipe<TA, 64><<<(unsigned)nwg, 256, 0, st>>>(g, (int)nbm, nbn); break;
    case 32: f32_pipe<TA, 32><<<(unsigned)nwg, 256, 0, st>>>(g, (int)nbm, nbn); break;
    default: f32_pipe<TA, 16><<<(unsigned)nwg, 256, 0, st>>>(g, (int)nbm, nbn); break;
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
  int64_t nbm = (g.m + bm - 1) / bm;
  if (g.sorted_ids) nbm = (nbm + 7) / 8 * 8;  // every XCD covers 1/8 of the capacity (tile_of)
  const int64_t nwg = nbm * nbn;
  if (nwg <= 0 || nwg > 0x7FFFFFFF || nbm > 0x7FFFFFFF) {
    set_error("f32 gemm: bad grid");
    return MXFP4_ERR_VALUE;
  }
  switch (a_dtype) {
    case MXFP4_DT_F32: return launch_f32_typed<float>(g, bm, nbm, nbn, st);
    case MXFP4_DT_BF16: return launch_f32_typed<__bf16>(g, bm, nbm, nbn, st);
    case MXFP4_DT_F16: return launch_f32_typed<_Float16>(g, bm, nbm, nbn, st);
    default:
      set_error("f32 gemm: unsupported activation dtype %d", a_dtype);
      return MXFP4_ERR_TYPE;
  }
}

}  // namespace mx
