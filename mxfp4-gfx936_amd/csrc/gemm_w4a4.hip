// W4A4 GEMM: packed MXFP4 activations x packed MXFP4 weights on gfx950's
// block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4, both operands E2M1,
// one E8M0 scale per lane per 32 K).  This is the packed-A semantics of
// aiter:206-214 + 329-338 (tl.dot_scaled with a_mx/b_mx) and of the safe
// path's `dequant(A) @ dequant(B)^T` (soft:468-471, 487-490): every E2M1 x
// E2M1 product times its two power-of-two scales is exact, accumulation is
// FP32, and scales/route weights apply to the FP32 accumulator.
//
// Lane layout of the 16x16x128 MFMA (verified on the device): lane l
// supplies row/column l % 16 and the E8M0 byte of K block l/16 (K =
// (l/16)*32 .. +32) in byte 0 of its scale operand.  An E2M1 operand holds
// that block as 16 bytes (low nibble first) in its first four dwords; an
// FP8 operand (E4M3 / E5M2: the activation formats of aiter:11-20) holds K =
// (l/16)*16 .. +16 in dwords 0-3 and K = 64 + (l/16)*16 .. +16 in dwords 4-7
// (a one-wave probe with one-hot E2M1 rows and distinct FP8 bytes read the
// mapping off the products), the scale still that of block l/16.
//
// Tiling: 256-thread workgroups, 4 waves as WGM x WGN, wave tile FM x FN
// MFMA blocks; each 128-deep K stage stages A and B tiles (64 B per packed
// row, 128 B per FP8 row) and their scale bytes in LDS, double buffered.
// AF: MFMA format of A (4 = E2M1, 0 = E4M3, 1 = E5M2).
#include "gemm.h"

namespace mx {
namespace {

template <typename TO, int FM, int FN, int WGM, int WGN, int AF>
__global__ __launch_bounds__(256) void w4a4_tiled(GemmArgs g) {
  constexpr int BM = WGM * FM * 16;
  constexpr int BN = WGN * FN * 16;
  constexpr int BK = 128;
  constexpr int LD = 80;  // bytes per LDS row: 64 data + 16 pad (conflict-free b128 reads)
  constexpr bool F8 = AF != 4;
  constexpr int ACPR = F8 ? 8 : 4;  // 16-byte A chunks per row and stage
  constexpr int LDA = F8 ? 144 : LD;
  constexpr int A_CHUNKS = BM * ACPR;  // 16-byte chunks per stage
  constexpr int B_CHUNKS = BN * 4;
  static_assert(WGM * WGN == 4, "4 waves");
  static_assert(BN == 128, "tile config");

  __shared__ __attribute__((aligned(16))) uint8_t As[2][BM][LDA];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN][LD];
  __shared__ uint8_t Sa[2][BM][4];
  __shared__ uint8_t Sb[2][BN][4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int c16 = lane & 15;
  const int grp = lane >> 4;

  const int64_t pos0 = (int64_t)blockIdx.y * BM;
  if (pos0 >= rows_in_use(g)) return;
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = blockIdx.x * BN;

  if (expert < 0) {
    for (int idx = tid; idx < BM * BN; idx += 256) {
      const int r = idx / BN, cc = idx % BN;
      const RowInfo ri = row_info(g, pos0 + r);
      if (ri.valid && ncol0 + cc < g.n)
        static_cast<TO*>(g.c)[ri.out_row * g.ldc + ncol0 + cc] = from_f32<TO>(0.f);
    }
    return;
  }

  const uint8_t* a_src[(A_CHUNKS + 255) / 256];
  const uint8_t* as_src[(A_CHUNKS + 255) / 256];
  constexpr int A_PER = (A_CHUNKS + 255) / 256;
  constexpr int B_PER = (B_CHUNKS + 255) / 256;
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + i * 256;
    a_src[i] = nullptr;
    as_src[i] = nullptr;
    if (c < A_CHUNKS) {
      const RowInfo ri = row_info(g, pos0 + c / ACPR);
      if (ri.valid) {
        a_src[i] = static_cast<const uint8_t*>(g.a) + ri.a_row * g.lda;
        as_src[i] = g.a_mx ? g.a_mx + ri.a_row * g.lda_mx : nullptr;  // FP8: null = scale 1
      }
    }
  }
  const uint8_t* b_src[B_PER];
  const uint8_t* bs_src[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = tid + i * 256;
    const int row = ncol0 + (c >> 2);
    const bool ok = (c < B_CHUNKS) && row < g.n;
    b_src[i] = ok ? g.b + expert * g.b_e + (int64_t)row * g.b_n : nullptr;
    bs_src[i] = ok ? g.bs + expert * g.bs_e + (int64_t)row * g.bs_n : nullptr;
  }

  i32x4 areg[A_PER], breg[B_PER];
  uint8_t asreg[A_PER], bsreg[B_PER];

  auto load_global = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + i * 256;
      // packed: chunk c % 4 is 32-block c % 4; FP8: chunk c % 8 holds K
      // (c % 8) * 16 .. +16 of 32-block (c % 8) / 2
      const int k = F8 ? kt * BK + (c % ACPR) * 16 : kt * BK + (c & 3) * 32;
      const bool ok = a_src[i] && (k & ~31) < g.k;
      areg[i] = ok ? *reinterpret_cast<const i32x4*>(a_src[i] + (F8 ? k : (k >> 1)))
                   : i32x4{0, 0, 0, 0};
      asreg[i] = (ok && as_src[i]) ? as_src[i][k >> 5] : (uint8_t)127;
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + i * 256;
      const int k = kt * BK + (c & 3) * 32;
      const bool ok = b_src[i] && k < g.k;
      breg[i] = ok ? *reinterpret_cast<const i32x4*>(b_src[i] + (k >> 1)) : i32x4{0, 0, 0, 0};
      bsreg[i] = ok ? bs_src[i][k >> 5] : (uint8_t)127;
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + i * 256;
      if (c < A_CHUNKS) {
        *reinterpret_cast<i32x4*>(&As[buf][c / ACPR][(c % ACPR) * 16]) = areg[i];
        if (!F8 || (c & 1) == 0) Sa[buf][c / ACPR][F8 ? (c % ACPR) / 2 : (c & 3)] = asreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<i32x4*>(&Bs[buf][c >> 2][(c & 3) * 16]) = breg[i];
      Sb[buf][c >> 2][c & 3] = bsreg[i];
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (g.k + BK - 1) / BK;
  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_global(kt + 1);
    i32x8 af[FM];
    int asc[FM];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int r = wm * FM * 16 + fm * 16 + c16;
      const i32x4 v = *reinterpret_cast<const i32x4*>(&As[buf][r][grp * 16]);
      if constexpr (F8) {
        const i32x4 w = *reinterpret_cast<const i32x4*>(&As[buf][r][(4 + grp) * 16]);
        af[fm] = i32x8{v[0], v[1], v[2], v[3], w[0], w[1], w[2], w[3]};
      } else {
        af[fm] = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
      }
      asc[fm] = Sa[buf][r][grp];
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int r = wn * FN * 16 + fn * 16 + c16;
      const i32x4 v = *reinterpret_cast<const i32x4*>(&Bs[buf][r][grp * 16]);
      const i32x8 bf = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
      const int bsc = Sb[buf][r][grp];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        acc[fm][fn] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            af[fm], bf, acc[fm][fn], AF, 4, 0, asc[fm], 0, bsc);
    }
    if (kt + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  float alpha = scalar_alpha(g, expert);
  if (g.ref_round) {
    ref_pass<TO>(g, expert, acc);
    alpha = 1.0f;
  }
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const RowInfo r = row_info(g, pos0 + wm * FM * 16 + fm * 16 + grp * 4 + i);
      if (!r.valid) continue;
      const float rw = g.route_w ? g.route_w[r.out_row] : 1.0f;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = ncol0 + wn * FN * 16 + fn * 16 + c16;
        if (col < g.n) {
          float o = acc[fm][fn][i] * alpha;
          if (g.route_w) o *= rw;
          static_cast<TO*>(g.c)[r.out_row * g.ldc + col] = from_f32<TO>(o);
        }
      }
    }
  }
}

template <typename TO, int AF>
int launch_w4a4_typed(const GemmArgs& g, hipStream_t st) {
  const int64_t cap = g.m;
  const bool routed = g.sorted_ids != nullptr;
  const int64_t ntiles = (g.n + 127) / 128;
  int bm;
  if (routed && g.block_m % 32 != 0) {
    bm = 16;
  } else {
    bm = 32;
    const int cands[2] = {128, 64};
    for (int i = 0; i < 2; ++i) {
      const int c = cands[i];
      if (routed && (g.block_m % c) != 0) continue;
      if (((cap + c - 1) / c) * ntiles >= 512) {
        bm = c;
        break;
      }
    }
    if (!routed && cap <= 16) bm = 16;
  }
  const int64_t gy = (cap + bm - 1) / bm;
  if (gy > 65535) {
    set_error("w4a4: too many row tiles (%lld)", (long long)gy);
    return MXFP4_ERR_VALUE;
  }
  dim3 grid((unsigned)ntiles, (unsigned)(gy > 0 ? gy : 1));
  switch (bm) {
    case 128: w4a4_tiled<TO, 4, 4, 2, 2, AF><<<grid, 256, 0, st>>>(g); break;
    case 64: w4a4_tiled<TO, 2, 4, 2, 2, AF><<<grid, 256, 0, st>>>(g); break;
    case 32: w4a4_tiled<TO, 1, 4, 2, 2, AF><<<grid, 256, 0, st>>>(g); break;
    default: w4a4_tiled<TO, 1, 2, 1, 4, AF><<<grid, 256, 0, st>>>(g); break;
  }
  return launch_status("w4a4 launch");
}

template <int AF>
int launch_tiled_out(const GemmArgs& g, int out_dtype, hipStream_t st) {
  switch (out_dtype) {
    case MXFP4_DT_BF16: return launch_w4a4_typed<__bf16, AF>(g, st);
    case MXFP4_DT_F16: return launch_w4a4_typed<_Float16, AF>(g, st);
    default: return launch_w4a4_typed<float, AF>(g, st);
  }
}

}  // namespace

int launch_w4a4(const GemmArgs& g, int out_dtype, hipStream_t st) {
  if (out_dtype == MXFP4_DT_BF16 || out_dtype == MXFP4_DT_F16 || out_dtype == MXFP4_DT_F32) {
    const int cfg = p4_supported(g) ? p4_choose(g, out_dtype) : -1;
    if (cfg >= 0) return launch_w4a4_pf(g, out_dtype, cfg, st);
  }
  if (out_dtype != MXFP4_DT_BF16 && out_dtype != MXFP4_DT_F16 && out_dtype != MXFP4_DT_F32) {
    set_error("w4a4: unsupported output dtype %d", out_dtype);
    return MXFP4_ERR_TYPE;
  }
  switch (g.a_fp8) {
    case 1: return launch_tiled_out<0>(g, out_dtype, st);
    case 2: return launch_tiled_out<1>(g, out_dtype, st);
    default: return launch_tiled_out<4>(g, out_dtype, st);
  }
}

}  // namespace mx
