// W4A4 GEMM, direct-to-LDS pipeline (gfx950): packed MXFP4 activations x
// packed MXFP4 weights on the block-scaled MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4, both operands E2M1).  Same semantics
// as w4a4_tiled (aiter:206-214 + 329-338; soft:468-471, 487-490): every
// E2M1 x E2M1 product times its two power-of-two scales is exact, FP32
// accumulation, scales / route weights on the FP32 accumulator, one
// rounding to the output type.
//
// Tile BM x BN (activation rows x weight rows), WGM x WGN waves of FM x FN
// MFMA blocks, K in 128-deep stages.  Feeding FP4 MFMAs takes 4x the bytes
// per FLOP of BF16 ones, so the tile is as large as the registers allow
// (256 x 256 with 8 waves of 128 x 64, 3 stages) and everything moves
// global -> LDS with `buffer_load_dwordx4 ... lds` (16 bytes per lane at LDS
// base + 16 x lane; out-of-range offsets read zero, so padding rows and
// partial tiles need no branches):
//
// * A and B stages hold 64-byte rows (128 E2M1 codes), written by 1 KB
//   wave-loads of 16 rows; the MFMA fragment of lane l (row l % 16, K
//   (l/16)*32 .. +32) is the 16-byte chunk l/16 of its row, so a wave reads
//   one contiguous KB per fragment.
// * The four E8M0 bytes of a row's stage (one per 32-block) are one dword,
//   staged by 4-byte-per-lane wave-loads; lane l reads byte l/16 of its
//   row's dword into byte 0 of its scale operand.
// * The MFMA takes the weights as its A operand and the activations as its
//   B operand, so a lane owns 4 consecutive output columns of one row; the
//   epilogue stages the finished tile in LDS and writes 16-byte chunks.
//
// Requirements (else the register-staged w4a4_tiled runs): K % 128 == 0,
// 16-byte aligned A / B rows and scale rows 4-byte aligned, operands below
// 2 GiB.
#include "gemm.h"

namespace mx {
namespace {

template <int WGM, int WGN, int FM, int FN, int STAGES>
struct P4Shape {
  static constexpr int NW = WGM * WGN;
  static constexpr int NT = 64 * NW;
  static constexpr int BM = WGM * FM * 16;
  static constexpr int BN = WGN * FN * 16;
  static constexpr int A_STAGE = BM * 64;
  static constexpr int B_STAGE = BN * 64;
  static constexpr int A_TOT = BM / 16;  // 1 KB wave-loads per stage
  static constexpr int B_TOT = BN / 16;
  static constexpr int SA_TOT = (BM + 63) / 64;  // 256-byte scale wave-loads
  static constexpr int SB_TOT = (BN + 63) / 64;
  static constexpr int SA_STAGE = SA_TOT * 256;
  static constexpr int SB_STAGE = SB_TOT * 256;
  static constexpr int A_PER = (A_TOT + NW - 1) / NW;
  static constexpr int B_PER = (B_TOT + NW - 1) / NW;
  static constexpr int S_PER = (SA_TOT + SB_TOT + NW - 1) / NW;
  static constexpr int STAGE = A_STAGE + B_STAGE + SA_STAGE + SB_STAGE;
  static constexpr int PIPE = STAGES * STAGE;
};

template <typename TO>
__device__ __forceinline__ void store4(uint8_t* p, const float* o) {
  if constexpr (sizeof(TO) == 4) {
    *reinterpret_cast<f32x4*>(p) = f32x4{o[0], o[1], o[2], o[3]};
  } else {
    const TO a = from_f32<TO>(o[0]), b = from_f32<TO>(o[1]), c = from_f32<TO>(o[2]),
             d = from_f32<TO>(o[3]);
    const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, a) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
    const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, c) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, d) << 16);
    *reinterpret_cast<uint2*>(p) = uint2{lo, hi};
  }
}

template <typename TO, int WGM, int WGN, int FM, int FN, int STAGES, int MINB>
__global__ __launch_bounds__(64 * WGM * WGN, MINB) void w4a4_pf(GemmArgs g, int nbm, int nbn) {
  typedef P4Shape<WGM, WGN, FM, FN, STAGES> S;
  constexpr int BM = S::BM, BN = S::BN, NT = S::NT;
  constexpr int C_LD = BN * (int)sizeof(TO) + 16;  // bytes per staged output row
  constexpr int EPI_PASSES = BM * C_LD <= S::PIPE ? 1 : WGM;
  constexpr int EPI_ROWS = BM / EPI_PASSES;
  constexpr int SMEM = S::PIPE > EPI_ROWS * C_LD ? S::PIPE : EPI_ROWS * C_LD;
  static_assert(STAGES >= 2 && STAGES <= 4, "2 to 4 stages");
  static_assert(STAGES == 2 || (S::A_TOT % S::NW == 0 && S::B_TOT % S::NW == 0 &&
                                (S::SA_TOT + S::SB_TOT) % S::NW == 0),
                "deeper pipelines count the same loads on every wave");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the per-wave load choices and LDS addresses
  // (M0) then need no lane-to-scalar moves or exec masking
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int c16 = lane & 15;
  const int grp = lane >> 4;

  int bm, bn;
  if (!tile_of(g, BM, nbm, nbn, bm, bn, blockIdx.x, gridDim.x)) return;
  const int64_t pos0 = (int64_t)bm * BM;
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = bn * BN;

  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    for (int idx = tid; idx < BM * BN; idx += NT) {
      const int r = idx / BN, cc = idx % BN;
      const RowInfo ri = row_info(g, pos0 + r);
      if (ri.valid && ncol0 + cc < g.n)
        static_cast<TO*>(g.c)[ri.out_row * g.ldc + ncol0 + cc] = from_f32<TO>(0.f);
    }
    return;
  }

  const i32x4 rA = make_rsrc(g.a, (uint32_t)(g.a_rows * g.lda));
  const i32x4 rSA = make_rsrc(g.a_mx, (uint32_t)(g.a_rows * g.lda_mx));
  const i32x4 rB = make_rsrc(g.b + expert * g.b_e, (uint32_t)((int64_t)g.n * g.b_n));
  const i32x4 rSB = make_rsrc(g.bs + expert * g.bs_e, (uint32_t)((int64_t)g.n * g.bs_n));

  // per-lane offsets for stage 0 (stage kt adds kt*64 / kt*4 as the scalar
  // offset); wave-load q of a stage is issued by wave q % NW
  uint32_t a_off[S::A_PER];
#pragma unroll
  for (int j = 0; j < S::A_PER; ++j) {
    const int q = j * S::NW + wave;
    const int row = q * 16 + (lane >> 2);
    a_off[j] = kOOB;
    if (q < S::A_TOT) {
      const RowInfo ri = row_info(g, pos0 + row);
      if (ri.valid) a_off[j] = (uint32_t)(ri.a_row * g.lda) + (lane & 3) * 16;
    }
  }
  uint32_t b_off[S::B_PER];
#pragma unroll
  for (int j = 0; j < S::B_PER; ++j) {
    const int q = j * S::NW + wave;
    const int row = ncol0 + q * 16 + (lane >> 2);
    b_off[j] = (q < S::B_TOT && row < g.n) ? (uint32_t)(row * g.b_n) + (lane & 3) * 16 : kOOB;
  }
  // scale wave-loads (64 rows x 4 bytes): q < SA_TOT are A rows q*64 ..,
  // the rest B rows; dealt round-robin over the waves like the tiles
  uint32_t s_off[S::S_PER];
#pragma unroll
  for (int j = 0; j < S::S_PER; ++j) {
    const int q = j * S::NW + wave;
    s_off[j] = kOOB;
    if (q < S::SA_TOT) {
      const int row = q * 64 + lane;
      if (row < BM) {
        const RowInfo ri = row_info(g, pos0 + row);
        if (ri.valid) s_off[j] = (uint32_t)(ri.a_row * g.lda_mx);
      }
    } else if (q < S::SA_TOT + S::SB_TOT) {
      const int row = (q - S::SA_TOT) * 64 + lane;
      if (row < BN && ncol0 + row < g.n) s_off[j] = (uint32_t)((ncol0 + row) * g.bs_n);
    }
  }

  const int nk = g.k / 128;
  auto issue = [&](int kt) {
    uint8_t* base = smem + (kt % STAGES) * S::STAGE;
#pragma unroll
    for (int j = 0; j < S::A_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::A_TOT % S::NW == 0 || q < S::A_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rA, lds_ptr(base + q * 1024), 16, (int)a_off[j], kt * 64,
                                        0, 0);
    }
#pragma unroll
    for (int j = 0; j < S::B_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::B_TOT % S::NW == 0 || q < S::B_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rB, lds_ptr(base + S::A_STAGE + q * 1024), 16,
                                        (int)b_off[j], kt * 64, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < S::S_PER; ++j) {
      const int q = j * S::NW + wave;
      // A and B scale slots are contiguous: slot q at base + A + B + q*256
      if (q < S::SA_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rSA, lds_ptr(base + S::A_STAGE + S::B_STAGE + q * 256), 4,
                                        (int)s_off[j], kt * 4, 0, 0);
      else if (q < S::SA_TOT + S::SB_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rSB, lds_ptr(base + S::A_STAGE + S::B_STAGE + q * 256), 4,
                                        (int)s_off[j], kt * 4, 0, 0);
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // lane reads: activation fragment fm = rows wm*FM*16 + fm*16 + c16, chunk
  // grp; weight fragment fn likewise; scale bytes grp of those rows
  const int a_rd = (wm * FM * 16 + c16) * 64 + grp * 16;
  const int b_rd = (wn * FN * 16 + c16) * 64 + grp * 16;
  const int sa_rd = (wm * FM * 16 + c16) * 4 + grp;
  const int sb_rd = (wn * FN * 16 + c16) * 4 + grp;

#pragma unroll
  // the stage waits count loads per stage in issue order: a compiler fence
  // after each prologue stage keeps stage s + 1's loads behind stage s's
  for (int s = 0; s < STAGES - 1; ++s) {
    if (s < nk) issue(s);
    asm volatile("" ::: "memory");
  }
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt has landed once at most the later stages' loads of this wave
    // are outstanding (PER_STAGE each); the barrier publishes it and retires
    // the reads of the buffer issue() refills
    constexpr int PER_STAGE = S::A_PER + S::B_PER + S::S_PER;
    const int later = (nk - 1 - kt) < (STAGES - 2) ? (nk - 1 - kt) : (STAGES - 2);
    if (STAGES >= 4 && later >= 2) wait_vmcnt<2 * PER_STAGE>();
    else if (STAGES >= 3 && later >= 1) wait_vmcnt<PER_STAGE>();
    else wait_vmcnt<0>();
    barrier_only();
    if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
    const uint8_t* base = smem + (kt % STAGES) * S::STAGE;
    const uint8_t* As = base;
    const uint8_t* Bs = base + S::A_STAGE;
    const uint8_t* Sa = base + S::A_STAGE + S::B_STAGE;
    const uint8_t* Sb = Sa + S::SA_STAGE;
    i32x8 af[FM];
    int asc[FM];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const i32x4 v = *reinterpret_cast<const i32x4*>(As + a_rd + fm * 16 * 64);
      af[fm] = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
      asc[fm] = Sa[sa_rd + fm * 16 * 4];
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const i32x4 v = *reinterpret_cast<const i32x4*>(Bs + b_rd + fn * 16 * 64);
      const i32x8 bf = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
      const int bsc = Sb[sb_rd + fn * 16 * 4];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        acc[fm][fn] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af[fm], acc[fm][fn], 4,
                                                                       4, 0, bsc, 0, asc[fm]);
    }
  }

  // ---- epilogue: lane owns row wm*FM*16 + fm*16 + c16 and columns
  // wn*FN*16 + fn*16 + grp*4 .. +3; stage rows in LDS, write 16-byte chunks
  barrier_only();  // every wave is done reading the stage buffers
  const float alpha = scalar_alpha(g, expert);
#pragma unroll
  for (int pass = 0; pass < EPI_PASSES; ++pass) {
    if (EPI_PASSES == 1 || wm == pass) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int trow = wm * FM * 16 + fm * 16 + c16;
        float rw = 1.0f;
        if (g.route_w) {
          const RowInfo r = row_info(g, pos0 + trow);
          rw = r.valid ? g.route_w[r.out_row] : 0.f;
        }
        uint8_t* crow = smem + (trow - pass * EPI_ROWS) * C_LD;
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int tcol = wn * FN * 16 + fn * 16 + grp * 4;
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = acc[fm][fn][i] * alpha * rw;
          store4<TO>(crow + tcol * (int)sizeof(TO), o);
        }
      }
    }
    __syncthreads();
    constexpr int EPC = 16 / (int)sizeof(TO);  // elements per 16-byte chunk
    constexpr int CHUNKS = BN / EPC;
    for (int idx = tid; idx < EPI_ROWS * CHUNKS; idx += NT) {
      const int prow = idx / CHUNKS, ch = idx % CHUNKS;
      const int trow = pass * EPI_ROWS + prow;
      const int col = ncol0 + ch * EPC;
      if (col >= g.n) continue;
      const RowInfo r = row_info(g, pos0 + trow);
      if (!r.valid) continue;
      const uint8_t* src = smem + prow * C_LD + ch * 16;
      TO* dst = static_cast<TO*>(g.c) + r.out_row * g.ldc + col;
      if (col + EPC <= g.n && (g.ldc % EPC) == 0) {
        *reinterpret_cast<i32x4*>(dst) = *reinterpret_cast<const i32x4*>(src);
      } else {
        const TO* s16 = reinterpret_cast<const TO*>(src);
        for (int i = 0; i < EPC && col + i < g.n; ++i) dst[i] = s16[i];
      }
    }
    if (EPI_PASSES > 1 && pass + 1 < EPI_PASSES) __syncthreads();
  }
}

template <typename TO, int WGM, int WGN, int FM, int FN, int STAGES, int MINB>
int launch_cfg(const GemmArgs& g, hipStream_t st) {
  typedef P4Shape<WGM, WGN, FM, FN, STAGES> S;
  const int nbn = (g.n + S::BN - 1) / S::BN;
  int64_t nbm = (g.m + S::BM - 1) / S::BM;
  if (g.sorted_ids) nbm = (nbm + 7) / 8 * 8;  // every XCD covers 1/8 of the capacity (tile_of)
  const int64_t nwg = nbm * nbn;
  if (nwg <= 0 || nwg > 0x7FFFFFFF) {
    set_error("w4a4 prefill: bad grid");
    return MXFP4_ERR_VALUE;
  }
  w4a4_pf<TO, WGM, WGN, FM, FN, STAGES, MINB><<<(unsigned)nwg, S::NT, 0, st>>>(g, (int)nbm, nbn);
  return launch_status("w4a4 prefill launch");
}

template <typename TO>
int launch_typed(const GemmArgs& g, int cfg, hipStream_t st) {
  // FP32 output stages 4-byte rows: its epilogue fits LDS only up to 128 x 128
  if constexpr (sizeof(TO) == 4) {
    if (cfg == P4_64x128) return launch_cfg<TO, 1, 4, 4, 2, 2, 2>(g, st);
    return launch_cfg<TO, 1, 4, 8, 2, 2, 2>(g, st);
  } else {
    // Measured (8192 x 4096 x 4096, bf16 out): 2 x 4 waves of 128 x 64 with
    // 3 stages ~2.9-3.0 PFLOP/s, 2 stages ~2.6-2.75, 4 stages no better;
    // 2 x 2 waves of 128 x 128 (one wave per SIMD) ~2.3-2.6; 16 waves of
    // 128 x 64 (256 x 512) does not fit the register file.
    switch (cfg) {
      case P4_256x256: return launch_cfg<TO, 2, 4, 8, 4, 3, 1>(g, st);
      case P4_128x128: return launch_cfg<TO, 1, 4, 8, 2, 2, 2>(g, st);
      default: return launch_cfg<TO, 1, 4, 4, 2, 2, 2>(g, st);  // P4_64x128
    }
  }
}

}  // namespace

bool p4_supported(const GemmArgs& g) {
  if (g.k % 128 != 0 || g.k <= 0 || g.a_rows <= 0) return false;
  if ((reinterpret_cast<uintptr_t>(g.a) & 15) || (reinterpret_cast<uintptr_t>(g.b) & 15) ||
      (reinterpret_cast<uintptr_t>(g.a_mx) & 3) || (reinterpret_cast<uintptr_t>(g.bs) & 3) ||
      (reinterpret_cast<uintptr_t>(g.c) & 15) || (g.lda & 15) || (g.lda_mx & 3))
    return false;
  if (g.a_rows * g.lda >= (int64_t)0x7FFFFFFF) return false;
  if ((int64_t)g.n * g.b_n >= (int64_t)0x7FFFFFFF) return false;
  return true;
}

int p4_choose(const GemmArgs& g, int out_dtype) {
  const bool routed = g.sorted_ids != nullptr;
  auto allowed = [&](int bm) { return !routed || g.block_m % bm == 0; };
  auto tiles = [&](int bm, int bn) { return ((g.m + bm - 1) / bm) * (int64_t)((g.n + bn - 1) / bn); };
  // FP32 output stages 4-byte rows: keep its epilogue within 128 x 128.
  // 256 x 256 needs a tile for every CU (steady clocks, bf16 out: 2.99 vs
  // 2.06 PFLOP/s at M = 8192 K = N = 4096 with 512 tiles; with 160 tiles,
  // M = 2048 K = 2048 N = 5120, 128 x 128 wins 1.69 vs 1.59).
  const bool wide = out_dtype != MXFP4_DT_F32;
  if (wide && allowed(256) && tiles(256, 256) >= 256) return P4_256x256;
  if (allowed(128) && tiles(128, 128) >= 128) return P4_128x128;
  if (allowed(64)) return P4_64x128;
  return -1;
}

int launch_w4a4_pf(const GemmArgs& g, int out_dtype, int cfg, hipStream_t st) {
  switch (out_dtype) {
    case MXFP4_DT_BF16: return launch_typed<__bf16>(g, cfg, st);
    case MXFP4_DT_F16: return launch_typed<_Float16>(g, cfg, st);
    default: return launch_typed<float>(g, cfg, st);
  }
}

}  // namespace mx
