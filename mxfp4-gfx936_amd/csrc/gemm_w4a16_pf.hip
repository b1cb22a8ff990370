// W4A16 prefill GEMM, direct-to-LDS pipeline (gfx950).
//
// Tile BM x BN (output rows x weight rows), WGM x WGN waves, each wave FM x
// FN MFMA blocks of 16x16, K in 64-deep stages:
//
// * Staging.  A (BM x 64 bf16/fp16) and packed B (BN rows x 32 bytes) go
//   global -> LDS with `buffer_load_dwordx4 ... lds` (16 bytes per lane land
//   at LDS base + 16 * lane): no VGPR staging, no ds_write.  Out-of-range
//   buffer offsets read as zero, so invalid (padding / non-routed) rows and
//   partial N tiles cost no branches: their offset is pushed past the end of
//   the buffer.  The E8M0 bytes of 4 consecutive 32-blocks of a row (one
//   dword, 128 K) are staged the same way every other stage.  STAGES stages
//   are in flight; one barrier per stage.
// * LDS layout.  Rows are dense (A: 128 B, B: 32 B per row) with an XOR
//   swizzle of the 16-byte chunk index, applied through the global address
//   each lane loads, so the MFMA fragment reads spread over the banks.
// * Math.  Each lane decodes its B fragment (8 E2M1 codes of one weight row
//   + the row's block scale) with four v_cvt_scalef32_pk_* right before the
//   MFMA.  The MFMA takes the weights as its A operand and the activations as
//   its B operand, so a lane owns 4 consecutive output columns of one row.
// * Epilogue.  Scales / route weight / bias / SiLU*mul are applied in
//   registers, the tile is staged in LDS (reusing the stage buffers) and
//   written back as full 16-byte chunks, whole output rows per instruction.
//   EPI_PARTIAL (split K) instead stores the raw FP32 sums of one K slice;
//   splitk_reduce (below) adds the slices.
// * Order.  Workgroups are dealt round-robin over the 8 XCDs; tile_of
//   (gemm.h) gives each XCD a contiguous range of rows.
//
// Requirements (else the host falls back to the register-staged kernel):
// K % 128 == 0; activation and weight byte ranges below 2 GiB; 16-byte
// aligned A / B rows and 4-byte aligned scale rows.
#include <atomic>

#include "gemm.h"
#include "silu.h"

namespace mx {
namespace {

template <typename T>
struct V8Of;
template <>
struct V8Of<__bf16> {
  typedef bf16x8 type;
};
template <>
struct V8Of<_Float16> {
  typedef f16x8 type;
};

template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const T x = from_f32<T>(a), y = from_f32<T>(b);
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}

template <int WGM, int WGN, int FM, int FN, int STAGES, bool PRE = false, int BG = 1>
struct PfShape {
  static constexpr int NW = WGM * WGN;  // waves
  static constexpr int NT = 64 * NW;    // threads
  static constexpr int BM = WGM * FM * 16;
  static constexpr int BN = WGN * FN * 16;
  static constexpr int GRP = BN / 16;       // 16-row weight groups
  static constexpr int A_STAGE = BM * 128;  // BM rows x 64 elements x 2 bytes
  static constexpr int B_STAGE = BN * 32;   // BN rows x 64 nibbles
  static constexpr int A_TOT = BM / 8;      // 1 KB wave-loads per stage (8 rows each)
  static constexpr int B_TOT = BN / 32;     // (32 rows each)
  // Original layout in weight-line groups (BG > 1): a weight row's BG x 32
  // bytes (BG stages) in one piece, in two alternating group slots
  static constexpr int RBB = 32 * BG;              // bytes of a row per group
  static constexpr int B_GRP = BN * RBB;           // bytes per group slot
  static constexpr int B_GTOT = B_GRP / 1024;      // 1 KB wave-loads per group
  static constexpr int B_GPER = (B_GTOT + NW - 1) / NW;
  static constexpr int B_REGION = BG > 1 ? 2 * B_GRP : STAGES * B_STAGE;
  // Scales.  Original layout: the 4 E8M0 bytes of a weight row's 128 K,
  // staged every other stage (a slot per stage pair), 4-byte lanes.
  // Prepacked: the 16-bit scale operand halves of a row's two 32-blocks of
  // the stage (64 bytes per group), every stage, in 16-byte lanes, or for
  // 3+ stages in 4-byte lanes with the wave-loads rounded up to a multiple
  // of the waves (every wave then issues the same number of loads per
  // stage, which the partial vmcnt waits count on; the extra lanes read
  // past the end, i.e. zeros, into the slot's unused tail).
  static constexpr int S_LANE = (PRE && STAGES == 2) ? 16 : 4;
  static constexpr int S_BYTES = PRE ? GRP * 64 : BN * 4;
  static constexpr int S_RAW = (S_BYTES + 64 * S_LANE - 1) / (64 * S_LANE);
  static constexpr int S_TOT = (PRE && STAGES > 2) ? (S_RAW + NW - 1) / NW * NW : S_RAW;
  static constexpr int S_PER = (S_TOT + NW - 1) / NW;
  static constexpr int A_PER = (A_TOT + NW - 1) / NW;
  static constexpr int B_PER = (B_TOT + NW - 1) / NW;
  static constexpr bool EVEN =
      A_TOT % NW == 0 && B_TOT % NW == 0 && (!PRE || S_TOT % NW == 0);
  static constexpr int S_SLOT = S_TOT * 64 * S_LANE;
  // scale slots: one per stage (prepacked) or stage pair, enough for every
  // stage in flight
  static constexpr int S_SLOTS = PRE ? STAGES : (STAGES + 2) / 2;
  static constexpr int PIPE = STAGES * A_STAGE + B_REGION + S_SLOTS * S_SLOT;
  // loads a wave issues for one stage (the prepacked scales come every stage;
  // the original ones every other, which waiting for this count covers)
  static constexpr int PER_STAGE = A_PER + B_PER + (PRE ? S_PER : 0);
};

// The finished tile is staged in LDS (reusing the pipeline buffers) in as
// few row passes as fit: the smallest power of two P, keeping BM / P a
// multiple of 16, with (BM / P) * row_bytes <= pipe_bytes.
constexpr int epi_passes(int bm, int row_bytes, int pipe_bytes) {
  int p = 1;
  while ((bm / p) * row_bytes > pipe_bytes && (bm / p) % 32 == 0) p *= 2;
  return p;
}

// One 64-deep stage of a wave's FM x FN block of 16 x 16 outputs: all LDS
// reads of the stage first (the reads of ks = 1 overlap the MFMAs of ks = 0),
// then per ks: decode every weight fragment, then the FM x FN MFMAs back to
// back.  Logical chunk ks*4 + grp of an A row sits at physical chunk (grp ^
// sw) ^ (ks*4): flipping bit 6 of the byte offset selects the ks = 1 half.
// Original weights: Ss points at the stage's two scale bytes of the wave's
// first weight row, each fragment is a dword of its row (b_rd, b_sw swizzle).
// Prepacked (PRE): a fragment's two dwords (ks = 0, 1) are 8 consecutive
// bytes per lane of its group's 512-byte block (b_rd = group block + 8 *
// lane), and the high halves of its two scale operands one dword of the
// group's 64-byte scale block (s_rd = group block + 4 * row): conflict-free
// reads, one shift or mask per scale.
template <typename T, int FM, int FN, bool PRE, int RB = 32>
__device__ __forceinline__ void stage_math(const uint8_t* As, const uint8_t* Bs, const uint8_t* Ss,
                                           int a_rd0, int b_rd, int b_sw, int s_rd,
                                           f32x4 (&acc)[FM][FN], int cb = 0) {
  typedef typename V8Of<T>::type V8;
  V8 af[2][FM];
  uint32_t raw[2][FN];
  float sc[2][FN];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
      af[ks][fm] = *reinterpret_cast<const V8*>(As + ((a_rd0 + fm * 16 * 128) ^ (ks * 64)));
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    if constexpr (PRE) {
      // (written as dword reads, which the compiler pairs into 8-byte reads:
      // through a uint2 / float2 type the reads lose the LDS alias
      // information that lets them run while the next stage's direct-to-LDS
      // loads are in flight, and a full vmcnt wait precedes them)
      raw[0][fn] = *reinterpret_cast<const uint32_t*>(Bs + b_rd + fn * 512);
      raw[1][fn] = *reinterpret_cast<const uint32_t*>(Bs + b_rd + fn * 512 + 4);
      const uint32_t sv = *reinterpret_cast<const uint32_t*>(Ss + s_rd + fn * 64);
      sc[0][fn] = __uint_as_float(sv << 16);
      sc[1][fn] = __uint_as_float(sv & 0xFFFF0000u);
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        raw[ks][fn] =
            *reinterpret_cast<const uint32_t*>(Bs + b_rd + fn * 16 * RB + (((cb + ks) ^ b_sw) * 16));
        sc[ks][fn] = e8m0_scale(Ss[s_rd + fn * 16 * 4 + ks]);
      }
    }
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    V8 bf[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) bf[fn] = Decode<T>::run(raw[ks][fn], sc[ks][fn]);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) acc[fm][fn] = mfma16(bf[fn], af[ks][fm], acc[fm][fn]);
  }
}

template <typename T, int WGM, int WGN, int FM, int FN, int STAGES, int EPI, int MINB, bool PRE,
          int BG = 1>
__global__ __launch_bounds__(64 * WGM * WGN, MINB) void w4a16_pf(GemmArgs g, int nbm, int nbn) {
  typedef PfShape<WGM, WGN, FM, FN, STAGES, PRE, BG> S;
  constexpr int BM = S::BM, BN = S::BN, NT = S::NT;
  constexpr int OUT_COLS = (EPI == EPI_SILU_MUL) ? BN / 2 : BN;
  constexpr int ES = (EPI == EPI_PARTIAL) ? 4 : 2;  // bytes per output element
  constexpr int C_LD = OUT_COLS * ES + 16;         // bytes per staged output row
  constexpr int EPI_PASSES = epi_passes(BM, C_LD, S::PIPE);
  constexpr int EPI_ROWS = BM / EPI_PASSES;
  constexpr int SMEM = S::PIPE > EPI_ROWS * C_LD ? S::PIPE : EPI_ROWS * C_LD;
  static_assert(BN % 32 == 0 && EPI_ROWS % 16 == 0, "tile config");
  static_assert(STAGES == 2 || S::EVEN, "multi-stage waits count loads per wave");
  static_assert(STAGES >= 2 && STAGES <= 8, "2 to 8 stages");
  static_assert((STAGES - 2) * S::PER_STAGE <= 63, "vmcnt holds at most 63");
  static_assert(EPI != EPI_SILU_MUL || FN % 2 == 0, "SiLU pairs need even FN");
  static_assert(BG == 1 || (!PRE && EPI != EPI_PARTIAL && STAGES <= 3 && BG <= 4 &&
                            S::B_GTOT % S::NW == 0),
                "weight-line groups: original layout, whole K, at most 3 stages");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  uint8_t* const sA = smem;
  uint8_t* const sB = smem + STAGES * S::A_STAGE;
  uint8_t* const sS = smem + STAGES * S::A_STAGE + S::B_REGION;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the per-wave load choices and LDS addresses
  // (M0) then need no lane-to-scalar moves or exec masking
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int c16 = lane & 15;
  const int grp = lane >> 4;

  // split K: workgroup i computes slice i / (nbm * nbn) of tile i % (nbm * nbn)
  const int ntile = nbm * nbn;
  const int split = (EPI == EPI_PARTIAL) ? (int)blockIdx.x / ntile : 0;
  int bm, bn;
  if (EPI == EPI_PARTIAL) {
    if (!tile_of(g, BM, nbm, nbn, bm, bn, (int)blockIdx.x % ntile, ntile)) return;
  } else {
    if (!tile_of(g, BM, nbm, nbn, bm, bn, blockIdx.x, gridDim.x)) return;
  }
  const int64_t pos0 = (int64_t)bm * BM;
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = bn * OUT_COLS;

  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    for (int idx = tid; idx < BM * OUT_COLS; idx += NT) {
      const int r = idx / OUT_COLS, cc = idx % OUT_COLS;
      const RowInfo ri = row_info(g, pos0 + r);
      if (ri.valid && ncol0 + cc < g.n) {
        if constexpr (EPI == EPI_STORE_F32)
          static_cast<float*>(g.c)[ri.out_row * g.ldc + ncol0 + cc] = 0.f;
        else
          static_cast<T*>(g.c)[ri.out_row * g.ldc + ncol0 + cc] = from_f32<T>(0.f);
      }
    }
    return;
  }

  // ---- buffer resources
  const i32x4 rA = make_rsrc(g.a, (uint32_t)(g.a_rows * g.lda * (int64_t)sizeof(T)));
  const int64_t b_rows_total = (EPI == EPI_SILU_MUL) ? 2 * (int64_t)g.inter : (int64_t)g.n;
  const i32x4 rB = make_rsrc(g.b + expert * g.b_e,
                             (uint32_t)(PRE ? prepacked_nibble_bytes(b_rows_total, g.k)
                                            : b_rows_total * g.b_n));
  const i32x4 rS = make_rsrc(g.bs + expert * g.bs_e,
                             (uint32_t)(PRE ? prepacked_scale_bytes(b_rows_total, g.k)
                                            : b_rows_total * g.bs_n));
  const int64_t nk_all = g.k / 64;  // stages of the whole K (prepacked group stride)

  // B-tile row -> weight row (or -1 past N).  With SiLU, 16-row blocks
  // alternate gate (even) and up (odd) rows of the same output columns.
  auto weight_row = [&](int i) -> int {
    if (i >= BN) return -1;
    int orow, grow;
    if (EPI == EPI_SILU_MUL) {
      const int cbk = i >> 4;
      orow = ncol0 + (cbk >> 1) * 16 + (i & 15);
      grow = (cbk & 1 ? g.inter : 0) + orow;
    } else {
      orow = ncol0 + i;
      grow = orow;
    }
    return orow < g.n ? grow : -1;
  };

  // ---- per-lane load offsets for stage 0; stage kt adds kt * stride as
  // the instruction's scalar offset (no per-stage vector adds; offsets of
  // padding lanes stay past the end of the buffer).
  // Wave-load q of a stage (q < A_TOT / B_TOT) is issued by wave q % NW.
  uint32_t a_off[S::A_PER];
#pragma unroll
  for (int j = 0; j < S::A_PER; ++j) {
    const int q = j * S::NW + wave;
    const int row = q * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (row & 7);
    a_off[j] = kOOB;
    if (q < S::A_TOT) {
      const RowInfo ri = row_info(g, pos0 + row);
      if (ri.valid) a_off[j] = (uint32_t)(ri.a_row * g.lda * (int64_t)sizeof(T)) + c * 16;
    }
  }
  // Prepacked: B wave-load q holds groups 2q and 2q + 1 (lanes 0-31, 32-63;
  // 16 bytes each of the group's 512-byte stage block); scale byte b of the
  // stage's scale region is byte b % 64 of group b / 64's 64-byte block.
  // Weight-line groups: wave-load q holds rows q * 64 / CPRB .., lane l
  // filling slot l % CPRB of its row with the chunk that belongs there
  // (chunk c of row r sits in slot c ^ (r * BG / 8) % CPRB: the 16 rows of a
  // fragment read hit all 64 banks).
  constexpr int BPW = BG > 1 ? S::B_GPER : S::B_PER;
  uint32_t b_off[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int q = j * S::NW + wave;
    if constexpr (BG > 1) {
      constexpr int CPRB = 2 * BG;
      const int row = q * (64 / CPRB) + lane / CPRB;
      const int c = (lane % CPRB) ^ ((row * BG / 8) % CPRB);
      const int grow = q < S::B_GTOT ? weight_row(row) : -1;
      b_off[j] = grow >= 0 ? (uint32_t)(grow * g.b_n) + c * 16 : kOOB;
    } else if constexpr (PRE) {
      const int gt = 2 * q + (lane >> 5);
      const int grow = (q < S::B_TOT && gt < S::GRP) ? weight_row(gt * 16) : -1;
      b_off[j] = grow >= 0 ? (uint32_t)((grow >> 4) * nk_all * 512) + (lane & 31) * 16 : kOOB;
    } else {
      const int row = q * 32 + (lane >> 1);
      const int c = (lane & 1) ^ ((row >> 3) & 1);
      const int grow = q < S::B_TOT ? weight_row(row) : -1;
      b_off[j] = grow >= 0 ? (uint32_t)(grow * g.b_n) + c * 16 : kOOB;
    }
  }
  uint32_t s_off[S::S_PER];
#pragma unroll
  for (int j = 0; j < S::S_PER; ++j) {
    const int q = j * S::NW + wave;
    if constexpr (PRE) {
      const int sb = (q * 64 + lane) * S::S_LANE;
      const int gt = sb >> 6;
      const int grow = (q < S::S_TOT && gt < S::GRP) ? weight_row(gt * 16) : -1;
      s_off[j] = grow >= 0 ? (uint32_t)((grow >> 4) * nk_all * 64) + (sb & 63) : kOOB;
    } else {
      const int grow = q < S::S_TOT ? weight_row(q * 64 + lane) : -1;
      s_off[j] = grow >= 0 ? (uint32_t)(grow * g.bs_n) : kOOB;
    }
  }

  // 64-deep stages [k_begin, k_end) of this workgroup's K slice; slices
  // start on even stages (the scale loads cover stage pairs)
  int k_begin = 0, k_end = g.k / 64;
  if (EPI == EPI_PARTIAL) {
    const int per = ((k_end + g.splitk - 1) / g.splitk + 1) & ~1;
    k_begin = split * per < k_end ? split * per : k_end;
    k_end = k_begin + per < k_end ? k_begin + per : k_end;
  }
  auto issue = [&](int kt) {
    const int st = kt % STAGES;
    if constexpr (BG > 1) {
      // stages kt .. kt + BG - 1 of every weight row, with the first of them
      if (kt % BG == 0) {
        uint8_t* const slot = sB + ((kt / BG) & 1) * S::B_GRP;
#pragma unroll
        for (int j = 0; j < BPW; ++j)
          llvm_amdgcn_raw_buffer_load_lds(rB, lds_ptr(slot + (j * S::NW + wave) * 1024), 16,
                                          (int)b_off[j], kt * 32, 0, 0);
      }
    }
    if constexpr (PRE) {
#pragma unroll
      for (int j = 0; j < S::S_PER; ++j) {
        const int q = j * S::NW + wave;
        if (S::S_TOT % S::NW == 0 || q < S::S_TOT)
          llvm_amdgcn_raw_buffer_load_lds(rS, lds_ptr(sS + st * S::S_SLOT + q * 64 * S::S_LANE),
                                          S::S_LANE, (int)s_off[j], kt * 64, 0, 0);
      }
    } else if ((kt & 1) == 0) {
#pragma unroll
      for (int j = 0; j < S::S_PER; ++j) {
        const int q = j * S::NW + wave;
        if (q < S::S_TOT)
          llvm_amdgcn_raw_buffer_load_lds(rS, lds_ptr(sS + ((kt >> 1) % S::S_SLOTS) * S::S_SLOT + q * 256),
                                          4, (int)s_off[j], (kt >> 1) * 4, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < S::A_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::A_TOT % S::NW == 0 || q < S::A_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rA, lds_ptr(sA + st * S::A_STAGE + q * 1024), 16,
                                        (int)a_off[j], kt * 128, 0, 0);
    }
    if constexpr (BG == 1) {
#pragma unroll
      for (int j = 0; j < S::B_PER; ++j) {
        const int q = j * S::NW + wave;
        if (S::B_TOT % S::NW == 0 || q < S::B_TOT)
          llvm_amdgcn_raw_buffer_load_lds(rB, lds_ptr(sB + st * S::B_STAGE + q * 1024), 16,
                                          (int)b_off[j], kt * (PRE ? 512 : 32), 0, 0);
      }
    }
  };
  // weight-line groups: this wave's loads of stage x (a per-wave count: the
  // A and scale wave-loads need not divide among the waves)
  int a_w = 0, s_w = 0;
#pragma unroll
  for (int j = 0; j < S::A_PER; ++j) a_w += (S::A_TOT % S::NW == 0 || j * S::NW + wave < S::A_TOT);
#pragma unroll
  for (int j = 0; j < S::S_PER; ++j) s_w += (j * S::NW + wave < S::S_TOT);
  auto stage_loads = [&](int x) {
    return a_w + (x % BG == 0 ? S::B_GPER : 0) + ((x & 1) == 0 ? s_w : 0);
  };

  // ---- per-lane LDS read offsets (fragment rows differ from c16 by
  // multiples of 16, so the swizzle terms are lane constants)
  const int a_rd0 = (wm * FM * 16 + c16) * 128 + ((grp ^ (c16 & 7)) * 16);
  const int b_sw = (c16 * BG / 8) % (2 * BG);
  const int b_rd = (wn * FN * 16 + c16) * S::RBB + grp * 4;
  const int s_rd = (wn * FN * 16 + c16) * 4;
  const int b_rd_pre = wn * FN * 512 + lane * 8;  // group wn*FN's block, lane's 8 bytes
  const int s_rd_pre = wn * FN * 64 + c16 * 4;    // group wn*FN's scales, row c16

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  // the stage waits count loads per stage in issue order: a compiler fence
  // after each prologue stage keeps stage s + 1's loads behind stage s's
  for (int s = 0; s < STAGES - 1; ++s) {
    if (k_begin + s < k_end) issue(k_begin + s);
    asm volatile("" ::: "memory");
  }
  for (int kt = k_begin; kt < k_end; ++kt) {
    // Stage kt has landed once at most the later stages' loads are
    // outstanding.  A bare s_barrier (not __syncthreads, whose release fence
    // would drain every outstanding load) then publishes it to all waves and
    // retires the reads of the buffer the next issue() overwrites.
    // (a wave's loads of one later stage number at most PER_STAGE, plus,
    // original layout, one scale load on even stages, which waiting for
    // PER_STAGE covers)
    const int later = (k_end - 1 - kt) < (STAGES - 2) ? (k_end - 1 - kt) : (STAGES - 2);
    if constexpr (BG > 1) {
      // at most one later stage in flight (STAGES <= 3): its exact count
      const int cnt = later > 0 ? stage_loads(kt + 1) : 0;
      static_for<0, S::A_PER + S::B_GPER + S::S_PER + 1>([&](auto c) {
        if (cnt == decltype(c)::value) wait_vmcnt<decltype(c)::value>();
      });
    } else {
      static_for<0, STAGES - 1>([&](auto c) {
        if (later == decltype(c)::value) wait_vmcnt<decltype(c)::value * S::PER_STAGE>();
      });
    }
    barrier_only();
    if (kt + STAGES - 1 < k_end) issue(kt + STAGES - 1);
    if constexpr (PRE)
      stage_math<T, FM, FN, true>(sA + (kt % STAGES) * S::A_STAGE, sB + (kt % STAGES) * S::B_STAGE,
                                  sS + (kt % STAGES) * S::S_SLOT, a_rd0, b_rd_pre, 0, s_rd_pre, acc);
    else if constexpr (BG > 1)
      stage_math<T, FM, FN, false, S::RBB>(
          sA + (kt % STAGES) * S::A_STAGE, sB + ((kt / BG) & 1) * S::B_GRP,
          sS + ((kt >> 1) % S::S_SLOTS) * S::S_SLOT + (kt & 1) * 2, a_rd0, b_rd, b_sw, s_rd, acc,
          2 * (kt % BG));
    else
      stage_math<T, FM, FN, false>(sA + (kt % STAGES) * S::A_STAGE, sB + (kt % STAGES) * S::B_STAGE,
                                   sS + ((kt >> 1) % S::S_SLOTS) * S::S_SLOT + (kt & 1) * 2, a_rd0,
                                   b_rd, b_sw, s_rd, acc);
  }

  // ---- epilogue: lane owns row wm*FM*16 + fm*16 + c16 and columns
  // fn*16 + grp*4 .. +3 of its wave's sub-tile; stage the finished rows in
  // LDS and write whole 16-byte chunks
  barrier_only();  // every wave is done reading the stage buffers
  // a K slice's partial sums are stored raw; scaling and bias come once,
  // after the slices are summed
  float alpha = (EPI == EPI_PARTIAL) ? 1.0f : scalar_alpha(g, expert);
  if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_F32) {
    if (g.ref_round) {
      ref_pass<std::conditional_t<EPI == EPI_STORE_F32, float, T>>(g, expert, acc);
      alpha = 1.0f;
    }
  }
  // the lane's bias values, once (columns past N read as zero)
  constexpr bool kBias = EPI == EPI_STORE || EPI == EPI_STORE_F32;
  float bv[kBias ? FN : 1][4];
  if (kBias && g.bias) {
#pragma unroll
    for (int fn = 0; fn < (kBias ? FN : 1); ++fn) {
      const int col = ncol0 + wn * FN * 16 + fn * 16 + grp * 4;
      const T* bp = static_cast<const T*>(g.bias) + col;
      if (col + 4 <= g.n && (reinterpret_cast<uintptr_t>(bp) & 7) == 0) {
        const uint2 v = *reinterpret_cast<const uint2*>(bp);
        bv[fn][0] = to_f32(__builtin_bit_cast(T, (uint16_t)(v.x & 0xFFFF)));
        bv[fn][1] = to_f32(__builtin_bit_cast(T, (uint16_t)(v.x >> 16)));
        bv[fn][2] = to_f32(__builtin_bit_cast(T, (uint16_t)(v.y & 0xFFFF)));
        bv[fn][3] = to_f32(__builtin_bit_cast(T, (uint16_t)(v.y >> 16)));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) bv[fn][i] = col + i < g.n ? to_f32(bp[i]) : 0.f;
      }
    }
  }
  if constexpr (EPI == EPI_STORE_F32) {
    // C in FP32: a lane's 4 consecutive columns of a fragment are one
    // 16-byte store, nothing rounded to T (the products of bf16 A and the
    // E2M1 x 2^k weights are exact, summed in FP32 by the MFMA)
    float* const cbase = static_cast<float*>(g.c);
    const bool vec = g.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(g.c) & 15) == 0;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const RowInfo r = row_info(g, pos0 + wm * FM * 16 + fm * 16 + c16);
      if (!r.valid) continue;
      const float rw = g.route_w ? g.route_w[r.out_row] : 1.0f;
      float* const crow = cbase + r.out_row * g.ldc;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = ncol0 + wn * FN * 16 + fn * 16 + grp * 4;
        if (col >= g.n) continue;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[i] = acc[fm][fn][i] * alpha;
          if (g.route_w) o[i] *= rw;
          if (g.bias) o[i] += bv[fn][i];
        }
        if (vec && col + 4 <= g.n) {
          *reinterpret_cast<f32x4*>(crow + col) = f32x4{o[0], o[1], o[2], o[3]};
        } else {
          for (int i = 0; i < 4 && col + i < g.n; ++i) crow[col + i] = o[i];
        }
      }
    }
    return;
  }
  if constexpr (EPI == EPI_STORE && FN >= 2) {
    if (g.ldc % 8 == 0) {
      // Straight from the registers (no LDS staging, no barrier): lane
      // pairs (grp 0, 1) and (2, 3) trade halves with v_permlane16_swap so
      // that each lane holds 8 consecutive columns of one block (even grp:
      // block 2fp, odd grp: block 2fp + 1) and stores 16 bytes; an odd
      // last block goes out as 8 bytes per lane.  Same arithmetic as the
      // staged path below.
      T* const cbase = static_cast<T*>(g.c);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int trow = wm * FM * 16 + fm * 16 + c16;
        const RowInfo r = row_info(g, pos0 + trow);
        float rw = 1.0f;
        if (g.route_w) rw = r.valid ? g.route_w[r.out_row] : 0.f;
        T* const crow = cbase + (r.valid ? r.out_row : 0) * g.ldc;
        auto outv = [&](int fn, int i) {
          float o = acc[fm][fn][i] * alpha * rw;
          if (g.bias) o += bv[fn][i];
          return o;
        };
#pragma unroll
        for (int fp = 0; fp < FN / 2; ++fp) {
          uint32_t pv[2], qv[2];  // pv: block 2fp, qv: block 2fp + 1 (4 columns each)
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            pv[w] = pack2<T>(outv(2 * fp, 2 * w), outv(2 * fp, 2 * w + 1));
            qv[w] = pack2<T>(outv(2 * fp + 1, 2 * w), outv(2 * fp + 1, 2 * w + 1));
            const auto sw = __builtin_amdgcn_permlane16_swap(pv[w], qv[w], false, false);
            pv[w] = sw[0];
            qv[w] = sw[1];
          }
          const int col = ncol0 + wn * FN * 16 + (2 * fp + (grp & 1)) * 16 + (grp & 2) * 4;
          if (!r.valid || col >= g.n) continue;
          const uint32_t v[4] = {pv[0], pv[1], qv[0], qv[1]};
          if (col + 8 <= g.n) {
            *reinterpret_cast<i32x4*>(crow + col) =
                i32x4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
          } else {
            for (int i = 0; i < 8 && col + i < g.n; ++i)
              crow[col + i] = __builtin_bit_cast(T, (uint16_t)(v[i / 2] >> (16 * (i & 1))));
          }
        }
        if constexpr (FN % 2 == 1) {
          constexpr int fn = FN - 1;
          const int col = ncol0 + wn * FN * 16 + fn * 16 + grp * 4;
          const uint32_t v0 = pack2<T>(outv(fn, 0), outv(fn, 1));
          const uint32_t v1 = pack2<T>(outv(fn, 2), outv(fn, 3));
          if (r.valid && col < g.n) {
            if (col + 4 <= g.n) {
              *reinterpret_cast<uint2*>(crow + col) = uint2{v0, v1};
            } else {
              const uint32_t v[2] = {v0, v1};
              for (int i = 0; i < 4 && col + i < g.n; ++i)
                crow[col + i] = __builtin_bit_cast(T, (uint16_t)(v[i / 2] >> (16 * (i & 1))));
            }
          }
        }
      }
      return;
    }
  }
#pragma unroll
  for (int pass = 0; pass < EPI_PASSES; ++pass) {
    {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        if ((wm * FM * 16 + fm * 16) / EPI_ROWS != pass) continue;  // another pass's rows
        const int trow = wm * FM * 16 + fm * 16 + c16;
        float rw = 1.0f;
        if (EPI == EPI_STORE && g.route_w) {
          const RowInfo r = row_info(g, pos0 + trow);
          rw = r.valid ? g.route_w[r.out_row] : 0.f;
        }
        uint8_t* crow = smem + (trow - pass * EPI_ROWS) * C_LD;
        if (EPI == EPI_SILU_MUL) {
#pragma unroll
          for (int fn = 0; fn < FN; fn += 2) {
            const int tcol = ((wn * FN + fn) >> 1) * 16 + grp * 4;
            float h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              // vllm:249-252 on tensors of T: gate and up rounded to T, silu
              // in FP32 rounded to T, the product rounded to T (below)
              const T gb = from_f32<T>(acc[fm][fn][i] * alpha);
              const T ub = from_f32<T>(acc[fm][fn + 1][i] * alpha);
              const T sb = silu_round<T>(gb);
              h[i] = to_f32(sb) * to_f32(ub);
            }
            *reinterpret_cast<uint2*>(crow + tcol * 2) =
                uint2{pack2<T>(h[0], h[1]), pack2<T>(h[2], h[3])};
          }
        } else if (EPI == EPI_PARTIAL) {
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            const int tcol = wn * FN * 16 + fn * 16 + grp * 4;
            *reinterpret_cast<f32x4*>(crow + tcol * 4) = acc[fm][fn];
          }
        } else {
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            const int tcol = wn * FN * 16 + fn * 16 + grp * 4;
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = acc[fm][fn][i] * alpha * rw;
            if (g.bias) {
#pragma unroll
              for (int i = 0; i < 4; ++i) o[i] += bv[fn][i];
            }
            *reinterpret_cast<uint2*>(crow + tcol * 2) =
                uint2{pack2<T>(o[0], o[1]), pack2<T>(o[2], o[3])};
          }
        }
      }
    }
    __syncthreads();
    // whole 16-byte chunks, consecutive lanes along a row
    typedef typename std::conditional<EPI == EPI_PARTIAL, float, T>::type TO;
    constexpr int VALS = 16 / ES;  // outputs per chunk
    constexpr int CHUNKS = OUT_COLS / VALS;
    TO* const cbase = (EPI == EPI_PARTIAL)
                          ? reinterpret_cast<TO*>(g.splitk_ws + (int64_t)split * g.m * g.n)
                          : static_cast<TO*>(g.c);
    const int64_t ldc = (EPI == EPI_PARTIAL) ? (int64_t)g.n : g.ldc;
    for (int idx = tid; idx < EPI_ROWS * CHUNKS; idx += NT) {
      const int prow = idx / CHUNKS, ch = idx % CHUNKS;
      const int trow = pass * EPI_ROWS + prow;
      const int col = ncol0 + ch * VALS;
      if (col >= g.n) continue;
      const RowInfo r = row_info(g, pos0 + trow);
      if (!r.valid) continue;
      const uint8_t* src = smem + prow * C_LD + ch * 16;
      TO* dst = cbase + r.out_row * ldc + col;
      if (col + VALS <= g.n && (ldc % VALS) == 0) {
        *reinterpret_cast<i32x4*>(dst) = *reinterpret_cast<const i32x4*>(src);
      } else {
        const TO* sv = reinterpret_cast<const TO*>(src);
        for (int i = 0; i < VALS && col + i < g.n; ++i) dst[i] = sv[i];
      }
    }
    if (EPI_PASSES > 1 && pass + 1 < EPI_PASSES) __syncthreads();
  }
}

// ---------------------------------------------------------------- persistent
// Grids of several rounds (more tiles than resident workgroups) pay a fixed
// cost per tile in the kernel above: the first stage's load latency, the
// epilogue and the workgroup turnover, all exposed because the resident
// workgroups run in step.  At K = 768 (a MoE down projection) that is ~20%
// of a tile.  w4a16_pp keeps one workgroup per slot and walks tiles t =
// blockIdx.x, + gridDim.x, ... (gridDim.x a multiple of 8, so every tile
// stays on the XCD that tile_of assigns it).  The stage counter runs on
// across tiles: the last stage of a tile issues the first stage of the next
// one into the free buffer, so the pipeline never drains.  The epilogue
// writes 4 outputs per lane straight from the accumulators (8-byte buffer
// stores; no LDS staging, which would need room beside the stage buffers).
// Per-row metadata goes through two LDS tables (this tile, next tile): the
// next tile's sorted ids are loaded during the current tile's first stage
// and turned into output / activation rows at its last one; route weights
// and bias are loaded during the tile's own first stage.  Same MFMA order
// and epilogue arithmetic as w4a16_pf: results are bitwise equal.
// Requirements (host): the w4a16_pf ones, 2 stages, 1 x 4 waves, output
// columns and row stride multiples of 4, 8-byte aligned output and output
// rows below 2 GiB.  The epilogue stores 16 bytes per lane where columns
// and row stride are multiples of 8 and the output 16-byte aligned, else 8.

extern "C" __device__ void llvm_amdgcn_raw_buffer_store_v2i32(i32x2 vdata, i32x4 rsrc,
                                                              uint32_t voffset, int soffset,
                                                              int aux)
    __asm("llvm.amdgcn.raw.buffer.store.v2i32");
extern "C" __device__ void llvm_amdgcn_raw_buffer_store_v4i32(i32x4 vdata, i32x4 rsrc,
                                                              uint32_t voffset, int soffset,
                                                              int aux)
    __asm("llvm.amdgcn.raw.buffer.store.v4i32");

template <typename T, int FM, int FN, int EPI, int MINB, bool PRE>
__global__ __launch_bounds__(256, MINB) void w4a16_pp(GemmArgs g, int nbm, int nbn,
                                                      uint32_t c_bytes) {
  typedef PfShape<1, 4, FM, FN, 2, PRE> S;
  constexpr int BM = S::BM, BN = S::BN, NT = S::NT;
  constexpr int OUT_COLS = (EPI == EPI_SILU_MUL) ? BN / 2 : BN;
  constexpr int BIAS_PER = (OUT_COLS + NT - 1) / NT;
  // table slot: output row, activation row (-1: none), route weight per
  // tile row; bias per output column
  constexpr int TAB = BM * 12 + OUT_COLS * 4;
  static_assert(EPI == EPI_STORE || EPI == EPI_SILU_MUL, "plain or SiLU epilogue");
  static_assert(EPI != EPI_SILU_MUL || FN % 2 == 0, "SiLU pairs need even FN");
  static_assert(BM <= NT, "one table row per thread");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S::PIPE + 2 * TAB];
  uint8_t* const sA = smem;
  uint8_t* const sB = smem + 2 * S::A_STAGE;
  uint8_t* const sS = smem + 2 * (S::A_STAGE + S::B_STAGE);
  uint8_t* const sT = smem + S::PIPE;
  auto t_orow = [&](int slot) { return reinterpret_cast<int*>(sT + slot * TAB); };
  auto t_arow = [&](int slot) { return reinterpret_cast<int*>(sT + slot * TAB + BM * 4); };
  auto t_rw = [&](int slot) { return reinterpret_cast<float*>(sT + slot * TAB + BM * 8); };
  auto t_bias = [&](int slot) { return reinterpret_cast<float*>(sT + slot * TAB + BM * 12); };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // = wn (one wave row)
  const int c16 = lane & 15;
  const int grp = lane >> 4;
  const int ntile = nbm * nbn;
  const int nk = g.k / 64;
  const int64_t b_rows_total = (EPI == EPI_SILU_MUL) ? 2 * (int64_t)g.inter : (int64_t)g.n;

  // sorted id (or dense row) of row `tid` of the tile at row block bm_ ->
  // output row and activation row, -1 when the row is padding
  auto rows_of = [&](int bm_, int sid, int& orow, int& arow) {
    const int64_t pos = (int64_t)bm_ * BM + tid;
    if (g.sorted_ids == nullptr) {
      orow = pos < g.m ? (int)pos : -1;
      arow = orow;
    } else {
      const bool ok = sid >= 0 && sid < g.num_valid;
      orow = ok ? sid : -1;
      arow = ok ? sid / g.top_k : -1;
    }
  };

  int t = blockIdx.x, bm, bn;
  if (!tile_of(g, BM, nbm, nbn, bm, bn, t, ntile)) return;
  int expert = g.sorted_ids ? block_expert(g, (int64_t)bm * BM) : 0;
  if (tid < BM) {
    const int sid = g.sorted_ids ? g.sorted_ids[(int64_t)bm * BM + tid] : 0;
    int o, a;
    rows_of(bm, sid, o, a);
    t_orow(0)[tid] = o;
    t_arow(0)[tid] = a;
  }
  __syncthreads();

  // ---- load offsets and buffer resources of a tile (its rows in table
  // `slot`); stage kt adds kt * stride as the instruction's scalar offset
  uint32_t a_off[S::A_PER], b_off[S::B_PER], s_off[S::S_PER];
  i32x4 rA = make_rsrc(g.a, (uint32_t)(g.a_rows * g.lda * (int64_t)sizeof(T)));
  i32x4 rB, rS;
  auto setup = [&](int bn_, int expert_, int slot) {
    const int ncol0_ = bn_ * OUT_COLS;
    const int e = expert_ < 0 ? 0 : expert_;
    // expert < 0: empty resources, every operand reads zero
    const int64_t b_bytes =
        PRE ? prepacked_nibble_bytes(b_rows_total, g.k) : b_rows_total * g.b_n;
    const int64_t s_bytes =
        PRE ? prepacked_scale_bytes(b_rows_total, g.k) : b_rows_total * g.bs_n;
    rB = make_rsrc(g.b + e * g.b_e, expert_ < 0 ? 0u : (uint32_t)b_bytes);
    rS = make_rsrc(g.bs + e * g.bs_e, expert_ < 0 ? 0u : (uint32_t)s_bytes);
    auto weight_row = [&](int i) -> int {
      int orow, grow;
      if (EPI == EPI_SILU_MUL) {
        const int cbk = i >> 4;
        orow = ncol0_ + (cbk >> 1) * 16 + (i & 15);
        grow = (cbk & 1 ? g.inter : 0) + orow;
      } else {
        orow = ncol0_ + i;
        grow = orow;
      }
      return orow < g.n ? grow : -1;
    };
#pragma unroll
    for (int j = 0; j < S::A_PER; ++j) {
      const int q = j * S::NW + wave;
      const int row = q * 8 + (lane >> 3);
      const int c = (lane & 7) ^ (row & 7);
      const int ar = q < S::A_TOT ? t_arow(slot)[row] : -1;
      a_off[j] = (ar >= 0 && expert_ >= 0) ? (uint32_t)(ar * g.lda * (int64_t)sizeof(T)) + c * 16
                                           : kOOB;
    }
    // (prepacked addressing as in w4a16_pf)
#pragma unroll
    for (int j = 0; j < S::B_PER; ++j) {
      const int q = j * S::NW + wave;
      if constexpr (PRE) {
        const int gt = 2 * q + (lane >> 5);
        const int grow = (q < S::B_TOT && gt < S::GRP) ? weight_row(gt * 16) : -1;
        b_off[j] = grow >= 0 ? (uint32_t)((grow >> 4) * (int64_t)nk * 512) + (lane & 31) * 16 : kOOB;
      } else {
        const int row = q * 32 + (lane >> 1);
        const int c = (lane & 1) ^ ((row >> 3) & 1);
        const int grow = q < S::B_TOT ? weight_row(row) : -1;
        b_off[j] = grow >= 0 ? (uint32_t)(grow * g.b_n) + c * 16 : kOOB;
      }
    }
#pragma unroll
    for (int j = 0; j < S::S_PER; ++j) {
      const int q = j * S::NW + wave;
      if constexpr (PRE) {
        const int sb = (q * 64 + lane) * S::S_LANE;
        const int gt = sb >> 6;
        const int grow = (q < S::S_TOT && gt < S::GRP) ? weight_row(gt * 16) : -1;
        s_off[j] = grow >= 0 ? (uint32_t)((grow >> 4) * (int64_t)nk * 64) + (sb & 63) : kOOB;
      } else {
        const int grow = q < S::S_TOT ? weight_row(q * 64 + lane) : -1;
        s_off[j] = grow >= 0 ? (uint32_t)(grow * g.bs_n) : kOOB;
      }
    }
  };
  // stage kt of the current tile into buffer gk % 2 (gk: stage counter
  // across tiles; every tile has an even number of stages, so gk and kt
  // have the same parity and the scale slots alternate as in w4a16_pf)
  auto issue = [&](int kt, int gk) {
    const int st = gk & 1;
    if constexpr (PRE) {
#pragma unroll
      for (int j = 0; j < S::S_PER; ++j) {
        const int q = j * S::NW + wave;
        if (S::S_TOT % S::NW == 0 || q < S::S_TOT)
          llvm_amdgcn_raw_buffer_load_lds(rS, lds_ptr(sS + st * S::S_SLOT + q * 64 * S::S_LANE),
                                          S::S_LANE, (int)s_off[j], kt * 64, 0, 0);
      }
    } else if ((kt & 1) == 0) {
#pragma unroll
      for (int j = 0; j < S::S_PER; ++j) {
        const int q = j * S::NW + wave;
        if (q < S::S_TOT)
          llvm_amdgcn_raw_buffer_load_lds(rS, lds_ptr(sS + ((gk >> 1) & 1) * S::S_SLOT + q * 256),
                                          4, (int)s_off[j], (kt >> 1) * 4, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < S::A_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::A_TOT % S::NW == 0 || q < S::A_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rA, lds_ptr(sA + st * S::A_STAGE + q * 1024), 16,
                                        (int)a_off[j], kt * 128, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < S::B_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::B_TOT % S::NW == 0 || q < S::B_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rB, lds_ptr(sB + st * S::B_STAGE + q * 1024), 16,
                                        (int)b_off[j], kt * (PRE ? 512 : 32), 0, 0);
    }
  };

  const int a_rd0 = c16 * 128 + ((grp ^ (c16 & 7)) * 16);
  const int b_sw = (c16 >> 3) & 1;
  const int b_rd = (wave * FN * 16 + c16) * 32 + grp * 4;
  const int s_rd = (wave * FN * 16 + c16) * 4;
  const int b_rd_pre = wave * FN * 512 + lane * 8;
  const int s_rd_pre = wave * FN * 64 + c16 * 4;
  const i32x4 rC = make_rsrc(g.c, c_bytes);
  // 16-byte stores where every 8-column run starting below N ends within
  // it and the rows are 16-byte aligned
  const bool wide =
      g.n % 8 == 0 && g.ldc % 8 == 0 && (reinterpret_cast<uintptr_t>(g.c) & 15) == 0;

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  setup(bn, expert, 0);
  int gk = 0;
  issue(0, 0);
  for (int slot = 0;; slot ^= 1) {
    const int tn = t + (int)gridDim.x;
    int bm_n = 0, bn_n = 0;
    const bool has_next = tn < ntile && tile_of(g, BM, nbm, nbn, bm_n, bn_n, tn, ntile);
    const int expert_n = (has_next && g.sorted_ids) ? block_expert(g, (int64_t)bm_n * BM) : 0;
    const int ncol0 = bn * OUT_COLS;
    int sid_n = 0;     // next tile: sorted id of row tid
    float rwv = 1.0f;  // this tile: route weight of row tid
    float biasv[BIAS_PER];
#pragma unroll
    for (int i = 0; i < BIAS_PER; ++i) biasv[i] = 0.f;
    // stage gk of the tile's buffer pair -> MFMAs
    auto math = [&]() {
      if constexpr (PRE)
        stage_math<T, FM, FN, true>(sA + (gk & 1) * S::A_STAGE, sB + (gk & 1) * S::B_STAGE,
                                    sS + (gk & 1) * S::S_SLOT, a_rd0, b_rd_pre, 0, s_rd_pre, acc);
      else
        stage_math<T, FM, FN, false>(sA + (gk & 1) * S::A_STAGE, sB + (gk & 1) * S::B_STAGE,
                                     sS + ((gk >> 1) & 1) * S::S_SLOT + (gk & 1) * 2, a_rd0, b_rd,
                                     b_sw, s_rd, acc);
    };
    // Every stage: wait until stage gk has landed (nothing later is in
    // flight), then a barrier publishes it and retires the reads of the
    // buffer the next issue overwrites.  The first and last stages are
    // peeled off so that the loop in between is the plain pipeline.
    // -- first stage: also the metadata loads consumed at the last one
    wait_vmcnt<0>();
    barrier_only();
    issue(1, gk + 1);
    if (tid < BM) {
      if (has_next && g.sorted_ids) sid_n = g.sorted_ids[(int64_t)bm_n * BM + tid];
      if (EPI == EPI_STORE && g.route_w) {
        const int o = t_orow(slot)[tid];
        rwv = o >= 0 ? g.route_w[o] : 0.f;
      }
    }
    if (EPI == EPI_STORE && g.bias) {
#pragma unroll
      for (int i = 0; i < BIAS_PER; ++i) {
        const int col = ncol0 + tid + i * NT;
        if (tid + i * NT < OUT_COLS && col < g.n)
          biasv[i] = to_f32(static_cast<const T*>(g.bias)[col]);
      }
    }
    // keep the fragment reads below the extra code (register pressure)
    __builtin_amdgcn_sched_barrier(0);
    math();
    ++gk;
    // -- stages 1 .. nk - 2
    for (int kt = 1; kt < nk - 1; ++kt, ++gk) {
      wait_vmcnt<0>();
      barrier_only();
      issue(kt + 1, gk + 1);
      math();
    }
    // -- last stage: tables (this tile's route weights and bias for its
    // epilogue, the next tile's rows for its loads), then the next tile's
    // first stage into the free buffer
    wait_vmcnt<0>();
    if (tid < BM) {
      t_rw(slot)[tid] = rwv;
      if (has_next) {
        int o, a;
        rows_of(bm_n, sid_n, o, a);
        t_orow(slot ^ 1)[tid] = o;
        t_arow(slot ^ 1)[tid] = a;
      }
    }
    if (EPI == EPI_STORE && g.bias) {
#pragma unroll
      for (int i = 0; i < BIAS_PER; ++i)
        if (tid + i * NT < OUT_COLS) t_bias(slot)[tid + i * NT] = biasv[i];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    barrier_only();
    if (has_next) {
      setup(bn_n, expert_n, slot ^ 1);
      issue(0, gk + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    math();
    ++gk;

    // ---- epilogue: lane holds rows fm*16 + c16, columns fn*16 + grp*4 ..
    // +3 of the wave's 16-column blocks; expert < 0 (not on this device)
    // writes zeros (aiter:156-172)
    float alpha = expert >= 0 ? scalar_alpha(g, expert) : 0.f;
    if constexpr (EPI == EPI_STORE) {
      if (g.ref_round && expert >= 0) {
        ref_pass<T>(g, expert, acc);
        alpha = 1.0f;
      }
    }
    // table reads first: the compiler does not move LDS reads across the
    // buffer stores
    uint32_t base[FM];
    float rw[FM];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int orow = t_orow(slot)[fm * 16 + c16];
      base[fm] = orow >= 0 ? (uint32_t)(orow * g.ldc * (int64_t)sizeof(T)) : kOOB;
      rw[fm] = (EPI == EPI_STORE && g.route_w) ? t_rw(slot)[fm * 16 + c16] : 1.0f;
    }
    float bv[EPI == EPI_STORE ? FN : 1][4];
    if (EPI == EPI_STORE) {
#pragma unroll
      for (int fn = 0; fn < (EPI == EPI_STORE ? FN : 1); ++fn)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          bv[fn][i] = g.bias ? t_bias(slot)[wave * FN * 16 + fn * 16 + grp * 4 + i] : 0.f;
    }
    // output fragments of 16 columns: FN for a plain store, FN / 2 for
    // SiLU*mul (gate fn, up fn + 1); outp packs values i, i + 1 of one
    constexpr int OF = (EPI == EPI_SILU_MUL) ? FN / 2 : FN;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      auto outp = [&](int j, int i) -> uint32_t {
        float o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if constexpr (EPI == EPI_SILU_MUL) {
            // vllm:249-252 on tensors of T (as in w4a16_pf)
            const T gb = from_f32<T>(acc[fm][2 * j][i + h] * alpha);
            const T ub = from_f32<T>(acc[fm][2 * j + 1][i + h] * alpha);
            const T sb = silu_round<T>(gb);
            o[h] = expert >= 0 ? to_f32(sb) * to_f32(ub) : 0.f;
          } else {
            o[h] = acc[fm][j][i + h] * alpha * rw[fm];
            if (g.bias) o[h] += bv[j < (EPI == EPI_STORE ? FN : 1) ? j : 0][i + h];
            if (expert < 0) o[h] = 0.f;
          }
        }
        return pack2<T>(o[0], o[1]);
      };
      auto offset = [&](int col) -> uint32_t {
        return (base[fm] != kOOB && col < g.n) ? base[fm] + col * (int)sizeof(T) : kOOB;
      };
      if (OF >= 2 && wide) {
        // lanes 16 apart trade fragment halves: each lane then holds 8
        // consecutive columns of fragment 2fp (even grp) or 2fp + 1 (odd)
#pragma unroll
        for (int fp = 0; fp < OF / 2; ++fp) {
          uint32_t pv[2], qv[2];
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            pv[w] = outp(2 * fp, 2 * w);
            qv[w] = outp(2 * fp + 1, 2 * w);
            const auto sw = __builtin_amdgcn_permlane16_swap(pv[w], qv[w], false, false);
            pv[w] = sw[0];
            qv[w] = sw[1];
          }
          const int col = ncol0 + wave * OF * 16 + (2 * fp + (grp & 1)) * 16 + (grp & 2) * 4;
          llvm_amdgcn_raw_buffer_store_v4i32(
              i32x4{(int)pv[0], (int)pv[1], (int)qv[0], (int)qv[1]}, rC, offset(col), 0, 0);
        }
        if constexpr (OF % 2 == 1) {
          const int col = ncol0 + wave * OF * 16 + (OF - 1) * 16 + grp * 4;
          llvm_amdgcn_raw_buffer_store_v2i32(i32x2{(int)outp(OF - 1, 0), (int)outp(OF - 1, 2)},
                                             rC, offset(col), 0, 0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < OF; ++j) {
          const int col = ncol0 + wave * OF * 16 + j * 16 + grp * 4;
          llvm_amdgcn_raw_buffer_store_v2i32(i32x2{(int)outp(j, 0), (int)outp(j, 2)}, rC,
                                             offset(col), 0, 0);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!has_next) break;
    t = tn;
    bm = bm_n;
    bn = bn_n;
    expert = expert_n;
  }
}

template <typename T, int WGM, int WGN, int FM, int FN, int STAGES, int EPI, int MINB, bool PRE,
          int BG = 1>
int launch_cfg(const GemmArgs& g, hipStream_t st) {
  typedef PfShape<WGM, WGN, FM, FN, STAGES, PRE> S;
  // weight-line groups where the configuration takes them (else per stage)
  constexpr int BGV = (BG > 1 && !PRE && EPI != EPI_PARTIAL && STAGES <= 3 && STAGES - 1 <= BG &&
                       (S::BN * 32 * BG / 1024) % S::NW == 0)
                          ? BG
                          : 1;
  const int out_cols = (EPI == EPI_SILU_MUL) ? S::BN / 2 : S::BN;
  const int nbn = (g.n + out_cols - 1) / out_cols;
  int64_t nbm = (g.m + S::BM - 1) / S::BM;
  if (g.sorted_ids) nbm = (nbm + 7) / 8 * 8;  // every XCD covers 1/8 of the capacity (tile_of)
  int64_t nwg = nbm * nbn;
  if (EPI == EPI_PARTIAL) nwg *= g.splitk;  // one workgroup per tile and K slice
  if (nwg <= 0 || nwg > 0x7FFFFFFF) {
    set_error("w4a16 prefill: bad grid");
    return MXFP4_ERR_VALUE;
  }
  if constexpr (BGV == 1 && EPI != EPI_PARTIAL && EPI != EPI_STORE_F32 && WGM == 1 &&
                WGN == 4 && STAGES == 2 && FN <= 4) {
    // routed grid of more tiles than resident workgroups: the persistent
    // kernel (dense grids run 2-5% slower in it: their tiles start with
    // one load round trip, not the routed two, and gain nothing)
    const int64_t c_bytes = g.num_valid * g.ldc * (int64_t)sizeof(T);
    if (g.sorted_ids && g.n % 4 == 0 && g.ldc % 4 == 0 && c_bytes < (int64_t)0x7FFFFFFF) {
      auto kern = w4a16_pp<T, FM, FN, EPI, MINB, PRE>;
      // same on every device of the build target; threads that race here
      // store the same value
      static std::atomic<int> per_cu_cache{-1};
      int per_cu = per_cu_cache.load(std::memory_order_relaxed);
      if (per_cu < 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, S::NT, 0) != hipSuccess) nb = 0;
        per_cu = nb;
        per_cu_cache.store(nb, std::memory_order_relaxed);
      }
      const int64_t slots = ((int64_t)per_cu * device_cus()) & ~(int64_t)7;
      if (slots >= 8 && nwg > slots) {
        kern<<<(unsigned)slots, S::NT, 0, st>>>(g, (int)nbm, nbn, (uint32_t)c_bytes);
        return launch_status("w4a16 persistent prefill launch");
      }
    }
  }
  w4a16_pf<T, WGM, WGN, FM, FN, STAGES, EPI, MINB, PRE, BGV><<<(unsigned)nwg, S::NT, 0, st>>>(
      g, (int)nbm, nbn);
  return launch_status("w4a16 prefill launch");
}

// Tile configurations (waves WGM x WGN, wave tile FM x FN MFMA blocks,
// stages, workgroups per CU).  Every configuration puts its waves side by
// side on columns (WGM = 1): a wave then spans all BM rows, so each decoded
// weight fragment feeds BM / 16 MFMAs and the per-MFMA decode work is the
// smallest the tile allows (+2-7% at 128 rows, +13-15% at 32-64 rows
// against 2 x 2 waves).  Measured at steady clocks on MI355X (bf16): the
// wide tiles 128 x 256 and 128 x 320 (waves of 128 x 64 / 128 x 80: per
// MFMA 1/2 and 2/5 of the activation LDS bytes of 128 x 128) run two
// workgroups per CU, so they pay off when their tiles fill whole rounds of
// the 512 slots: M = 8192 K = N = 4096 (1024 tiles of 128 x 256): 1310 vs
// 1212 TFLOP/s; M = K = N = 4096 (512): -6%; qkv M = 4096 (512 tiles of
// 128 x 320): -3%; M = 8192 K = 2048 N = 5120 (1024 of 128 x 320): -4%;
// MoE down at 4096 tokens: -3%.  With 640 tiles of 128 x 256 (qkv M =
// 4096) or 800 (N = 6400) they lose 4-6% to 128 x 128 (three per CU), and
// below 512 tiles more.  pf_choose takes the wide tile whose rounds are
// >= 80% full, else 128 x 128; 64 x 128 and 32 x 128 (3 stages) for mid M
// (M ~ 1024 and ~ 370, and MoE blocks of 64).
// Rejected: 128 x 256 with 8 waves of 128 x 32 (1150 vs 1183 TFLOP/s at
// M = 8192 K = N = 4096; MoE layer at 4096 tokens 496 vs 454 us); 256 x
// 160 and 256 x 128 of 2 x 2 waves (128 x 80 / 128 x 64: slower than the
// better of the two above at both sizes); 128 x 192 and 3-stage 128 x 256
// (slower at every size); 128 x 160 of 2 x 2 waves of 64 x 80 (no steady
// gain over M = 3072-6144 at qkv); 128 x 320, 256 x 256, 128 x 512, 192 x
// 256, 64 x 256/512, 32 x 256/512; 5 or 10 waves (a wave count that is not
// a multiple of the 4 SIMDs loads one SIMD twice); 3-4 stages at 128 rows
// (the extra LDS costs a workgroup per CU: -10-20% for the routed GEMMs);
// 4-8 stages at 32 x 128 and 5 at 64 x 128 (M = 256-1024: 0-15% slower);
// weights prefetched 2-4 stages ahead of the activations (no gain: the
// routed GEMMs wait on activation rows as much); two K-groups of 4 waves
// per 64 x 128 tile, each computing alternate 64-deep halves of 128-deep
// stages, partial sums added through LDS (8 waves for grids of ~1 tile per
// CU): qkv M = 370 / 512 / 768 only 2 / 4 / 5% faster, 32 x 128 and split-K
// shapes slower, and the summation order would differ between the
// prepacked and checkpoint layouts.
template <typename T, int EPI, bool PRE>
int launch_pf_typed(const GemmArgs& g, int cfg, hipStream_t st) {
  switch (cfg) {
    case PF_256x320:
      if constexpr (EPI == EPI_STORE) return launch_cfg<T, 2, 4, 8, 5, 2, EPI, 1, PRE>(g, st);
      else return launch_cfg<T, 1, 4, 8, 4, 2, EPI, 2, PRE>(g, st);  // (not chosen)
    case PF_256x256:
      if constexpr (EPI == EPI_STORE) return launch_cfg<T, 2, 4, 8, 4, 2, EPI, 1, PRE>(g, st);
      else return launch_cfg<T, 1, 4, 8, 4, 2, EPI, 2, PRE>(g, st);  // (not chosen)
    case PF_64x256: return launch_cfg<T, 1, 4, 4, 4, 3, EPI, 3, PRE>(g, st);
    case PF_32x256: return launch_cfg<T, 1, 4, 2, 4, 3, EPI, 4, PRE>(g, st);
    case PF_32x384: return launch_cfg<T, 1, 4, 2, 6, 2, EPI, 4, PRE>(g, st);
    case PF_32x512: return launch_cfg<T, 1, 4, 2, 8, 2, EPI, 3, PRE>(g, st);
    case PF_64x384: return launch_cfg<T, 1, 4, 4, 6, 2, EPI, 3, PRE>(g, st);
    case PF_128x320:
      if constexpr (EPI != EPI_SILU_MUL) return launch_cfg<T, 1, 4, 8, 5, 2, EPI, 2, PRE>(g, st);
      else return launch_cfg<T, 1, 4, 8, 4, 2, EPI, 2, PRE>(g, st);  // SiLU pairs need even FN
    case PF_128x256: return launch_cfg<T, 1, 4, 8, 4, 2, EPI, 2, PRE>(g, st);
    case PF_128x128: return launch_cfg<T, 1, 4, 8, 2, 2, EPI, 2, PRE>(g, st);
    case PF_64x128: return launch_cfg<T, 1, 4, 4, 2, 3, EPI, 4, PRE>(g, st);
    default: return launch_cfg<T, 1, 4, 2, 2, 3, EPI, 4, PRE>(g, st);
  }
}

// Checkpoint-layout weights in weight-line groups (a row's 32 bytes of BG
// stages in one piece: 1/BG of the L1 -> L2 requests for the weights, at
// 2 x BG x 32 bytes of LDS per weight row) where that measured faster, the
// same configurations as launch_pf_typed otherwise (bitwise the same
// results).  Measured (one job, eager loops, us, per-stage -> groups):
// 32 x 128 with 2-stage groups -- soft op (E=128, top-8, K=2048, N=1536)
// 64 / 128 / 256 / 384 tokens 53.4 / 54.7 / 56.7 / 63.0 -> 52.9 / 53.5 /
// 55.4 / 55.4, MoE layer 128 / 256 tokens 101.5 / 108.9 -> 94.5 / 99.5,
// AITER's entry with BLOCK_SIZE_M 32 at 512 tokens 66.1 -> 55.9 (4-stage
// groups: better at 64-256 tokens, 60.6 at 384; dense 32 x 128 lost: qkv
// K=2048 N=5120 M=370 15.7 -> 16.9); dense 64 x 128 with
// 2-stage groups -- qkv K=2048 N=5120 M=1024 30.6 -> 28.7 (routed 64 x 128
// lost: soft op 512 tokens 64.2 -> 66.9); dense 128 x 128 with 2-stage
// groups -- o_proj K=4096 N=2048 M=4096 63.8 -> 61.4, qkv M=2048 44.2 ->
// 43.5 (4-stage groups: 60.7 and 48.6); the one-round dense
// 256-row tiles with 4-stage groups -- qkv M=4096 / 8192 70.9 / 140.6 ->
// 69.8 / 138.0 (128 x 320 with 4-stage groups lost: one workgroup per CU,
// qkv M=8192 173.9).  Routed 32 x 256 with 2-stage groups: AITER's entry
// (BLOCK_SIZE_M 32, K=2048 N=1536) at 768 / 1024 tokens 79.9 / 97.0 ->
// 67.4 / 83.7; routed 64 x 128 as a 2-stage pipeline with 2-stage groups
// (four workgroups per CU; the 3-stage one with groups holds three and
// lost): 1024 tokens 87.3 -> 80.1, 512 / 768 tokens within 0.5.
template <typename T, int EPI>
int launch_pf_checkpoint(const GemmArgs& g, int cfg, hipStream_t st) {
  if constexpr (EPI != EPI_PARTIAL) {
    const bool dense = g.sorted_ids == nullptr;
    switch (cfg) {
      case PF_32x128:
        // 4-stage groups (128 bytes of each weight row per load) while the
        // experts average <= 20 routes; with more, the tiles of an expert
        // share its weights through the caches and the 2-stage groups' five
        // workgroups per CU (three with 4-stage ones) win.  Cold weights
        // (3 copies rotated, E=128, top-8, K=2048, N=1536): soft op at 128 /
        // 256 / 320 tokens 65.9 / 68.5 / 69.4 -> 60.0 / 62.2 / 63.1 us,
        // 384 70.98 vs 72.84 (kept 2-stage); MoE layer 128-320 tokens -5 us
        if (!dense) {
          if ((int64_t)g.num_valid <= 20 * (int64_t)g.num_experts)
            return launch_cfg<T, 1, 4, 2, 2, 3, EPI, 4, false, 4>(g, st);
          return launch_cfg<T, 1, 4, 2, 2, 3, EPI, 4, false, 2>(g, st);
        }
        break;
      case PF_32x256:
        if (!dense) return launch_cfg<T, 1, 4, 2, 4, 3, EPI, 3, false, 2>(g, st);
        break;
      case PF_64x128:
        if (dense) return launch_cfg<T, 1, 4, 4, 2, 3, EPI, 3, false, 2>(g, st);
        // routed: two stages in flight keep four workgroups per CU
        return launch_cfg<T, 1, 4, 4, 2, 2, EPI, 4, false, 2>(g, st);
      case PF_128x128:
        if (dense) return launch_cfg<T, 1, 4, 8, 2, 2, EPI, 2, false, 2>(g, st);
        break;
      case PF_256x320:
        if constexpr (EPI == EPI_STORE) return launch_cfg<T, 2, 4, 8, 5, 2, EPI, 1, false, 4>(g, st);
        break;
      case PF_256x256:
        if constexpr (EPI == EPI_STORE) return launch_cfg<T, 2, 4, 8, 4, 2, EPI, 1, false, 4>(g, st);
        break;
      default: break;
    }
  }
  return launch_pf_typed<T, EPI, false>(g, cfg, st);
}

template <typename T, int EPI>
int launch_pf_layout(const GemmArgs& g, int cfg, hipStream_t st) {
  if (!pf_prepacked_usable(g)) return launch_pf_checkpoint<T, EPI>(g, cfg, st);
  GemmArgs p = g;
  p.b = g.pre_b;
  p.bs = reinterpret_cast<const uint8_t*>(g.pre_s);
  p.b_e = g.pre_b_e;
  p.bs_e = g.pre_s_e;
  p.prepacked = 1;
  return launch_pf_typed<T, EPI, true>(p, cfg, st);
}

}  // namespace

// Compute units of the current device (cached per device).
int device_cus() {
  // per device; threads that race here store the same value
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

bool pf_supported(const GemmArgs& g, int elem_bytes) {
  if (g.k % 128 != 0 || g.k <= 0 || g.a_rows <= 0) return false;
  if ((reinterpret_cast<uintptr_t>(g.a) & 15) || (reinterpret_cast<uintptr_t>(g.b) & 15) ||
      (reinterpret_cast<uintptr_t>(g.bs) & 3) || (reinterpret_cast<uintptr_t>(g.c) & 15) ||
      ((g.lda * elem_bytes) & 15))
    return false;
  if (g.a_rows * g.lda * (int64_t)elem_bytes >= (int64_t)0x7FFFFFFF) return false;
  const int64_t brows = g.inter > 0 ? 2 * (int64_t)g.inter : (int64_t)g.n;
  if (brows * g.b_n >= (int64_t)0x7FFFFFFF) return false;
  return true;
}

bool pf_prepacked_usable(const GemmArgs& g) {
  if (g.pre_b == nullptr || g.pre_s == nullptr) return false;
  // 16-row groups must not straddle the gate / up halves
  if (g.inter > 0 && g.inter % 16 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(g.pre_b) & 15) || (reinterpret_cast<uintptr_t>(g.pre_s) & 15))
    return false;
  const int64_t brows = g.inter > 0 ? 2 * (int64_t)g.inter : (int64_t)g.n;
  return prepacked_nibble_bytes(brows, g.k) < (int64_t)0x7FFFFFFF &&
         prepacked_scale_bytes(brows, g.k) < (int64_t)0x7FFFFFFF;
}

int pf_choose(const GemmArgs& g, int epi) {
  const bool routed = g.sorted_ids != nullptr;
  auto allowed = [&](int bm) { return !routed || g.block_m % bm == 0; };
  auto tiles = [&](int bm, int bn) {
    const int out = epi == EPI_SILU_MUL ? bn / 2 : bn;
    return ((g.m + bm - 1) / bm) * (int64_t)((g.n + out - 1) / out);
  };
  // share of the 512 workgroup slots (two per CU) that a wide tile keeps
  // busy over all its rounds; 0 below one full round
  auto fill = [&](int bn) {
    const int64_t t = tiles(128, bn);
    const int64_t rounds = (t + 511) / 512;
    return t >= 512 ? (double)t / (double)(rounds * 512) : 0.0;
  };
  // One round of 256-row tiles (8 waves of 128 x 80 or 128 x 64, one
  // workgroup per CU): the CU's waves finish together instead of a CU's
  // second workgroup running its epilogue alone at the end.  Taken where
  // the round does >= 90% useful work (M x N over CUs x tile area; steady
  // clocks, prepacked: qkv M=4096 256 x 320 65.7 -> 64.6 us, M=4096 K=4096
  // N=5120 118.8 -> 115.9 us, M=K=N=4096 256 x 256 99.2 -> 97.3 us; at 80%,
  // 256 x 320 on M=K=N=4096 took 107.6 us; two rounds (M=8192) and 8 waves
  // of 128 x 32 (o_proj M=4096: 58.9 vs 56.2 us) lose)
  if (!routed && epi == EPI_STORE) {
    const int64_t cus = device_cus();
    const int cand[2][2] = {{PF_256x320, 320}, {PF_256x256, 256}};
    int best = -1;
    double best_eff = 0.9;
    for (int i = 0; i < 2 && cus > 0; ++i) {
      if (tiles(256, cand[i][1]) > cus) continue;
      const double eff = (double)g.m * (double)g.n / ((double)cus * 256.0 * cand[i][1]);
      if (eff >= best_eff) {
        best = cand[i][0];
        best_eff = eff;
      }
    }
    if (best >= 0) return best;
  }
  // Routed plain GEMMs on the checkpoint layout stage 32 bytes of every
  // weight row per 64-deep step (a cache line per row and step), so tiles
  // of few rows and many columns -- the prepacked layout's choices below --
  // spend their time on weight requests.  Measured (E=128, top-8, routed
  // GEMM alone, graph replays; K=2048 N=1536 / K=768 N=2048): 128-row
  // blocks take 128 x 256 (1024 tokens 80.2 / 52.3 vs 128 x 128 87.8 /
  // 51.3 us; 4096 tokens 235.9 / 146.5 vs 242.5 / 161.0); 32- and 64-row
  // blocks BM x 128 while those tiles number <= 10 per CU, else BM x 256
  // (512 tokens, 64-row blocks: 64 x 128 59.0 / 35.9 vs 64 x 256 66.9 /
  // 39.1; 32-row blocks: 32 x 128 67.7 vs 32 x 256 75.3 and 32 x 512
  // 117 us; 1024 tokens, down: 64 x 256 49.3 vs 64 x 128 51.9).
  // The SiLU GEMM of the MoE layer on the checkpoint layout: BM x 128 tiles
  // on 32- / 64-row blocks, 128 x 256 on 128-row ones (MoE layer, graph
  // replays: 512 tokens, 64-row blocks, 64 x 128 126.1 vs 64 x 384 140.6
  // us; 256 tokens, 32-row blocks, 32 x 128 108.8 vs 32 x 256 112.2; 1024
  // tokens, 128-row blocks, 128 x 256 160.2 vs 128 x 128 165.1)
  if (routed && epi == EPI_SILU_MUL && !pf_prepacked_usable(g)) {
    if (allowed(128)) return PF_128x256;
    return allowed(64) ? PF_64x128 : PF_32x128;
  }
  if (routed && epi == EPI_STORE && !pf_prepacked_usable(g)) {
    if (allowed(128)) return PF_128x256;
    const int bm = allowed(64) ? 64 : 32;
    const int64_t cus = device_cus();
    const int64_t busy = g.num_experts < g.num_valid ? g.num_experts : g.num_valid;
    const int64_t blocks = g.num_valid / bm + busy / 2;
    const int64_t t128 = blocks * ((g.n + 127) / 128);
    const bool narrow = cus <= 0 || t128 <= 10 * cus;
    if (bm == 64) return narrow ? PF_64x128 : PF_64x256;
    return narrow ? PF_32x128 : PF_32x256;
  }
  if (allowed(128)) {
    const double f256 = fill(256);
    const double f320 = epi == EPI_STORE ? fill(320) : 0.0;
    if (f320 >= 0.8 && f320 >= f256) return PF_128x320;
    if (f256 >= 0.8) return PF_128x256;
    // dense grids from 448 tiles, 7/8 of one round at two per CU (qkv K=2048
    // N=5120 M=1536, graph replays: 30.4 vs 33.7 us on 64 x 128; M=1024, 320
    // tiles: 27.7 vs 26.2)
    if (tiles(128, 128) >= (routed ? 512 : 448)) return PF_128x128;
  }
  // Routed 64-row blocks (MoE prefill at ~300-1300 tokens): 64 x 256 tiles,
  // which stream each expert's weights in half as many tiles (MoE layer,
  // prepacked, 512 tokens 107.6 -> 105.4 us, 1024 tokens 154.2 -> 144.3 us;
  // 2 stages lost 35-40%, 4 stages 2-3%; dense mid-M grids lose with it,
  // having too few tiles)
  // The SiLU GEMM of 64-row blocks takes 64 x 384 tiles of 2 stages (192
  // outputs; two thirds of the tiles, each of its activation rows read by
  // 4 column tiles instead of 6): 1024 tokens 135.4 -> 129.8 us, 2048
  // 206.4 -> 199.2, 4096 354.6 -> 347.0, 8192 646 -> 627 us; neutral at
  // 640-1280.  (For the plain GEMM, 64 x 384 / 64 x 512 were 3-10 us
  // slower at 768-1024 tokens and ~2% faster elsewhere: not taken.)
  if (routed && allowed(64)) return epi == EPI_SILU_MUL ? PF_64x384 : PF_64x256;
  // and routed 32-row blocks (~30-500 tokens) 32 x 256 (MoE layer,
  // prepacked, 3 stages: 256 tokens 86.8 -> 81.6 us, 320 tokens 90.5 ->
  // 83.1 us; 2 stages 84.4 / 86.2 us) -- unless that grid would spill past
  // one round of the 4 resident workgroups per CU: then wider 2-stage tiles
  // that fit in one (32 x 384 for the SiLU GEMM, 4 per CU; 32 x 512 for
  // the plain one, 3 per CU).  Expected live blocks: routes / 32 plus half
  // a block per busy expert.  MoE layer, graph replays over 3 weight copies:
  // 512 tokens 106.8 -> 99.4 us, 448 tokens 99.7 -> 98.5 us; the wider
  // tiles lose 2-3 us where 32 x 256 fits in one round (96-384 tokens).
  if (routed && allowed(32)) {
    const int64_t cus = device_cus();
    const int64_t busy = g.num_experts < g.num_valid ? g.num_experts : g.num_valid;
    const int64_t blocks = g.num_valid / 32 + busy / 2;
    const int out_cols = epi == EPI_SILU_MUL ? 128 : 256;
    const int64_t t256 = blocks * ((g.n + out_cols - 1) / out_cols);
    if (cus > 0 && t256 > 4 * cus) return epi == EPI_SILU_MUL ? PF_32x384 : PF_32x512;
    return PF_32x256;
  }
  // 64-row waves halve the decode work per MFMA of 32-row ones, and win
  // once their tiles fill the chip: from 384 of them (graph replays over
  // cold weight copies, prepacked, 64 x 128 vs 32 x 128 tiles: qkv K=2048
  // N=5120 M=370 (240 tiles) 15.75 vs 14.65 us, M=512 (320) 18.51 vs 17.47,
  // M=640 (400) 18.93 vs 21.51; o_proj K=4096 N=2048 M=1024 (256) 26.80 vs
  // 24.70, M=1536 (384) 31.90 vs 32.23, M=2048 (512) 35.32 vs 40.23)
  if (allowed(64) && tiles(64, 128) >= 384) return PF_64x128;
  return PF_32x128;
}

int launch_w4a16_pf(const GemmArgs& g, int dtype, int epi, int cfg, hipStream_t st) {
  if (dtype == MXFP4_DT_BF16) {
    switch (epi) {
      case EPI_STORE: return launch_pf_layout<__bf16, EPI_STORE>(g, cfg, st);
      case EPI_PARTIAL: return launch_pf_layout<__bf16, EPI_PARTIAL>(g, cfg, st);
      case EPI_STORE_F32: return launch_pf_layout<__bf16, EPI_STORE_F32>(g, cfg, st);
      default: return launch_pf_layout<__bf16, EPI_SILU_MUL>(g, cfg, st);
    }
  }
  if (epi == EPI_STORE_F32) {
    set_error("w4a16 prefill: C in FP32 takes bf16 activations only");
    return MXFP4_ERR_TYPE;
  }
  switch (epi) {
    case EPI_STORE: return launch_pf_layout<_Float16, EPI_STORE>(g, cfg, st);
    case EPI_PARTIAL: return launch_pf_layout<_Float16, EPI_PARTIAL>(g, cfg, st);
    default: return launch_pf_layout<_Float16, EPI_SILU_MUL>(g, cfg, st);
  }
}

// ---------------------------------------------------------------- split K
// Dense GEMMs with few row blocks (mid M, e.g. a 370-token prefill chunk)
// leave most CUs idle: o_proj M=370 has 192 tiles of 32 x 128 for 256 CUs,
// each walking 64 stages of K.  Splitting K into S slices gives S times the
// workgroups (each of K / S), at the price of writing and re-reading
// S x M x N FP32 partial sums; splitk_reduce adds them in slice order
// (deterministic), applies the bias and rounds once.

namespace {

template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ ws, int splits,
                                                     int64_t m, int n, const T* __restrict__ bias,
                                                     T* __restrict__ out, int64_t ldc) {
  const int nq = (n + 3) / 4;
  const int64_t total = m * nq;
  const int64_t plane = m * (int64_t)n;
  const bool vec = (n & 3) == 0;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / nq;
    const int c = (int)(i % nq) * 4;
    const float* src = ws + row * n + c;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    if (vec) {
      for (int sl = 0; sl < splits; ++sl) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(src + sl * plane);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] += v[j];
      }
    } else {
      for (int sl = 0; sl < splits; ++sl)
        for (int j = 0; j < 4 && c + j < n; ++j) o[j] += src[sl * plane + j];
    }
    T* dst = out + row * ldc + c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (c + j >= n) break;
      float v = o[j];
      if (bias) v += to_f32(bias[c + j]);
      dst[j] = from_f32<T>(v);
    }
  }
}

}  // namespace

SplitPlan splitk_plan(int64_t m, int64_t k, int64_t n) {
  // Only where even 32-row tiles would leave CUs idle, and K is long (>= 64
  // stages) or the tiles very few: with 32 stages, qkv-sized grids (K=2048,
  // N=5120, M=96-128) run slower split (12.9 -> 15.9 us at M=128).  Tiles
  // of 32 rows up to M = 256, 64 above; slices double until the grid
  // reaches 384 workgroups, at most 8 slices of at least 16 stages each (8
  // while the grid is under 128 workgroups) (steady clocks, bf16, unsplit
  // -> split: o_proj K=4096 N=2048 M=128 / 200 / 256 / 370: 22.4 / 22.5 /
  // 22.5 / 22.6 -> 12.6 / 15.6 / 16.8 / 20.3 us; M=130 K=8192 N=640: 43.5
  // -> 13.4 us; M=64 K=2048 N=1536: 13.1 -> 10.4 us).
  // Long K (>= 64 stages) splits while the 32-row tiles number under 384
  // (o_proj M=512, 256 tiles: 2 slices 20.4-21.0 vs 22.7 us; M=640: 22.8 vs
  // 23.9; M=768, 384 tiles: 24.0 vs 24.0).
  SplitPlan p{m <= 256 ? PF_32x128 : PF_64x128, 1};
  const int64_t tiles32 = ((m + 31) / 32) * ((n + 127) / 128);
  if (tiles32 >= 384 || (k < 4096 && tiles32 >= 64)) return p;
  const int bm = m <= 256 ? 32 : 64;
  const int64_t tiles = ((m + bm - 1) / bm) * ((n + 127) / 128);
  const int64_t nk = k / 64;
  int s = 1;
  while (tiles * s < 384 && s < 8 && nk / (2 * s) >= (tiles * s < 128 ? 8 : 16)) s *= 2;
  p.splits = s;
  return p;
}

int64_t splitk_ws_bytes(int64_t m, int64_t k, int64_t n) {
  if (dense_skinny_rows(m, k, n, true)) return 0;  // the skinny kernel needs none
  const SplitPlan p = splitk_plan(m, k, n);
  return p.splits > 1 ? (int64_t)p.splits * m * n * (int64_t)sizeof(float) : 0;
}

int launch_splitk_reduce(const GemmArgs& g, int dtype, hipStream_t st) {
  const int64_t total = g.m * ((g.n + 3) / 4);
  const int64_t blocks = (total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192;
  if (dtype == MXFP4_DT_BF16)
    splitk_reduce<__bf16><<<(unsigned)blocks, 256, 0, st>>>(
        g.splitk_ws, g.splitk, g.m, g.n, static_cast<const __bf16*>(g.bias),
        static_cast<__bf16*>(g.c), g.ldc);
  else
    splitk_reduce<_Float16><<<(unsigned)blocks, 256, 0, st>>>(
        g.splitk_ws, g.splitk, g.m, g.n, static_cast<const _Float16*>(g.bias),
        static_cast<_Float16*>(g.c), g.ldc);
  return launch_status("split-K reduce launch");
}

}  // namespace mx
