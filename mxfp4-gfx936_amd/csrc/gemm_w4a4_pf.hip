// W4A4 GEMM, direct-to-LDS pipeline (gfx950): packed MXFP4 activations x
// packed MXFP4 weights on the block-scaled MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4, both operands E2M1).  Same semantics
// as w4a4_tiled (aiter:206-214 + 329-338; soft:468-471, 487-490): every
// E2M1 x E2M1 product times its two power-of-two scales is exact, FP32
// accumulation, scales / route weights on the FP32 accumulator, one
// rounding to the output type.
//
// Tile BM x BN (activation rows x weight rows), WGM x WGN waves of FM x FN
// MFMA blocks, K in 128 x KS-deep stages (KS MFMA steps each).  Feeding FP4 MFMAs takes 4x the bytes
// per FLOP of BF16 ones, so the tile is as large as the registers allow
// (256 x 256 with 8 waves of 128 x 64, 3 stages) and everything moves
// global -> LDS with `buffer_load_dwordx4 ... lds` (16 bytes per lane at LDS
// base + 16 x lane; out-of-range offsets read zero, so padding rows and
// partial tiles need no branches):
//
// * A and B stages hold 64 x KS-byte rows (128 x KS E2M1 codes), written by
//   1 KB wave-loads of 16 / KS rows; the MFMA fragment of lane l at step h
//   (row l % 16, K h*128 + (l/16)*32 .. +32) is the 16-byte chunk
//   h*4 + l/16 of its row.  With KS = 1 a wave reads one contiguous KB per
//   fragment.  With KS = 2 a row's stage is its whole 128-byte line (one
//   request instead of two half-line ones) and chunk c of row r sits in
//   slot c ^ ((r / 2) % 8): the lane that fills a slot loads the chunk
//   that belongs there, so the 16 rows of a fragment read cover all 64
//   banks.
// * Scales are staged SQ stages at a time: the 4 x SQ E8M0 bytes of a row
//   (one per 32-block) are 4 x SQ contiguous bytes of its scale row, loaded
//   by 4 x SQ-byte-per-lane wave-loads of 64 rows.  A row's stage uses only 4
//   bytes of its 128-byte scale line, so SQ = 4 (16 bytes per lane, one
//   request per row every 4 stages) quarters the scale requests of SQ = 1,
//   which at 8192 x 4096 x 4096 are as many as the A and B requests
//   together.  Lane l reads byte l/16 of its row's stage dword into byte 0
//   of its scale operand.
// * The MFMA takes the weights as its A operand and the activations as its
//   B operand, so a lane owns 4 consecutive output columns of one row; the
//   epilogue stages the finished tile in LDS and writes 16-byte chunks.
//
// * FP8 activations (AF = 0 E4M3 / 1 E5M2, aiter:11-20): A rows are K
//   bytes, so a stage holds 128 x KS bytes of each A row; the fragment of
//   lane l at step h is two chunks, K h*128 + (l/16)*16 .. +16 and h*128 +
//   64 + (l/16)*16 .. +16 (the FP8 operand layout of the 16x16x128 MFMA), in
//   slots swizzled by row so the 16 rows of a read cover all banks.  A
//   missing A scale (FP8 without A_mx_scale) is the constant 127 (1.0).
//
// Requirements (else the register-staged w4a4_tiled runs): K % 128 == 0,
// 16-byte aligned A / B rows and scale rows 4-byte aligned, operands below
// 2 GiB.
#include "gemm.h"

namespace mx {
namespace {

template <int WGM, int WGN, int FM, int FN, int STAGES, int SQ, int KS, int AF = 4>
struct P4Shape {
  static constexpr int NW = WGM * WGN;
  static constexpr int NT = 64 * NW;
  static constexpr int BM = WGM * FM * 16;
  static constexpr int BN = WGN * FN * 16;
  static constexpr int RB = 64 * KS;  // bytes of a (packed) row's stage
  static constexpr int RBA = (AF == 4 ? 64 : 128) * KS;  // bytes of an A row's stage
  static constexpr int A_STAGE = BM * RBA;
  static constexpr int B_STAGE = BN * RB;
  static constexpr int A_TOT = A_STAGE / 1024;  // 1 KB wave-loads per stage
  static constexpr int B_TOT = B_STAGE / 1024;
  static constexpr int SA_TOT = (BM + 63) / 64;  // 64-row scale wave-loads
  static constexpr int SB_TOT = (BN + 63) / 64;
  static constexpr int SA_BUF = SA_TOT * 256 * SQ;  // bytes per scale buffer
  static constexpr int SB_BUF = SB_TOT * 256 * SQ;
  static constexpr int A_PER = (A_TOT + NW - 1) / NW;
  static constexpr int B_PER = (B_TOT + NW - 1) / NW;
  static constexpr int S_PER = (SA_TOT + SB_TOT + NW - 1) / NW;
  static constexpr int STAGE = A_STAGE + B_STAGE;
  // scales of SQ MFMA steps per buffer: one buffer per stage (SQ = KS) or
  // two alternating ones (SQ > KS: the buffer of steps s .. s + SQ - 1 is
  // refilled with the loads of the stage holding step s, SQ / KS >=
  // STAGES - 1 stages after its previous occupant's last use)
  static constexpr int SBUFS = SQ == KS ? STAGES : 2;
  static constexpr int SC_BASE = STAGES * STAGE;
  static constexpr int PIPE = SC_BASE + SBUFS * (SA_BUF + SB_BUF);
};

template <typename TO, int WGM, int WGN, int FM, int FN, int STAGES, int MINB, int SQ, int KS,
          int AF>
__global__ __launch_bounds__(64 * WGM * WGN, MINB) void w4a4_pf(GemmArgs g, int nbm, int nbn) {
  typedef P4Shape<WGM, WGN, FM, FN, STAGES, SQ, KS, AF> S;
  constexpr int BM = S::BM, BN = S::BN, NT = S::NT;
  static_assert(FN % 2 == 0, "2-byte outputs pair the column blocks");
  static_assert(STAGES >= 2 && STAGES <= 4, "2 to 4 stages");
  static_assert((KS == 1 || KS == 2) && SQ % KS == 0 && (SQ == KS || SQ / KS >= STAGES - 1),
                "scale buffers cover whole stages and outlive the pipeline");
  static_assert(SQ == KS || STAGES <= 3, "grouped scales: at most one scale issue in flight");
  static_assert(STAGES == 2 || (S::A_TOT % S::NW == 0 && S::B_TOT % S::NW == 0 &&
                                (S::SA_TOT + S::SB_TOT) % S::NW == 0),
                "deeper pipelines count the same loads on every wave");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S::PIPE];

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
  // FP8 A without scales: the scale loads read nothing (offsets past an
  // empty range of the weight scales) and the operand is 127
  const bool amx = g.a_mx != nullptr;
  const i32x4 rSA = amx ? make_rsrc(g.a_mx, (uint32_t)(g.a_rows * g.lda_mx)) : make_rsrc(g.bs, 0u);
  const i32x4 rB = make_rsrc(g.b + expert * g.b_e, (uint32_t)((int64_t)g.n * g.b_n));
  const i32x4 rSB = make_rsrc(g.bs + expert * g.bs_e, (uint32_t)((int64_t)g.n * g.bs_n));

  // per-lane offsets for stage 0 (stage kt adds kt * RB / kt * 4 * KS as
  // the scalar offset); wave-load q of a stage is issued by wave q % NW;
  // lane l fills slot l % (4 KS) of tile row q * 16 / KS + l / (4 KS)
  constexpr int CPR = 4 * KS;        // 16-byte chunks per packed row stage
  constexpr int CPRA = S::RBA / 16;  // ... per A row stage
  // slot <-> chunk of a row's stage (an involution): rows of 4 chunks
  // unswizzled, of 8 XOR (row / 2) % 8, of 16 XOR row % 16
  auto swz = [&](int cpr, int trow) {
    return cpr == 4 ? 0 : (cpr == 8 ? (trow >> 1) & 7 : trow & 15);
  };
  auto chunk_of = [&](int trow) { return (lane % CPR) ^ swz(CPR, trow); };
  uint32_t a_off[S::A_PER];
#pragma unroll
  for (int j = 0; j < S::A_PER; ++j) {
    const int q = j * S::NW + wave;
    const int row = q * (64 / CPRA) + lane / CPRA;
    a_off[j] = kOOB;
    if (q < S::A_TOT) {
      const RowInfo ri = row_info(g, pos0 + row);
      if (ri.valid)
        a_off[j] = (uint32_t)(ri.a_row * g.lda) + ((lane % CPRA) ^ swz(CPRA, row)) * 16;
    }
  }
  uint32_t b_off[S::B_PER];
#pragma unroll
  for (int j = 0; j < S::B_PER; ++j) {
    const int q = j * S::NW + wave;
    const int trow = q * (16 / KS) + lane / CPR;
    const int row = ncol0 + trow;
    b_off[j] = (q < S::B_TOT && row < g.n) ? (uint32_t)(row * g.b_n) + chunk_of(trow) * 16 : kOOB;
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
      if (row < BM && amx) {
        const RowInfo ri = row_info(g, pos0 + row);
        if (ri.valid) s_off[j] = (uint32_t)(ri.a_row * g.lda_mx);
      }
    } else if (q < S::SA_TOT + S::SB_TOT) {
      const int row = (q - S::SA_TOT) * 64 + lane;
      if (row < BN && ncol0 + row < g.n) s_off[j] = (uint32_t)((ncol0 + row) * g.bs_n);
    }
  }

  const int nk = g.k / (128 * KS);
  auto issue = [&](int kt) {
    uint8_t* base = smem + (kt % STAGES) * S::STAGE;
    uint8_t* sbase = smem + S::SC_BASE + ((kt * KS / SQ) % S::SBUFS) * (S::SA_BUF + S::SB_BUF);
#pragma unroll
    for (int j = 0; j < S::A_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::A_TOT % S::NW == 0 || q < S::A_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rA, lds_ptr(base + q * 1024), 16, (int)a_off[j],
                                        kt * S::RBA, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < S::B_PER; ++j) {
      const int q = j * S::NW + wave;
      if (S::B_TOT % S::NW == 0 || q < S::B_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rB, lds_ptr(base + S::A_STAGE + q * 1024), 16,
                                        (int)b_off[j], kt * S::RB, 0, 0);
    }
    if ((kt * KS) % SQ != 0) return;
#pragma unroll
    for (int j = 0; j < S::S_PER; ++j) {
      const int q = j * S::NW + wave;
      // A and B scale slots are contiguous: slot q at sbase + q * 256 * SQ
      if (q < S::SA_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rSA, lds_ptr(sbase + q * 256 * SQ), 4 * SQ,
                                        (int)s_off[j], kt * 4 * KS, 0, 0);
      else if (q < S::SA_TOT + S::SB_TOT)
        llvm_amdgcn_raw_buffer_load_lds(rSB, lds_ptr(sbase + q * 256 * SQ), 4 * SQ,
                                        (int)s_off[j], kt * 4 * KS, 0, 0);
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // lane reads: activation fragment fm = rows wm*FM*16 + fm*16 + c16, chunk
  // h*4 + grp (in its slot); weight fragment fn likewise; scale bytes grp of
  // those rows.  The slot swizzle depends on the row only through c16.
  auto slot_of = [&](int h) { return KS == 1 ? grp : (h * 4 + grp) ^ ((c16 >> 1) & 7); };
  // FP8 A: chunks h*8 + grp and h*8 + 4 + grp (swizzled by the fragment row,
  // which differs from c16 by a multiple of 16)
  auto slot_a = [&](int chunk) { return chunk ^ swz(CPRA, c16); };
  const int a_rd = (wm * FM * 16 + c16) * S::RBA;
  const int b_rd = (wn * FN * 16 + c16) * S::RB;
  const int sa_rd = (wm * FM * 16 + c16) * 4 * SQ + grp;
  const int sb_rd = (wn * FN * 16 + c16) * 4 * SQ + grp;

#pragma unroll
  // the stage waits count loads per stage in issue order: a compiler fence
  // after each prologue stage keeps stage s + 1's loads behind stage s's
  for (int s = 0; s < STAGES - 1; ++s) {
    if (s < nk) issue(s);
    asm volatile("" ::: "memory");
  }
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt has landed once at most the later stages' loads of this wave
    // are outstanding (AB each, plus S_PER scale loads on stages whose first
    // step is a multiple of SQ); the barrier publishes it and retires the
    // reads of the buffers issue() refills
    constexpr int AB = S::A_PER + S::B_PER;
    const int later = (nk - 1 - kt) < (STAGES - 2) ? (nk - 1 - kt) : (STAGES - 2);
    if (STAGES >= 4 && later >= 2) {
      wait_vmcnt<2 * (AB + S::S_PER)>();  // SQ == 1 only
    } else if (STAGES >= 3 && later >= 1) {
      if (((kt + 1) * KS) % SQ == 0) wait_vmcnt<AB + S::S_PER>();
      else wait_vmcnt<AB>();
    } else {
      wait_vmcnt<0>();
    }
    barrier_only();
    if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
    const uint8_t* base = smem + (kt % STAGES) * S::STAGE;
    const uint8_t* As = base;
    const uint8_t* Bs = base + S::A_STAGE;
#pragma unroll
    for (int h = 0; h < KS; ++h) {
      const int step = kt * KS + h;
      const uint8_t* Sa = smem + S::SC_BASE +
                          ((step / SQ) % S::SBUFS) * (S::SA_BUF + S::SB_BUF) + (step % SQ) * 4;
      const uint8_t* Sb = Sa + S::SA_BUF;
      const int slot = slot_of(h) * 16;
      i32x8 af[FM];
      int asc[FM];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        if constexpr (AF == 4) {
          const i32x4 v = *reinterpret_cast<const i32x4*>(As + a_rd + slot + fm * 16 * S::RBA);
          af[fm] = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
        } else {
          const uint8_t* ar = As + a_rd + fm * 16 * S::RBA;
          const i32x4 v = *reinterpret_cast<const i32x4*>(ar + slot_a(h * 8 + grp) * 16);
          const i32x4 w = *reinterpret_cast<const i32x4*>(ar + slot_a(h * 8 + 4 + grp) * 16);
          af[fm] = i32x8{v[0], v[1], v[2], v[3], w[0], w[1], w[2], w[3]};
        }
        asc[fm] = amx ? (int)Sa[sa_rd + fm * 16 * 4 * SQ] : 127;
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const i32x4 v = *reinterpret_cast<const i32x4*>(Bs + b_rd + slot + fn * 16 * S::RB);
        const i32x8 bf = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
        const int bsc = Sb[sb_rd + fn * 16 * 4 * SQ];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          acc[fm][fn] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bf, af[fm], acc[fm][fn], 4, AF, 0, bsc, 0, asc[fm]);
      }
    }
  }

  // ---- epilogue, straight from registers: lane holds rows
  // wm*FM*16 + fm*16 + c16, columns wn*FN*16 + fn*16 + grp*4 .. +3.  For
  // 2-byte outputs the lane pairs (grp 0, 1) and (2, 3) trade halves with
  // v_permlane16_swap so that each lane holds 8 consecutive columns of one
  // block (even grp: block 2p, odd grp: block 2p + 1) and writes 16 bytes;
  // a store instruction then covers 64 contiguous bytes of 16 rows.  No LDS
  // staging and no barrier: the tile ends with its stores in flight.
  float alpha = scalar_alpha(g, expert);
  if (g.ref_round) {
    ref_pass<TO>(g, expert, acc);
    alpha = 1.0f;
  }
  const bool vec = (g.ldc % (16 / (int)sizeof(TO))) == 0;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int trow = wm * FM * 16 + fm * 16 + c16;
    const RowInfo r = row_info(g, pos0 + trow);
    float rw = 1.0f;
    if (g.route_w) rw = r.valid ? g.route_w[r.out_row] : 0.f;
    const float sc = alpha * rw;
    TO* const crow = static_cast<TO*>(g.c) + (r.valid ? r.out_row : 0) * g.ldc;
    if constexpr (sizeof(TO) == 4) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = ncol0 + wn * FN * 16 + fn * 16 + grp * 4;
        const f32x4 o = f32x4{acc[fm][fn][0] * sc, acc[fm][fn][1] * sc, acc[fm][fn][2] * sc,
                              acc[fm][fn][3] * sc};
        if (!r.valid || col >= g.n) continue;
        if (vec && col + 4 <= g.n) {
          *reinterpret_cast<f32x4*>(crow + col) = o;
        } else {
          for (int i = 0; i < 4 && col + i < g.n; ++i) crow[col + i] = o[i];
        }
      }
    } else {
#pragma unroll
      for (int fp = 0; fp < FN / 2; ++fp) {
        uint32_t p[2], q[2];  // p: block 2fp, q: block 2fp + 1 (4 columns each)
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const TO a0 = from_f32<TO>(acc[fm][2 * fp][2 * w] * sc);
          const TO a1 = from_f32<TO>(acc[fm][2 * fp][2 * w + 1] * sc);
          const TO b0 = from_f32<TO>(acc[fm][2 * fp + 1][2 * w] * sc);
          const TO b1 = from_f32<TO>(acc[fm][2 * fp + 1][2 * w + 1] * sc);
          p[w] = (uint32_t)__builtin_bit_cast(uint16_t, a0) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, a1) << 16);
          q[w] = (uint32_t)__builtin_bit_cast(uint16_t, b0) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, b1) << 16);
          // odd grp lanes take p from the even partner's q; even lanes take
          // q from the odd partner's p
          const auto sw = __builtin_amdgcn_permlane16_swap(p[w], q[w], false, false);
          p[w] = sw[0];
          q[w] = sw[1];
        }
        // even grp: columns grp*4 .. +7 of block 2fp; odd grp: columns
        // (grp - 1)*4 .. +7 of block 2fp + 1
        const int col = ncol0 + wn * FN * 16 + (2 * fp + (grp & 1)) * 16 + (grp & 2) * 4;
        if (!r.valid || col >= g.n) continue;
        const uint32_t v[4] = {p[0], p[1], q[0], q[1]};
        if (vec && col + 8 <= g.n) {
          *reinterpret_cast<i32x4*>(crow + col) =
              i32x4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
        } else {
          for (int i = 0; i < 8 && col + i < g.n; ++i)
            crow[col + i] = __builtin_bit_cast(TO, (uint16_t)(v[i / 2] >> (16 * (i & 1))));
        }
      }
    }
  }
}

// STAGES1: stages of the per-stage-scale kernel; STAGES4 x KS4: stages and
// steps per stage of the grouped-scale kernel; AF: activation format
template <typename TO, int AF, int WGM, int WGN, int FM, int FN, int MINB, int STAGES1, int STAGES4,
          int KS4>
int launch_cfg(const GemmArgs& g, hipStream_t st) {
  typedef P4Shape<WGM, WGN, FM, FN, STAGES1, 1, 1, AF> S;
  const int nbn = (g.n + S::BN - 1) / S::BN;
  int64_t nbm = (g.m + S::BM - 1) / S::BM;
  if (g.sorted_ids) nbm = (nbm + 7) / 8 * 8;  // every XCD covers 1/8 of the capacity (tile_of)
  const int64_t nwg = nbm * nbn;
  if (nwg <= 0 || nwg > 0x7FFFFFFF) {
    set_error("w4a4 prefill: bad grid");
    return MXFP4_ERR_VALUE;
  }
  // 16-byte scale groups: whole groups of aligned rows (K % 512 == 0)
  const bool amx_ok = g.a_mx == nullptr ||
                      (g.lda_mx % 16 == 0 && !(reinterpret_cast<uintptr_t>(g.a_mx) & 15));
  const bool sq4 = g.k % 512 == 0 && amx_ok && g.bs_n % 16 == 0 &&
                   !(reinterpret_cast<uintptr_t>(g.bs) & 15) && g.bs_e % 16 == 0;
  if (sq4)
    w4a4_pf<TO, WGM, WGN, FM, FN, STAGES4, MINB, 4, KS4, AF>
        <<<(unsigned)nwg, S::NT, 0, st>>>(g, (int)nbm, nbn);
  else
    w4a4_pf<TO, WGM, WGN, FM, FN, STAGES1, MINB, 1, 1, AF>
        <<<(unsigned)nwg, S::NT, 0, st>>>(g, (int)nbm, nbn);
  return launch_status("w4a4 prefill launch");
}

template <typename TO, int AF>
int launch_typed(const GemmArgs& g, int cfg, hipStream_t st) {
  if constexpr (AF != 4) {
    // FP8 activations: A rows twice the bytes, 128-deep stages (LDS of
    // 256 x 256: 3 x (32 + 16) KB + 16 KB of scales)
    switch (cfg) {
      case P4_256x256: return launch_cfg<TO, AF, 2, 4, 8, 4, 1, 3, 3, 1>(g, st);
      case P4_128x128: return launch_cfg<TO, AF, 1, 4, 8, 2, 2, 3, 3, 1>(g, st);
      case P4_32x128: return launch_cfg<TO, AF, 1, 4, 2, 2, 4, 2, 2, 1>(g, st);
      default: return launch_cfg<TO, AF, 1, 4, 4, 2, 2, 2, 2, 1>(g, st);  // P4_64x128
    }
  } else {
    // Measured (8192 x 4096 x 4096, bf16 out): 2 x 4 waves of 128 x 64,
    // grouped scales, 2 stages of 256 ~3.5-3.6 PFLOP/s (8192^3: 4.07), 3
    // stages of 128 ~3.2 (3.56); per-stage scales, 3 stages of 128 ~3.0;
    // 2 x 2 waves of 128 x 128 (one wave per SIMD) ~2.3-2.6; 16 waves of
    // 128 x 64 (256 x 512) does not fit the register file.  128 x 128 tiles
    // at M = 2048, K = N = 4096: 256-deep stages 2.56 vs 2.23 PFLOP/s.
    switch (cfg) {
      case P4_256x256: return launch_cfg<TO, 4, 2, 4, 8, 4, 1, 3, 2, 2>(g, st);
      case P4_128x128: return launch_cfg<TO, 4, 1, 4, 8, 2, 2, 2, 2, 2>(g, st);
      case P4_32x128: return launch_cfg<TO, 4, 1, 4, 2, 2, 4, 2, 2, 1>(g, st);
      default: return launch_cfg<TO, 4, 1, 4, 4, 2, 2, 2, 2, 1>(g, st);  // P4_64x128
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
  // 256 x 256 needs a tile for every CU (steady clocks, bf16 out: 2.99 vs
  // 2.06 PFLOP/s at M = 8192 K = N = 4096 with 512 tiles; with 160 tiles,
  // M = 2048 K = 2048 N = 5120, 128 x 128 wins 1.69 vs 1.59).
  (void)out_dtype;
  if (allowed(256) && tiles(256, 256) >= 256) return P4_256x256;
  if (allowed(128) && tiles(128, 128) >= 128) return P4_128x128;
  if (allowed(64)) return P4_64x128;
  // routed 32-row blocks (the register-staged kernel took them before)
  if (allowed(32)) return P4_32x128;
  return -1;
}

template <int AF>
int launch_out(const GemmArgs& g, int out_dtype, int cfg, hipStream_t st) {
  switch (out_dtype) {
    case MXFP4_DT_BF16: return launch_typed<__bf16, AF>(g, cfg, st);
    case MXFP4_DT_F16: return launch_typed<_Float16, AF>(g, cfg, st);
    default: return launch_typed<float, AF>(g, cfg, st);
  }
}

int launch_w4a4_pf(const GemmArgs& g, int out_dtype, int cfg, hipStream_t st) {
  switch (g.a_fp8) {
    case 1: return launch_out<0>(g, out_dtype, cfg, st);
    case 2: return launch_out<1>(g, out_dtype, cfg, st);
    default: return launch_out<4>(g, out_dtype, cfg, st);
  }
}

}  // namespace mx
