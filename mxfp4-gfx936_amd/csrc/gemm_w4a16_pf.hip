// W4A16 prefill GEMM, direct-to-LDS pipeline (gfx950).
//
// Tile BM x BN (output rows x weight rows), 256 threads = 2 x 2 waves, each
// wave FM x FN MFMA blocks of 16x16, K in 64-deep stages:
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
//   A wave tile of 64 x 128 reads 192 LDS bytes per MFMA (vs 320 at 64 x 64).
// * Epilogue.  Scales / route weight / bias / SiLU*mul are applied in
//   registers, the tile is staged in LDS (reusing the stage buffers) and
//   written back as full 16-byte chunks, whole output rows per instruction.
// * Order.  Tiles are remapped so each XCD (workgroups are dealt round-robin
//   over the 8 XCDs) gets a contiguous range, walked in groups of 4 row
//   blocks, keeping each XCD's A rows and B columns L2-resident.
//
// Requirements (else the host falls back to the register-staged kernel):
// K % 128 == 0; activation and weight byte ranges below 2 GiB; 16-byte
// aligned A / B rows and 4-byte aligned scale rows.
#include "gemm.h"

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

template <int FM, int FN, int STAGES>
struct PfShape {
  static constexpr int BM = 2 * FM * 16;
  static constexpr int BN = 2 * FN * 16;
  static constexpr int A_STAGE = BM * 128;  // BM rows x 64 elements x 2 bytes
  static constexpr int B_STAGE = BN * 32;   // BN rows x 64 nibbles
  static constexpr int S_SLOT = BN * 4;     // 4 scale bytes (128 K) per row
  static constexpr int A_LOADS = BM / 32;   // 1 KB wave-loads per wave per stage
  static constexpr int B_LOADS = BN / 128;
  static constexpr int S_WAVES = BN / 64;   // waves that load a scale slot (64 rows each)
  static constexpr int PIPE = STAGES * (A_STAGE + B_STAGE) + 2 * S_SLOT;
};

template <typename T, int FM, int FN, int STAGES, int EPI, int MINB>
__global__ __launch_bounds__(256, MINB) void w4a16_pf(GemmArgs g, int nbm, int nbn) {
  typedef typename V8Of<T>::type V8;
  typedef PfShape<FM, FN, STAGES> S;
  constexpr int BM = S::BM, BN = S::BN;
  constexpr int OUT_COLS = (EPI == EPI_SILU_MUL) ? BN / 2 : BN;
  constexpr int C_LD = OUT_COLS * 2 + 16;  // bytes per staged output row
  constexpr int SMEM = S::PIPE > BM * C_LD ? S::PIPE : BM * C_LD;
  static_assert(S::S_WAVES <= 4 && BN % 128 == 0, "tile config");
  static_assert(EPI != EPI_SILU_MUL || FN % 2 == 0, "SiLU pairs need even FN");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  uint8_t* const sA = smem;
  uint8_t* const sB = smem + STAGES * S::A_STAGE;
  uint8_t* const sS = smem + STAGES * (S::A_STAGE + S::B_STAGE);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int c16 = lane & 15;
  const int grp = lane >> 4;

  // ---- tile order: XCD-contiguous ranges, groups of 4 row blocks
  int pid = blockIdx.x;
  {
    const int nwg = gridDim.x, per = nwg / 8, rem = nwg % 8, x = pid % 8, i = pid / 8;
    pid = x * per + (x < rem ? x : rem) + i;
  }
  constexpr int GROUP = 4;
  const int first_m = (pid / (GROUP * nbn)) * GROUP;
  const int gsize = (nbm - first_m) < GROUP ? (nbm - first_m) : GROUP;
  const int bm = first_m + (pid % (GROUP * nbn)) % gsize;
  const int bn = (pid % (GROUP * nbn)) / gsize;

  const int64_t pos0 = (int64_t)bm * BM;
  if (pos0 >= rows_in_use(g)) return;
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = bn * OUT_COLS;

  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    for (int idx = tid; idx < BM * OUT_COLS; idx += 256) {
      const int r = idx / OUT_COLS, cc = idx % OUT_COLS;
      const RowInfo ri = row_info(g, pos0 + r);
      if (ri.valid && ncol0 + cc < g.n)
        static_cast<T*>(g.c)[ri.out_row * g.ldc + ncol0 + cc] = from_f32<T>(0.f);
    }
    return;
  }

  // ---- buffer resources
  const i32x4 rA = make_rsrc(g.a, (uint32_t)(g.a_rows * g.lda * (int64_t)sizeof(T)));
  const int64_t b_rows_total = (EPI == EPI_SILU_MUL) ? 2 * (int64_t)g.inter : (int64_t)g.n;
  const i32x4 rB = make_rsrc(g.b + expert * g.b_e, (uint32_t)(b_rows_total * g.b_n));
  const i32x4 rS = make_rsrc(g.bs + expert * g.bs_e, (uint32_t)(b_rows_total * g.bs_n));

  // B-tile row -> weight row (or -1 past N).  With SiLU, 16-row blocks
  // alternate gate (even) and up (odd) rows of the same output columns.
  auto weight_row = [&](int i) -> int {
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

  // ---- per-lane load offsets for stage 0; stage kt adds kt * stride
  uint32_t a_off[S::A_LOADS];
#pragma unroll
  for (int j = 0; j < S::A_LOADS; ++j) {
    const int row = (wave * S::A_LOADS + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (row & 7);
    const RowInfo ri = row_info(g, pos0 + row);
    a_off[j] = ri.valid ? (uint32_t)(ri.a_row * g.lda * (int64_t)sizeof(T)) + c * 16 : kOOB;
  }
  uint32_t b_off[S::B_LOADS];
#pragma unroll
  for (int j = 0; j < S::B_LOADS; ++j) {
    const int row = (wave * S::B_LOADS + j) * 32 + (lane >> 1);
    const int c = (lane & 1) ^ ((row >> 3) & 1);
    const int grow = weight_row(row);
    b_off[j] = grow >= 0 ? (uint32_t)(grow * g.b_n) + c * 16 : kOOB;
  }
  uint32_t s_off = kOOB;
  if (wave < S::S_WAVES) {
    const int grow = weight_row(wave * 64 + lane);
    s_off = grow >= 0 ? (uint32_t)(grow * g.bs_n) : kOOB;
  }

  const int nk = g.k / 64;
  auto issue = [&](int kt) {
    const int st = kt % STAGES;
    if ((kt & 1) == 0 && wave < S::S_WAVES)
      llvm_amdgcn_raw_buffer_load_lds(rS, lds_ptr(sS + ((kt >> 1) & 1) * S::S_SLOT + wave * 256),
                                      4, (int)(s_off + (uint32_t)(kt >> 1) * 4u), 0, 0, 0);
#pragma unroll
    for (int j = 0; j < S::A_LOADS; ++j)
      llvm_amdgcn_raw_buffer_load_lds(
          rA, lds_ptr(sA + st * S::A_STAGE + (wave * S::A_LOADS + j) * 1024), 16,
          (int)(a_off[j] + (uint32_t)kt * 128u), 0, 0, 0);
#pragma unroll
    for (int j = 0; j < S::B_LOADS; ++j)
      llvm_amdgcn_raw_buffer_load_lds(
          rB, lds_ptr(sB + st * S::B_STAGE + (wave * S::B_LOADS + j) * 1024), 16,
          (int)(b_off[j] + (uint32_t)kt * 32u), 0, 0, 0);
  };

  // ---- per-lane LDS read offsets (fragment rows differ from c16 by
  // multiples of 16, so the swizzle terms are lane constants)
  const int a_rd0 = (wm * FM * 16 + c16) * 128 + ((grp ^ (c16 & 7)) * 16);
  const int b_sw = (c16 >> 3) & 1;
  const int b_rd = (wn * FN * 16 + c16) * 32 + grp * 4;
  const int s_rd = (wn * FN * 16 + c16) * 4;

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) issue(s);
  for (int kt = 0; kt < nk; ++kt) {
    // Stage kt has landed once at most the later stages' loads are
    // outstanding.  A bare s_barrier (not __syncthreads, whose release fence
    // would drain every outstanding load) then publishes it to all waves and
    // retires the reads of the buffer the next issue() overwrites.
    constexpr int PER_STAGE = S::A_LOADS + S::B_LOADS;
    if (STAGES == 3 && kt + 1 < nk) wait_vmcnt<PER_STAGE>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
    const uint8_t* As = sA + (kt % STAGES) * S::A_STAGE;
    const uint8_t* Bs = sB + (kt % STAGES) * S::B_STAGE;
    const uint8_t* Ss = sS + ((kt >> 1) & 1) * S::S_SLOT + (kt & 1) * 2;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      // logical chunk ks*4 + grp sits at physical chunk (grp ^ sw) ^ (ks*4):
      // flipping bit 6 of the byte offset selects the ks = 1 half
      V8 af[FM];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        af[fm] = *reinterpret_cast<const V8*>(As + ((a_rd0 + fm * 16 * 128) ^ (ks * 64)));
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const uint32_t raw =
            *reinterpret_cast<const uint32_t*>(Bs + b_rd + fn * 16 * 32 + ((ks ^ b_sw) * 16));
        const V8 bf = Decode<T>::run(raw, e8m0_scale(Ss[s_rd + fn * 16 * 4 + ks]));
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) acc[fm][fn] = mfma16(bf, af[fm], acc[fm][fn]);
      }
    }
  }

  // ---- epilogue: lane owns row wm*FM*16 + fm*16 + c16 and columns
  // fn*16 + grp*4 .. +3 of its wave's sub-tile; stage the finished tile in LDS
  __builtin_amdgcn_s_barrier();  // every wave is done reading the stage buffers
  const float alpha = scalar_alpha(g, expert);
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int trow = wm * FM * 16 + fm * 16 + c16;
    float rw = 1.0f;
    if (g.route_w) {
      const RowInfo r = row_info(g, pos0 + trow);
      rw = r.valid ? g.route_w[r.out_row] : 0.f;
    }
    uint8_t* crow = smem + trow * C_LD;
    if (EPI == EPI_SILU_MUL) {
#pragma unroll
      for (int fn = 0; fn < FN; fn += 2) {
        const int tcol = ((wn * FN + fn) >> 1) * 16 + grp * 4;
        float h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // vllm:249-252 on tensors of T: gate and up rounded to T, silu in
          // FP32 rounded to T, the product rounded to T (below)
          const T gb = from_f32<T>(acc[fm][fn][i] * alpha);
          const T ub = from_f32<T>(acc[fm][fn + 1][i] * alpha);
          const T sb = from_f32<T>(silu_f32(to_f32(gb)));
          h[i] = to_f32(sb) * to_f32(ub);
        }
        *reinterpret_cast<uint2*>(crow + tcol * 2) = uint2{pack2<T>(h[0], h[1]), pack2<T>(h[2], h[3])};
      }
    } else {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int tcol = wn * FN * 16 + fn * 16 + grp * 4;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = acc[fm][fn][i] * alpha * rw;
        if (g.bias) {
          const T* bp = static_cast<const T*>(g.bias) + ncol0 + tcol;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (ncol0 + tcol + i < g.n) o[i] += to_f32(bp[i]);
        }
        *reinterpret_cast<uint2*>(crow + tcol * 2) = uint2{pack2<T>(o[0], o[1]), pack2<T>(o[2], o[3])};
      }
    }
  }
  __syncthreads();
  // whole 16-byte chunks, consecutive lanes along a row
  constexpr int CHUNKS = OUT_COLS / 8;
  for (int idx = tid; idx < BM * CHUNKS; idx += 256) {
    const int trow = idx / CHUNKS, ch = idx % CHUNKS;
    const int col = ncol0 + ch * 8;
    if (col >= g.n) continue;
    const RowInfo r = row_info(g, pos0 + trow);
    if (!r.valid) continue;
    const uint8_t* src = smem + trow * C_LD + ch * 16;
    T* dst = static_cast<T*>(g.c) + r.out_row * g.ldc + col;
    if (col + 8 <= g.n && (g.ldc & 7) == 0) {
      *reinterpret_cast<i32x4*>(dst) = *reinterpret_cast<const i32x4*>(src);
    } else {
      const T* s16 = reinterpret_cast<const T*>(src);
      for (int i = 0; i < 8 && col + i < g.n; ++i) dst[i] = s16[i];
    }
  }
}

template <typename T, int FM, int FN, int STAGES, int EPI, int MINB>
int launch_cfg(const GemmArgs& g, hipStream_t st) {
  typedef PfShape<FM, FN, STAGES> S;
  const int out_cols = (EPI == EPI_SILU_MUL) ? S::BN / 2 : S::BN;
  const int nbn = (g.n + out_cols - 1) / out_cols;
  const int64_t nbm = (g.m + S::BM - 1) / S::BM;
  const int64_t nwg = nbm * nbn;
  if (nwg <= 0 || nwg > 0x7FFFFFFF) {
    set_error("w4a16 prefill: bad grid");
    return MXFP4_ERR_VALUE;
  }
  w4a16_pf<T, FM, FN, STAGES, EPI, MINB><<<(unsigned)nwg, 256, 0, st>>>(g, (int)nbm, nbn);
  return launch_status("w4a16 prefill launch");
}

// Tile configurations (BM x BN weight rows, stages, workgroups per CU).
// Measured on MI355X (bf16): 128 x 128 / 2 stages is best for M = 4096 at
// qkv (K 2048, N 5120) and o_proj (K 4096, N 2048) shapes, 128 x 256 once
// there are >= 1024 such tiles (M 8192, K N 4096), 64 x 128 / 3 stages at
// M ~ 370; smaller M uses 32 x 128.
template <typename T, int EPI>
int launch_pf_typed(const GemmArgs& g, int cfg, hipStream_t st) {
  switch (cfg) {
    case PF_128x256: return launch_cfg<T, 4, 8, 2, EPI, 2>(g, st);
    case PF_128x128: return launch_cfg<T, 4, 4, 2, EPI, 2>(g, st);
    case PF_64x128: return launch_cfg<T, 2, 4, 3, EPI, 4>(g, st);
    default: return launch_cfg<T, 1, 4, 3, EPI, 4>(g, st);
  }
}

}  // namespace

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

int pf_choose(const GemmArgs& g, int epi) {
  const bool routed = g.sorted_ids != nullptr;
  auto allowed = [&](int bm) { return !routed || g.block_m % bm == 0; };
  auto tiles = [&](int bm, int bn) {
    const int out = epi == EPI_SILU_MUL ? bn / 2 : bn;
    return ((g.m + bm - 1) / bm) * (int64_t)((g.n + out - 1) / out);
  };
  if (allowed(128)) {
    if (tiles(128, 256) >= 1024) return PF_128x256;
    if (tiles(128, 128) >= 512) return PF_128x128;
  }
  if (allowed(64) && tiles(64, 128) >= 200) return PF_64x128;
  return PF_32x128;
}

int launch_w4a16_pf(const GemmArgs& g, int dtype, int epi, int cfg, hipStream_t st) {
  if (dtype == MXFP4_DT_BF16)
    return epi == EPI_STORE ? launch_pf_typed<__bf16, EPI_STORE>(g, cfg, st)
                            : launch_pf_typed<__bf16, EPI_SILU_MUL>(g, cfg, st);
  return epi == EPI_STORE ? launch_pf_typed<_Float16, EPI_STORE>(g, cfg, st)
                          : launch_pf_typed<_Float16, EPI_SILU_MUL>(g, cfg, st);
}

}  // namespace mx
