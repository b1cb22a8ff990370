// W4A16 GEMM kernels: BF16/FP16 activations x packed MXFP4 weights, FP32
// accumulation on the 16x16x32 MFMA, E2M1 decode in registers.
//
// Two shapes of kernel serve the dense linear (soft:310-376) and the routed
// grouped GEMM (soft:65-173, 379-494):
//
// * skinny (decode, <= 32 rows per tile): a workgroup owns 16 output columns
//   and one 16/32-row block; its waves split K.  Each lane streams 16 bytes
//   of packed weights (32 K values = exactly one E8M0 block) per step straight
//   from HBM into registers -- per row 4 lanes cover 64 contiguous bytes --
//   decodes them to 4 MFMA B fragments, and reuses them for up to two 16-row
//   A blocks.  The waves' partial tiles are reduced through LDS in a fixed
//   order, so results are bitwise repeatable (no atomics).
//
// * tiled (prefill): 256-thread workgroups own a BM x BN tile; each 64-deep K
//   stage moves the A tile (BM x 64 bf16) and the packed B tile (BN x 32 B +
//   2 scale bytes per row) global -> registers -> LDS, double buffered with
//   one barrier per stage; waves (2 x 2) read MFMA fragments from LDS and
//   decode B fragments in registers right before the MFMA.  The packed B
//   tile is 4x smaller than a bf16 one, so LDS traffic is dominated by A.
//
// The SiLU*mul epilogue (vllm:249-252) pairs gate column j with up column
// inter + j inside the same lane, so the gate_up GEMM writes h directly.
#include <algorithm>
#include <type_traits>

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

template <typename V>
__device__ __forceinline__ V zero_v8() {
  return __builtin_bit_cast(V, i32x4{0, 0, 0, 0});
}

// Epilogue for one output element.
template <typename T, int EPI>
__device__ __forceinline__ void store_out(const GemmArgs& g, const RowInfo& r, int col,
                                          float alpha, float v0, float v1, int expert) {
  T* cp = static_cast<T*>(g.c) + r.out_row * g.ldc + col;
  if (EPI == EPI_STORE) {
    float o = g.ref_round ? ref_scaled<T>(g, v0, expert) : v0 * alpha;
    if (g.route_w) o *= g.route_w[r.out_row];
    if (g.bias) o += to_f32(static_cast<const T*>(g.bias)[col]);
    *cp = from_f32<T>(o);
  } else {
    // vllm:249-252 on tensors of T: gate_up rounded to T, silu evaluated in
    // FP32 and rounded to T, the product rounded to T.
    const T gb = from_f32<T>(v0 * alpha);
    const T ub = from_f32<T>(v1 * alpha);
    const T sb = silu_round<T>(gb);
    *cp = from_f32<T>(to_f32(sb) * to_f32(ub));
  }
}

// ---------------------------------------------------------------- direct routing
constexpr int kDirectMaxRoutes = 256;  // routes scanned by one wave (4 x 64)

// Rows of workgroup row r under direct routing: r leads if its expert e is
// valid and r is the 0th, 16th, 32nd ... route of e (in route order); it
// then owns that route and the next 15 routes of e.  Every wave finds this
// on its own from ballots over all route ids (at most kDirectMaxRoutes,
// loaded as raw words first so no load waits for another), so no barrier
// is needed.  Returns nonzero if the workgroup has no work.
template <int RB>
__device__ __forceinline__ int direct_rows(const GemmArgs& g, int r, int c16, int* expert,
                                           int64_t* my_route) {
  static_assert(RB == 1, "direct routing uses 16-row blocks");
  constexpr int NC = kDirectMaxRoutes / 64;
  const int lane = threadIdx.x & 63;
  const int nr = (int)g.num_valid;
  const int esz = g.ids64 ? 8 : 4;
  const i32x4 rI = make_rsrc(g.route_ids, (uint32_t)(nr * esz));
  uint32_t lo[NC], hi[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t off = (uint32_t)((c * 64 + lane) * esz);
    if (g.ids64) {
      const i32x2 v = buf_load8(rI, off);
      lo[c] = (uint32_t)v[0];
      hi[c] = (uint32_t)v[1];
    } else {
      lo[c] = buf_load4(rI, off);
      hi[c] = 0;
    }
  }
  int64_t id[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t v =
        g.ids64 ? (int64_t)(((uint64_t)hi[c] << 32) | lo[c]) : (int64_t)(int32_t)lo[c];
    id[c] = c * 64 + lane < nr ? v : -1;
  }
  const int rchunk = r >> 6;
  int64_t e = -1;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c == rchunk) {
      const uint32_t elo = __builtin_amdgcn_readlane((int)(uint32_t)id[c], r & 63);
      const uint32_t ehi =
          __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)id[c] >> 32), r & 63);
      e = (int64_t)(((uint64_t)ehi << 32) | elo);
    }
  }
  if (e < 0 || e >= g.num_experts) {
    if (!g.zero_dropped) return 1;
    // the route's row alone, through the expert -1 path (zeros)
    *expert = -1;
    my_route[0] = c16 == 0 ? r : -1;
    return 0;
  }
  int rank = 0, got = 0;
  my_route[0] = -1;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c * 64 >= nr) break;
    uint64_t mk = __ballot(id[c] == e);
    if (c < rchunk) {
      rank += __popcll(mk);
      continue;
    }
    if (c == rchunk) {
      const uint64_t below = (1ull << (r & 63)) - 1;
      rank += __popcll(mk & below);
      if (rank & 15) return 1;
      mk &= ~below;
    }
    while (mk && got < 16) {
      const int b = __builtin_ctzll(mk);
      mk &= mk - 1;
      if (c16 == got) my_route[0] = c * 64 + b;
      ++got;
    }
  }
  *expert = (int)e;
  return 0;
}

// Activation rows the skinny kernel stages in LDS, and their LDS row
// stride for K = 128 x nunits (whole 1 KB pieces plus 16 bytes, so rows
// start on different banks).
constexpr int kStageRows = 4;
__host__ __device__ __forceinline__ int stage_stride(int nunits) {
  return (nunits * 256 + 1023) / 1024 * 1024 + 16;
}

// ---------------------------------------------------------------- skinny
// NW = WK x WN waves.  Each wave owns CG adjacent groups of 16 output
// columns (for SiLU each group is a gate block and an up block) and one of
// WK slices of K; WN such waves sit side by side on columns.  Loads are
// what bounds this kernel (each vector memory instruction costs the
// address unit about the same, however few lanes it has active), so a wave
// reuses each activation fragment for its CG column groups, and takes the
// scales of a whole trip with one load per column block.  A wave takes U
// consecutive 128-K units per trip and issues every load of the trip
// before its first MFMA; all loads are branch-free buffer loads (zero past
// the end) except the activation loads of padding rows, which are
// exec-masked off.  Routed blocks read the block's expert id and the padded
// row count with two independent scalar loads.
template <typename T, int RB, int WK, int WN, int CG, int U, int EPI, int SR>
__global__ __launch_bounds__(WK * WN * 64) void w4a16_skinny(GemmArgs g) {
  constexpr int srows = SR;  // block rows staged through LDS
  typedef typename V8Of<T>::type V8;
  constexpr int CB = (EPI == EPI_SILU_MUL) ? 2 : 1;
  constexpr int NB = CB * CG;  // weight blocks of 16 rows per wave
  static_assert(U == 2 || U == 4, "scale loads cover 2 or 4 units");
  __shared__ f32x4 red[WK][WN * CG][RB * CB][64];
  extern __shared__ __attribute__((aligned(16))) uint8_t a_lds[];  // staged activation rows

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar
  const int wk = wave % WK;
  const int wn = wave / WK;
  const int c16 = lane & 15;
  const int grp = lane >> 4;
  const int64_t pos0 = (int64_t)blockIdx.y * (16 * RB);
  __shared__ int64_t srow[RB * 16];  // output row of each tile row, -1 = none
  int expert = 0;
  int64_t my_route[RB];  // output row of this lane's tile row (c16) per row block
  if (g.route_ids) {
    if constexpr (RB == 1) {
      if (direct_rows<RB>(g, (int)blockIdx.y, c16, &expert, my_route)) return;
    } else {
      return;  // direct routing is launched with 16-row blocks only
    }
  } else if (g.sorted_ids) {
    const int64_t npp = *g.num_post_padded;
    const int e = block_expert(g, pos0);
    if (pos0 >= (npp < g.m ? npp : g.m)) return;
    expert = e;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const RowInfo ri = row_info(g, pos0 + rb * 16 + c16);
      my_route[rb] = ri.valid ? ri.out_row : -1;
    }
  } else {
    if (pos0 >= g.m) return;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t p = pos0 + rb * 16 + c16;
      my_route[rb] = p < g.m ? p : -1;
    }
  }
  if (wave == 0 && grp == 0) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) srow[rb * 16 + c16] = my_route[rb];
  }
  const int n0 = (blockIdx.x * WN + wn) * 16 * CG;

  f32x4 acc[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[rb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (expert >= 0) {
    // Buffer resources: this expert's weights and scales, and the whole
    // activation matrix (host-checked to stay below 2 GiB each).  Columns
    // past N re-read row 0 (their outputs are not stored); padding rows
    // and K past the end read zeros through kOOB.
    const int64_t b_rows_total = (CB == 2) ? 2 * (int64_t)g.inter : (int64_t)g.n;
    const i32x4 rB = make_rsrc(g.b + expert * g.b_e, (uint32_t)(b_rows_total * g.b_n));
    const i32x4 rS = make_rsrc(g.bs + expert * g.bs_e, (uint32_t)(b_rows_total * g.bs_n));
    const i32x4 rA = make_rsrc(g.a, (uint32_t)(g.a_rows * g.lda * (int64_t)sizeof(T)));
    uint32_t boff[NB], soff[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = n0 + (nb / CB) * 16 + c16;
      const int64_t brow = ((nb % CB) == 0 ? 0 : g.inter) + (col < g.n ? col : 0);
      boff[nb] = (uint32_t)(brow * g.b_n);
      soff[nb] = (uint32_t)(brow * g.bs_n);
    }
    uint32_t aoff[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t arow = (g.sorted_ids || g.route_ids) ? my_route[rb] / g.top_k : my_route[rb];
      aoff[rb] = my_route[rb] >= 0 ? (uint32_t)(arow * g.lda * (int64_t)sizeof(T)) : kOOB;
    }
    const int nunits = (g.k + 127) >> 7;
    // buffer dword loads need 4-byte aligned addresses
    const bool s_dword = ((g.bs_n | g.bs_e | (int64_t)reinterpret_cast<uintptr_t>(g.bs)) & 3) == 0;
    const uint32_t sshift = s_dword ? 8u * grp : 0u;
    // Activation staging: when one trip covers K, block rows
    // 0 .. srows-1 are copied once per workgroup into LDS with
    // direct-to-LDS loads (1 KB per instruction, all lanes active) instead
    // of 16 lane-masked loads per wave; other rows load per lane.  The
    // copies are issued after the weight loads, which do not wait for the
    // row ids they need.
    const bool stage = nunits <= WK * U;
    const int a_stride = stage_stride(nunits);
    const int trips = stage ? 1 : (nunits - wk * U + WK * U - 1) / (WK * U);
    for (int t = 0; t < trips; ++t) {
      const int u0 = wk * U + t * WK * U;
      // Scales: with 4-byte aligned scale rows one load per lane and weight
      // block covers the trip -- the U x 4 E8M0 bytes of its row (4 per
      // unit, one per lane group), lane group grp taking byte grp of each
      // unit's dword; otherwise one byte load per unit.  Bytes are
      // extracted where they are used, so no load result is consumed here.
      uint32_t sdw[NB][U];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint32_t so = soff[nb] + (uint32_t)(u0 * 4);
        if (s_dword) {
          if (U == 4) {
            const i32x4 v = buf_load16(rS, so);
#pragma unroll
            for (int uu = 0; uu < U; ++uu) sdw[nb][uu] = (uint32_t)v[uu];
          } else {
            const i32x2 v = buf_load8(rS, so);
#pragma unroll
            for (int uu = 0; uu < U; ++uu) sdw[nb][uu] = (uint32_t)v[uu];
          }
        } else {
#pragma unroll
          for (int uu = 0; uu < U; ++uu) sdw[nb][uu] = buf_load_u8(rS, so + 4 * uu + grp);
        }
      }
      i32x4 braw[U][NB];
#pragma unroll
      for (int uu = 0; uu < U; ++uu) {
        const int k0 = (u0 + uu) * 128 + grp * 32;
        const bool k_ok = k0 < g.k;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          braw[uu][nb] = buf_load16(rB, k_ok ? boff[nb] + (uint32_t)(k0 >> 1) : kOOB);
      }
      if (stage) {
        const int qn = (nunits * 256 + 1023) / 1024;
        for (int i = wave; i < srows * qn; i += WK * WN) {
          const int br = i / qn, q = i - (i / qn) * qn;
          const int route = __builtin_amdgcn_readlane((int)my_route[0], br);
          if (route < 0) continue;
          const int64_t arow = (g.sorted_ids || g.route_ids) ? route / g.top_k : route;
          const uint32_t kb = (uint32_t)(q * 1024 + lane * 16);
          const uint32_t off = kb < (uint32_t)(g.k * (int)sizeof(T))
                                   ? (uint32_t)(arow * g.lda * (int64_t)sizeof(T)) + kb
                                   : kOOB;
          llvm_amdgcn_raw_buffer_load_lds(rA, lds_ptr(a_lds + br * a_stride + q * 1024), 16, off,
                                          0, 0, 0);
        }
      }
      V8 af[U][RB][4];
#pragma unroll
      for (int uu = 0; uu < U; ++uu) {
        const int k0 = (u0 + uu) * 128 + grp * 32;
        const bool k_ok = k0 < g.k;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const bool staged = stage && rb * 16 + c16 < srows;
          // nothing in this branch consumes the loaded values, so no wait
          // is placed in it
          if (k_ok && aoff[rb] != kOOB && !staged) {
            const uint32_t o = aoff[rb] + (uint32_t)(k0 * (int)sizeof(T));
#pragma unroll
            for (int j = 0; j < 4; ++j)
              af[uu][rb][j] = __builtin_bit_cast(V8, buf_load16(rA, o + 16 * j));
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) af[uu][rb][j] = zero_v8<V8>();
          }
        }
      }
      if (stage) {
        // the staged rows have landed once every wave's loads are done
        wait_vmcnt<0>();
        barrier_only();
#pragma unroll
        for (int uu = 0; uu < U; ++uu)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const int br = rb * 16 + c16;
            const bool k_ok = (u0 + uu) * 128 + grp * 32 < g.k;
            if (br < srows && aoff[rb] != kOOB && k_ok) {
              const uint8_t* src = a_lds + br * a_stride + (u0 + uu) * 256 + grp * 64;
#pragma unroll
              for (int j = 0; j < 4; ++j) af[uu][rb][j] = *reinterpret_cast<const V8*>(src + 16 * j);
            }
          }
      }
#pragma unroll
      for (int uu = 0; uu < U; ++uu) {
        // K past the end: weights read as zero; the scale is forced to 1 so
        // bytes of the next row (possibly NaN) cannot leak in
        const bool k_ok = (u0 + uu) * 128 + grp * 32 < g.k;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const uint32_t sb = k_ok ? (sdw[nb][uu] >> sshift) & 0xFFu : 127u;
          const float sc = e8m0_scale(sb);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const V8 bf = Decode<T>::run((uint32_t)braw[uu][nb][j], sc);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              acc[rb][nb] = mfma16(af[uu][rb][j], bf, acc[rb][nb]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      red[wk][wn * CG + nb / CB][rb * CB + nb % CB][lane] = acc[rb][nb];
  __syncthreads();

  const float alpha = expert >= 0 ? scalar_alpha(g, expert) : 0.f;
  for (int idx = threadIdx.x; idx < WN * CG * RB * 256; idx += WK * WN * 64) {
    const int cgi = idx / (RB * 256);
    const int rb = (idx >> 8) % RB;
    const int l = (idx >> 2) & 63;
    const int i = idx & 3;
    const int col = (blockIdx.x * WN * CG + cgi) * 16 + (l & 15);
    RowInfo r;
    r.out_row = srow[rb * 16 + (l >> 4) * 4 + i];
    r.valid = r.out_row >= 0;
    if (!r.valid || col >= g.n) continue;
    if (expert < 0) {
      static_cast<T*>(g.c)[r.out_row * g.ldc + col] = from_f32<T>(0.f);
      continue;
    }
    float v[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < WK; ++w) s += red[w][cgi][rb * CB + cb][l][i];
      v[cb] = s;
    }
    store_out<T, EPI>(g, r, col, alpha, v[0], v[CB - 1], expert);
  }
}

// ---------------------------------------------------------------- stream
// Single-trip decode (one 16-row block; every wave's K slice is one trip of
// U 128-K units) over CS steps of WN groups of 16 output columns.  The
// workgroup looks up its rows and stages its activation rows once, then
// software-pipelines the steps: the weights and scales of step s + 1 are in
// flight while step s is decoded, multiplied, reduced across the WK waves
// (double-buffered LDS, one barrier per step) and stored.  For grids of
// many small workgroups (routed decode: an expert block times a column
// group each) this pays the row lookup and the first memory round trip
// once per CS column groups, and keeps weight loads streaming through the
// epilogues.  Same loads, rounding and reduction order as the skinny
// kernel, so results are identical.
template <typename T, int WK, int WN, int U, int CS, int EPI>
__global__ __launch_bounds__(WK * WN * 64) __attribute__((amdgpu_waves_per_eu(CS >= 4 ? 3 : 1)))
void w4a16_stream(GemmArgs g) {
  typedef typename V8Of<T>::type V8;
  constexpr int NB = (EPI == EPI_SILU_MUL) ? 2 : 1;
  static_assert(U == 2 || U == 4, "scale loads cover 2 or 4 units");
  __shared__ f32x4 red[2][WK][WN][NB][64];
  __shared__ int64_t srow[16];
  extern __shared__ __attribute__((aligned(16))) uint8_t a_lds[];  // staged activation rows

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar
  const int wk = wave % WK;
  const int wn = wave / WK;
  const int c16 = lane & 15;
  const int grp = lane >> 4;
  // the row lookup of the skinny kernel for one 16-row block
  const int64_t pos0 = (int64_t)blockIdx.y * 16;
  int expert = 0;
  int64_t my_route[1];
  if (g.route_ids) {
    if (direct_rows<1>(g, (int)blockIdx.y, c16, &expert, my_route)) return;
  } else if (g.sorted_ids) {
    const int64_t npp = *g.num_post_padded;
    const int e = block_expert(g, pos0);
    if (pos0 >= (npp < g.m ? npp : g.m)) return;
    expert = e;
    const RowInfo ri = row_info(g, pos0 + c16);
    my_route[0] = ri.valid ? ri.out_row : -1;
  } else {
    if (pos0 >= g.m) return;
    my_route[0] = pos0 + c16 < g.m ? pos0 + c16 : -1;
  }
  if (wave == 0 && grp == 0) srow[c16] = my_route[0];
  // first output column of wave-column w at step s
  auto col0 = [&](int s, int w) { return (((int)blockIdx.x * CS + s) * WN + w) * 16; };

  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    __syncthreads();
    for (int idx = threadIdx.x; idx < CS * WN * 256; idx += WK * WN * 64) {
      const int s = idx / (WN * 256), w = (idx >> 8) % WN;
      const int col = col0(s, w) + ((idx >> 2) & 15);
      const int64_t row = srow[((idx >> 6) & 3) * 4 + (idx & 3)];
      if (row >= 0 && col < g.n) static_cast<T*>(g.c)[row * g.ldc + col] = from_f32<T>(0.f);
    }
    return;
  }

  const int64_t b_rows_total = (NB == 2) ? 2 * (int64_t)g.inter : (int64_t)g.n;
  const i32x4 rB = make_rsrc(g.b + expert * g.b_e, (uint32_t)(b_rows_total * g.b_n));
  const i32x4 rS = make_rsrc(g.bs + expert * g.bs_e, (uint32_t)(b_rows_total * g.bs_n));
  const i32x4 rA = make_rsrc(g.a, (uint32_t)(g.a_rows * g.lda * (int64_t)sizeof(T)));
  const int u0 = wk * U;
  const int nunits = (g.k + 127) >> 7;
  const bool s_dword = ((g.bs_n | g.bs_e | (int64_t)reinterpret_cast<uintptr_t>(g.bs)) & 3) == 0;
  const uint32_t sshift = s_dword ? 8u * grp : 0u;

  // weights and scales of step s into ring slot b (columns past N re-read
  // row 0; their outputs are not stored)
  i32x4 braw[2][U][NB];
  uint32_t sdw[2][NB][U];
  auto load_step = [&](int s, auto slot_c) {
    constexpr int b = decltype(slot_c)::value;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = col0(s, wn) + c16;
      const int64_t brow = (nb == 0 ? 0 : g.inter) + (col < g.n ? col : 0);
      const uint32_t so = (uint32_t)(brow * g.bs_n) + (uint32_t)(u0 * 4);
      if (s_dword) {
        if (U == 4) {
          const i32x4 v = buf_load16(rS, so);
#pragma unroll
          for (int uu = 0; uu < U; ++uu) sdw[b][nb][uu] = (uint32_t)v[uu];
        } else {
          const i32x2 v = buf_load8(rS, so);
#pragma unroll
          for (int uu = 0; uu < U; ++uu) sdw[b][nb][uu] = (uint32_t)v[uu];
        }
      } else {
#pragma unroll
        for (int uu = 0; uu < U; ++uu) sdw[b][nb][uu] = buf_load_u8(rS, so + 4 * uu + grp);
      }
      const uint32_t bo = (uint32_t)(brow * g.b_n);
#pragma unroll
      for (int uu = 0; uu < U; ++uu) {
        const int k0 = (u0 + uu) * 128 + grp * 32;
        braw[b][uu][nb] = buf_load16(rB, k0 < g.k ? bo + (uint32_t)(k0 >> 1) : kOOB);
      }
    }
  };
  load_step(0, std::integral_constant<int, 0>{});

  // activation rows: rows 0 .. kStageRows-1 of the block go to LDS with
  // direct-to-LDS loads, other rows load per lane (as in the skinny kernel)
  const int64_t arow = (g.sorted_ids || g.route_ids) ? my_route[0] / g.top_k : my_route[0];
  const uint32_t aoff = my_route[0] >= 0 ? (uint32_t)(arow * g.lda * (int64_t)sizeof(T)) : kOOB;
  const int a_stride = stage_stride(nunits);
  {
    const int qn = (nunits * 256 + 1023) / 1024;
    for (int i = wave; i < kStageRows * qn; i += WK * WN) {
      const int br = i / qn, q = i - (i / qn) * qn;
      const int route = __builtin_amdgcn_readlane((int)my_route[0], br);
      if (route < 0) continue;
      const int64_t ar = (g.sorted_ids || g.route_ids) ? route / g.top_k : route;
      const uint32_t kb = (uint32_t)(q * 1024 + lane * 16);
      const uint32_t off =
          kb < (uint32_t)(g.k * (int)sizeof(T)) ? (uint32_t)(ar * g.lda * (int64_t)sizeof(T)) + kb
                                                : kOOB;
      llvm_amdgcn_raw_buffer_load_lds(rA, lds_ptr(a_lds + br * a_stride + q * 1024), 16, off, 0, 0,
                                      0);
    }
  }
  V8 af[U][4];
#pragma unroll
  for (int uu = 0; uu < U; ++uu) {
    const int k0 = (u0 + uu) * 128 + grp * 32;
    // nothing in this branch consumes the loaded values, so no wait is
    // placed in it
    if (k0 < g.k && aoff != kOOB && c16 >= kStageRows) {
      const uint32_t o = aoff + (uint32_t)(k0 * (int)sizeof(T));
#pragma unroll
      for (int j = 0; j < 4; ++j) af[uu][j] = __builtin_bit_cast(V8, buf_load16(rA, o + 16 * j));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) af[uu][j] = zero_v8<V8>();
    }
  }

  const float alpha = scalar_alpha(g, expert);
  static_for<0, CS>([&](auto step_c) {
    constexpr int s = decltype(step_c)::value;
    constexpr int b = s & 1;
    // the wait below lets the next step's loads stay in flight and counts
    // on every earlier load (the staging copies above all) having been
    // issued before them: a compiler fence keeps that order
    if constexpr (s == 0) asm volatile("" ::: "memory");
    if constexpr (s + 1 < CS) load_step(s + 1, std::integral_constant<int, b ^ 1>{});
    if constexpr (s == 0) {
      // the staged rows have landed once at most the next step's loads
      // (NB scale and U x NB weight loads in the dword-scale path, more
      // otherwise) are outstanding
      if constexpr (CS > 1) wait_vmcnt<NB + U * NB>();
      else wait_vmcnt<0>();
      barrier_only();
#pragma unroll
      for (int uu = 0; uu < U; ++uu) {
        const bool k_ok = (u0 + uu) * 128 + grp * 32 < g.k;
        if (c16 < kStageRows && aoff != kOOB && k_ok) {
          const uint8_t* src = a_lds + c16 * a_stride + (u0 + uu) * 256 + grp * 64;
#pragma unroll
          for (int j = 0; j < 4; ++j) af[uu][j] = *reinterpret_cast<const V8*>(src + 16 * j);
        }
      }
    }
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      // K past the end: weights read as zero, the scale forced to 1
      const bool k_ok = (u0 + uu) * 128 + grp * 32 < g.k;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint32_t sb = k_ok ? (sdw[b][nb][uu] >> sshift) & 0xFFu : 127u;
        const float sc = e8m0_scale(sb);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const V8 bf = Decode<T>::run((uint32_t)braw[b][uu][nb][j], sc);
          acc[nb] = mfma16(af[uu][j], bf, acc[nb]);
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[b][wk][wn][nb][lane] = acc[nb];
    // publish the partials (a bare barrier: the next step's loads stay in
    // flight); red[b] is rewritten two steps later, after the next barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (int idx = threadIdx.x; idx < WN * 256; idx += WK * WN * 64) {
      const int w = idx >> 8;
      const int l = (idx >> 2) & 63;
      const int i = idx & 3;
      const int col = col0(s, w) + (l & 15);
      RowInfo r;
      r.out_row = srow[(l >> 4) * 4 + i];
      r.valid = r.out_row >= 0;
      if (!r.valid || col >= g.n) continue;
      float v[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float acc_s = 0.f;
#pragma unroll
        for (int q = 0; q < WK; ++q) acc_s += red[b][q][w][nb][l][i];
        v[nb] = acc_s;
      }
      store_out<T, EPI>(g, r, col, alpha, v[0], v[NB - 1], expert);
    }
  });
}

// ---------------------------------------------------------------- tiled
template <typename T, int FM, int FN, int EPI>
__global__ __launch_bounds__(256) void w4a16_tiled(GemmArgs g) {
  typedef typename V8Of<T>::type V8;
  constexpr int WGM = 2, WGN = 2;
  constexpr int BM = WGM * FM * 16;  // tile rows
  constexpr int BN = WGN * FN * 16;  // B-tile rows (weight rows)
  constexpr int BK = 64;
  constexpr int A_LD = BK + 8;  // elements; 144-byte rows keep b128 reads conflict-free
  constexpr int B_LD = 40;      // bytes; 10-dword rows spread 16 rows over distinct banks
  constexpr int A_PER = BM * 8 / 256;
  constexpr int OUT_COLS = (EPI == EPI_SILU_MUL) ? BN / 2 : BN;
  static_assert(A_PER >= 1 && BN == 128, "tile config");
  static_assert(EPI != EPI_SILU_MUL || FN % 2 == 0, "SiLU pairs need even FN");

  __shared__ __attribute__((aligned(16))) T As[2][BM][A_LD];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN][B_LD];
  __shared__ uint8_t Ss[2][BN][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int c16 = lane & 15;
  const int grp = lane >> 4;

  const int64_t pos0 = (int64_t)blockIdx.y * BM;
  if (pos0 >= rows_in_use(g)) return;
  const int expert = g.sorted_ids ? block_expert(g, pos0) : 0;
  const int ncol0 = blockIdx.x * OUT_COLS;

  if (expert < 0) {  // aiter:156-172: expert not on this device -> zeros
    for (int idx = tid; idx < BM * OUT_COLS; idx += 256) {
      const int r = idx / OUT_COLS, cc = idx % OUT_COLS;
      const RowInfo ri = row_info(g, pos0 + r);
      if (ri.valid && ncol0 + cc < g.n)
        static_cast<T*>(g.c)[ri.out_row * g.ldc + ncol0 + cc] = from_f32<T>(0.f);
    }
    return;
  }

  // ---- per-thread global load assignments
  const T* a_src[A_PER];
  int a_r[A_PER], a_kc[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + i * 256;
    a_r[i] = c >> 3;
    a_kc[i] = c & 7;
    const RowInfo ri = row_info(g, pos0 + a_r[i]);
    a_src[i] = ri.valid ? static_cast<const T*>(g.a) + ri.a_row * g.lda : nullptr;
  }
  // B tile row -> weight row
  auto weight_row = [&](int i, bool& ok) -> int64_t {
    int orow;
    int64_t grow;
    if (EPI == EPI_SILU_MUL) {
      const int cbk = i >> 4;
      orow = ncol0 + (cbk >> 1) * 16 + (i & 15);
      grow = (cbk & 1 ? g.inter : 0) + orow;
    } else {
      orow = ncol0 + i;
      grow = orow;
    }
    ok = orow < g.n;
    return grow;
  };
  const int b_r = tid >> 1, b_h = tid & 1;  // 256 threads = BN rows x 2 halves
  bool b_ok;
  const int64_t b_grow = weight_row(b_r, b_ok);
  const uint8_t* b_src = b_ok ? g.b + expert * g.b_e + b_grow * g.b_n : nullptr;
  const uint8_t* s_src = nullptr;
  if (tid < BN) {
    bool ok;
    const int64_t grow = weight_row(tid, ok);
    s_src = ok ? g.bs + expert * g.bs_e + grow * g.bs_n : nullptr;
  }

  i32x4 areg[A_PER];
  i32x4 breg;
  uint8_t sreg0 = 127, sreg1 = 127;

  auto load_global = [&](int kt) {
    const int kbase = kt * BK;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int k = kbase + a_kc[i] * 8;
      areg[i] = (a_src[i] && k < g.k) ? *reinterpret_cast<const i32x4*>(a_src[i] + k)
                                       : i32x4{0, 0, 0, 0};
    }
    const int kb = kbase + b_h * 32;
    breg = (b_src && kb < g.k) ? *reinterpret_cast<const i32x4*>(b_src + (kb >> 1))
                               : i32x4{0, 0, 0, 0};
    if (tid < BN) {
      sreg0 = (s_src && kbase < g.k) ? s_src[kbase >> 5] : (uint8_t)127;
      sreg1 = (s_src && kbase + 32 < g.k) ? s_src[(kbase >> 5) + 1] : (uint8_t)127;
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      *reinterpret_cast<i32x4*>(&As[buf][a_r[i]][a_kc[i] * 8]) = areg[i];
    int64_t* bdst = reinterpret_cast<int64_t*>(&Bs[buf][b_r][b_h * 16]);
    const i32x4 bv = breg;
    bdst[0] = ((int64_t)(uint32_t)bv[1] << 32) | (uint32_t)bv[0];
    bdst[1] = ((int64_t)(uint32_t)bv[3] << 32) | (uint32_t)bv[2];
    if (tid < BN) {
      Ss[buf][tid][0] = sreg0;
      Ss[buf][tid][1] = sreg1;
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
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      V8 af[FM];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        af[fm] = *reinterpret_cast<const V8*>(
            &As[buf][wm * FM * 16 + fm * 16 + c16][ks * 32 + grp * 8]);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int br = wn * FN * 16 + fn * 16 + c16;
        const uint32_t raw = *reinterpret_cast<const uint32_t*>(&Bs[buf][br][ks * 16 + grp * 4]);
        const V8 bf = Decode<T>::run(raw, e8m0_scale(Ss[buf][br][ks]));
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) acc[fm][fn] = mfma16(af[fm], bf, acc[fm][fn]);
      }
    }
    if (kt + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue
  const float alpha = scalar_alpha(g, expert);
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const RowInfo r = row_info(g, pos0 + wm * FM * 16 + fm * 16 + grp * 4 + i);
      if (!r.valid) continue;
      if (EPI == EPI_SILU_MUL) {
#pragma unroll
        for (int fn = 0; fn < FN; fn += 2) {
          const int col = ncol0 + ((wn * FN + fn) >> 1) * 16 + c16;
          if (col < g.n) store_out<T, EPI>(g, r, col, alpha, acc[fm][fn][i], acc[fm][fn + 1][i],
                                         expert);
        }
      } else {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int col = ncol0 + wn * FN * 16 + fn * 16 + c16;
          if (col < g.n) store_out<T, EPI>(g, r, col, alpha, acc[fm][fn][i], 0.f, expert);
        }
      }
    }
  }
}


// ---------------------------------------------------------------- dispatch
// Wave layout for the skinny kernel: the fewest K-splitting waves WK whose
// single trip (WK x U units of 128) covers K, the rest of the 4 waves side
// by side on columns (8 K-splitting waves beyond 4 x U units).  For short
// K (at most 2 K-splitting waves) each wave takes two column groups
// (CG = 2) once the grid would otherwise hold more than 4 workgroups per
// CU; for longer K the extra registers cost more occupancy than the shared
// activation loads save (measured on the MoE decode shapes).
struct SkinnyShape {
  int rb, wk, wn, cg, u;
};

SkinnyShape skinny_shape(int64_t k, int64_t n, int64_t row_blocks, int rb) {
  const int64_t units = (k + 127) / 128;
  SkinnyShape s;
  s.rb = rb;
  s.u = rb == 1 ? 4 : 2;
  s.wk = 8;
  for (int wk = 1; wk <= 4; wk *= 2)
    if ((int64_t)wk * s.u >= units) {
      s.wk = wk;
      break;
    }
  s.wn = s.wk >= 4 ? 1 : 4 / s.wk;
  const int64_t wgs = (n + 16 * s.wn - 1) / (16 * s.wn) * row_blocks;
  s.cg = (wgs > 4 * 256 && s.wk <= 2) ? 2 : 1;
  return s;
}

// Rows of a skinny block staged through LDS (SR, a template argument: a
// run-time count costs the M=1 GEMV ~0.4 us).  Dense single-block GEMMs of
// 5-16 rows stage 8 or 16 rows within a 72 KB budget; routed blocks and the
// rest stage kStageRows (routed blocks mostly hold a route or two, and the
// larger allocation costs occupancy: MoE layer M=8 39.5 -> 40.1 us with 8).
int skinny_stage_rows(const GemmArgs& g, int rb) {
  if (g.sorted_ids || g.route_ids || rb != 1 || g.m <= kStageRows) return kStageRows;
  const int64_t fit = (int64_t)(72 << 10) / stage_stride((g.k + 127) / 128);
  if (g.m > 8 && fit >= 16) return 16;
  return fit >= 8 ? 8 : kStageRows;
}

template <typename T, int RB, int CG, int EPI, int SR>
void skinny_launch_sr(const GemmArgs& g, const SkinnyShape& s, dim3 grid, hipStream_t st) {
  constexpr int U = RB == 1 ? 4 : 2;
  const int nunits = (g.k + 127) / 128;
  const size_t lds = nunits <= s.wk * U ? (size_t)SR * stage_stride(nunits) : 0;
  switch (s.wk) {
    case 1: w4a16_skinny<T, RB, 1, 4, CG, U, EPI, SR><<<grid, 256, lds, st>>>(g); break;
    case 2: w4a16_skinny<T, RB, 2, 2, CG, U, EPI, SR><<<grid, 256, lds, st>>>(g); break;
    case 4: w4a16_skinny<T, RB, 4, 1, CG, U, EPI, SR><<<grid, 256, lds, st>>>(g); break;
    default: w4a16_skinny<T, RB, 8, 1, CG, U, EPI, SR><<<grid, 512, lds, st>>>(g); break;
  }
}

template <typename T, int RB, int CG, int EPI>
void skinny_launch_cg(const GemmArgs& g, const SkinnyShape& s, dim3 grid, hipStream_t st) {
  const int sr = skinny_stage_rows(g, RB);
  if constexpr (RB == 1 && EPI == EPI_STORE) {
    if (sr == 16) return skinny_launch_sr<T, RB, CG, EPI, 16>(g, s, grid, st);
    if (sr == 8) return skinny_launch_sr<T, RB, CG, EPI, 8>(g, s, grid, st);
  }
  skinny_launch_sr<T, RB, CG, EPI, kStageRows>(g, s, grid, st);
}

template <typename T, int CS, int EPI>
void stream_launch_cs(const GemmArgs& g, const SkinnyShape& s, dim3 grid, hipStream_t st) {
  const int nunits = (g.k + 127) / 128;
  const size_t lds = (size_t)kStageRows * stage_stride(nunits);
  switch (s.wk) {
    case 1: w4a16_stream<T, 1, 4, 4, CS, EPI><<<grid, 256, lds, st>>>(g); break;
    case 2: w4a16_stream<T, 2, 2, 4, CS, EPI><<<grid, 256, lds, st>>>(g); break;
    case 4: w4a16_stream<T, 4, 1, 4, CS, EPI><<<grid, 256, lds, st>>>(g); break;
    default: w4a16_stream<T, 8, 1, 4, CS, EPI><<<grid, 512, lds, st>>>(g); break;
  }
}

// Steps per workgroup of the pipelined single-trip kernel: 2 while that
// keeps >= 512 workgroups (two per CU) busy, else 1 (the skinny kernel).
// Measured on the MoE decode layer (graph replay, 3 weight copies): M=8
// 47.4 -> 43.1 us and M=32 97.0 -> 87.5 us with 2 steps; 4 steps (167-172
// VGPRs, two waves per SIMD) 45.5 / 88.5 us; at M=1 (8 expert blocks) both
// lose to the skinny kernel.
int stream_steps(const GemmArgs& g, const SkinnyShape& s, int64_t blocks, int64_t groups,
                 int epi) {
  if (s.rb != 1 || s.cg != 1 || (g.k + 127) / 128 > s.wk * s.u) return 1;
  if (epi == EPI_SILU_MUL && blocks * ((groups + 3) / 4) >= 512) return 4;
  return blocks * ((groups + 1) / 2) >= 512 ? 2 : 1;
}

template <typename T, int RB, int EPI>
void skinny_launch_rb(const GemmArgs& g, const SkinnyShape& s, dim3 grid, hipStream_t st) {
  if (s.cg == 2) skinny_launch_cg<T, RB, 2, EPI>(g, s, grid, st);
  else skinny_launch_cg<T, RB, 1, EPI>(g, s, grid, st);
}

}  // namespace

int dense_skinny_rows(int64_t m, int64_t k, int64_t n, bool split_ok) {
  if (m <= 16) return 1;
  if (m <= 32) return 2;
  if (m > 128) return 0;
  const int64_t pf_wgs = ((m + 31) / 32) * ((n + 127) / 128);
  if (pf_wgs >= 128 || k / 64 < 48) return 0;
  // given a split-K workspace, M > 64 or K > 4096 run faster as split-K
  // prefill tiles (o_proj M=96 / 128: 19.6 -> 13.7 / 14.9 us; K=8192
  // N=1024 M=64: 19.5 -> 13.7 us; o_proj M <= 64 stays at ~11.2 us skinny)
  if (split_ok && (m > 64 || k > 4096) && splitk_plan(m, k, n).splits > 1) return 0;
  return 2;
}

namespace {

template <typename T, int EPI>
int launch_typed(const GemmArgs& g, hipStream_t st) {
  const int64_t cap = g.m;  // dense rows or sorted capacity
  const bool routed = g.sorted_ids != nullptr;
  const int out_cols = g.n;
  // skinny for 16-row routed blocks (and any routed block size that is not
  // a multiple of 32) and dense M <= 32; tiled otherwise (split K for
  // dense grids too small to fill the GPU, when a workspace is given).  Routed 32-row
  // blocks take the 32 x 128 prefill tile: the 32-row skinny kernel loads
  // each block's activation rows per wave (MoE layer, 32-row blocks, 512
  // tokens: 415 vs 144 us).  Dense M <= 128 also takes 32-row skinny blocks
  // when the prefill grid would be small and its K loop long (fewer than
  // 128 workgroups, >= 48 stages of 64): o_proj K=4096 N=2048 at M=33-128
  // runs 12-20 us that way against ~25 us.
  int skinny_rb = 0;
  if (g.route_ids) {
    skinny_rb = 1;  // direct routing: one workgroup row per route
  } else if (routed) {
    if (g.block_m % 32 != 0) skinny_rb = 1;
  } else {
    skinny_rb = dense_skinny_rows(cap, g.k, g.n, EPI == EPI_STORE && g.splitk_ws != nullptr);
  }
  // the skinny kernel addresses its operands through 2 GiB buffer
  // resources; larger operands go to the tiled kernel where the block size
  // allows it
  const int64_t b_rows_total = (EPI == EPI_SILU_MUL) ? 2 * (int64_t)g.inter : (int64_t)g.n;
  const int64_t lim = 0x7FFFFFFF;
  if (skinny_rb && (g.a_rows * g.lda * (int64_t)sizeof(T) > lim || b_rows_total * g.b_n > lim ||
                    b_rows_total * g.bs_n > lim)) {
    if (g.route_ids || (routed && g.block_m % 32 != 0)) {
      set_error("w4a16: operands above 2 GiB need a routing block size that is a multiple of 32");
      return MXFP4_ERR_VALUE;
    }
    skinny_rb = 0;
  }
  if (skinny_rb) {
    const int rb = skinny_rb;
    const int64_t gy = g.route_ids ? g.num_valid : (cap + 16 * rb - 1) / (16 * rb);
    if (gy > 65535) {
      set_error("w4a16: too many row blocks (%lld)", (long long)gy);
      return MXFP4_ERR_VALUE;
    }
    // active row blocks: dense rows, or at most one partial block per
    // routed expert plus the full ones
    const int64_t blocks = (routed || g.route_ids)
                               ? std::min<int64_t>(gy, g.num_valid / (16 * rb) + g.num_experts)
                               : gy;
    SkinnyShape sh = skinny_shape(g.k, out_cols, blocks, rb);
    // the pipelined kernel (one column group per wave and step) where it
    // applies, before two column groups per wave (MoE M=32 down: 87.0 ->
    // 82.2 us for the layer)
    SkinnyShape sh1 = sh;
    sh1.cg = 1;
    const int64_t groups1 = (out_cols + 16 * sh1.wn - 1) / (16 * sh1.wn);
    const int cs = stream_steps(g, sh1, blocks, groups1, EPI);
    if (cs > 1) {
      dim3 grid((unsigned)((groups1 + cs - 1) / cs), (unsigned)(gy > 0 ? gy : 1));
      if (cs == 4) stream_launch_cs<T, 4, EPI>(g, sh1, grid, st);
      else stream_launch_cs<T, 2, EPI>(g, sh1, grid, st);
      return launch_status("w4a16 stream launch");
    }
    const int tile_cols = 16 * sh.wn * sh.cg;
    dim3 grid((unsigned)((out_cols + tile_cols - 1) / tile_cols), (unsigned)(gy > 0 ? gy : 1));
    if (rb == 1)
      skinny_launch_rb<T, 1, EPI>(g, sh, grid, st);
    else
      skinny_launch_rb<T, 2, EPI>(g, sh, grid, st);
    return launch_status("w4a16 skinny launch");
  }
  const int dt = std::is_same<T, __bf16>::value ? MXFP4_DT_BF16 : MXFP4_DT_F16;
  if (pf_supported(g, (int)sizeof(T))) {
    // dense GEMMs too small to fill the chip split K when given a workspace
    if (EPI == EPI_STORE && !routed && g.splitk_ws != nullptr) {
      const SplitPlan sp = splitk_plan(g.m, g.k, g.n);
      if (sp.splits > 1) {
        GemmArgs gp = g;
        gp.splitk = sp.splits;
        const int rc = launch_w4a16_pf(gp, dt, EPI_PARTIAL, sp.cfg, st);
        return rc ? rc : launch_splitk_reduce(gp, dt, st);
      }
    }
    return launch_w4a16_pf(g, dt, EPI, pf_choose(g, EPI), st);
  }
  // register-staged kernel: BM must divide block_m (routed); the largest BM
  // that still gives >= 512 workgroups, else the smallest
  const int tile_cols = (EPI == EPI_SILU_MUL) ? 64 : 128;
  const int64_t ntiles = (out_cols + tile_cols - 1) / tile_cols;
  int bm = 32;
  const int cands[3] = {128, 64, 32};
  for (int i = 0; i < 3; ++i) {
    const int c = cands[i];
    if (routed && (g.block_m % c) != 0) continue;
    if (((cap + c - 1) / c) * ntiles >= 512) {
      bm = c;
      break;
    }
  }
  dim3 grid((unsigned)ntiles, (unsigned)((cap + bm - 1) / bm));
  if (grid.y > 65535u) {
    set_error("w4a16: too many row tiles (%lld)", (long long)grid.y);
    return MXFP4_ERR_VALUE;
  }
  switch (bm) {
    case 128: w4a16_tiled<T, 4, 4, EPI><<<grid, 256, 0, st>>>(g); break;
    case 64: w4a16_tiled<T, 2, 4, EPI><<<grid, 256, 0, st>>>(g); break;
    default: w4a16_tiled<T, 1, 4, EPI><<<grid, 256, 0, st>>>(g); break;
  }
  return launch_status("w4a16 tiled launch");
}

}  // namespace

int launch_w4a16(const GemmArgs& g, int dtype, int epi, hipStream_t st) {
  if (epi == EPI_STORE_F32) {
    // bf16 A, C in FP32: routed blocks of a multiple of 32 rows on the
    // prefill tiles only (the other kernels store T)
    if (dtype != MXFP4_DT_BF16 || g.route_ids || !g.sorted_ids || g.block_m % 32 != 0 ||
        !pf_supported(g, 2)) {
      set_error("w4a16: C in FP32 needs bf16 activations on routed blocks of 32k rows");
      return MXFP4_ERR_VALUE;
    }
    return launch_w4a16_pf(g, MXFP4_DT_BF16, EPI_STORE_F32, pf_choose(g, EPI_STORE), st);
  }
  if (dtype == MXFP4_DT_BF16)
    return epi == EPI_STORE ? launch_typed<__bf16, EPI_STORE>(g, st)
                            : launch_typed<__bf16, EPI_SILU_MUL>(g, st);
  if (dtype == MXFP4_DT_F16)
    return epi == EPI_STORE ? launch_typed<_Float16, EPI_STORE>(g, st)
                            : launch_typed<_Float16, EPI_SILU_MUL>(g, st);
  set_error("w4a16: unsupported compute dtype %d", dtype);
  return MXFP4_ERR_TYPE;
}


}  // namespace mx
