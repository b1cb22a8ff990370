// MoE decode: the down projection fused with the top-k combine
// (vllm:253-265 for few tokens).
//
// A workgroup owns 16 output columns and a tile of whole tokens -- 16 / top_k
// of them, so the tile's routes t*top_k + k are R <= 16 consecutive rows of
// h.  Each route r needs its own expert's weights, so the MFMA takes the
// weights as its A operand (16 output columns) and the h rows of all R
// routes as its B operand (16 route columns): with expert e_r's weights the
// result's column r is h_r . W_{e_r}; the other columns are not used.  A
// wave keeps one accumulator per route it owns (RG = 4 routes per wave, RW
// such waves), and WK waves split K.  The h fragments are loaded once per
// trip and reused for all RG routes, and every load of a trip -- RG x U
// weight vectors, one scale load per route, the h fragments -- is issued
// before the first MFMA.
//
// The epilogue reproduces the two-kernel path's rounding: the K partial sums
// are added in wave order, each route's value is rounded to T after the
// route weight (the down GEMM's output, soft:164-173), and the routes of a
// token are summed in FP32 in slot order and rounded once (vllm:263-265).
// Routes whose expert id is outside [0, E) contribute nothing.
#include "gemm.h"

namespace mx {
namespace {

constexpr int kRG = 4;  // routes per wave
// Compute units the launch choices below assume (MI355X).  The K-wave count
// decides how K partial sums are grouped, so deriving it from the device
// would make the output bits depend on the SKU or partition mode; with a
// fixed model they depend on the inputs and shapes only.
constexpr int kModelCUs = 256;

struct DownArgs {
  const void* h;          // [routes, inter] of T
  const uint8_t* w;       // [E, hidden, inter/2]
  const uint8_t* ws;      // [E, hidden, inter/32]
  const float* route_w;   // [routes]
  const void* ids;        // [routes] int32 / int64
  void* out;              // [m, hidden] of T
  int64_t m;
  int32_t top_k, hidden, inter, num_experts, ids64;
  int32_t tpt;  // tokens per tile, tpt * top_k <= 16
  int32_t cw;   // output columns per workgroup: 16, or 8 when 16 would leave CUs idle
};

template <typename T, int RW, int WK, int U>
__global__ __launch_bounds__(RW * WK * 64) void moe_down_topk(DownArgs a) {
  typedef typename Decode<T>::vec8 V8;
  static_assert(U == 2 || U == 4, "scale loads cover 2 or 4 units");
  __shared__ f32x4 red[WK][64];
  // the tile's route weights (entries 0 .. 15; one slot per lane of the
  // direct-to-LDS load), loaded with the expert ids before the weight
  // stream so the combine needs no global loads and no registers
  __shared__ __attribute__((aligned(256))) float route_wt[64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar
  const int wk = wave % WK;
  const int rw = wave / WK;
  const int c16 = lane & 15;
  const int grp = lane >> 4;
  const int tpt = a.tpt;
  const int64_t t0 = (int64_t)blockIdx.y * tpt;
  const int64_t r0 = t0 * a.top_k;
  const int64_t routes = a.m * a.top_k;
  const int nrows = (int)((routes - r0) < tpt * a.top_k ? (routes - r0) : tpt * a.top_k);
  // lanes past the workgroup's cw columns load zeros (kOOB) and are not stored
  const int cw = a.cw;
  const bool col_ok = c16 < cw;
  const int col = blockIdx.x * cw + c16;

  // expert of each route of the tile: lane i loads route r0 + i's id (raw
  // words, one load), each wave reads its routes' ids from those lanes
  int e[kRG];
  uint64_t valid;  // bit i: route r0 + i has an expert in [0, E)
  {
    const int esz = a.ids64 ? 8 : 4;
    const i32x4 rI = make_rsrc(a.ids, (uint32_t)(routes * esz));
    const uint32_t off = (uint32_t)((r0 + lane) * esz);
    uint32_t lo, hi;
    if (a.ids64) {
      const i32x2 v = buf_load8(rI, off);
      lo = (uint32_t)v[0];
      hi = (uint32_t)v[1];
    } else {
      lo = buf_load4(rI, off);
      hi = 0;
    }
    const int64_t id = a.ids64 ? (int64_t)(((uint64_t)hi << 32) | lo) : (int64_t)(int32_t)lo;
    const int ok = (lane < nrows && id >= 0 && id < a.num_experts) ? (int)id : -1;
#pragma unroll
    for (int q = 0; q < kRG; ++q) e[q] = __builtin_amdgcn_readlane(ok, (rw * kRG + q) & 63);
    valid = __ballot(ok >= 0);
    if (wave == 0) {
      const i32x4 rW = make_rsrc(a.route_w, (uint32_t)(routes * 4));
      llvm_amdgcn_raw_buffer_load_lds(rW, lds_ptr(reinterpret_cast<uint8_t*>(route_wt)), 4,
                                      lane < nrows ? (int)((r0 + lane) * 4) : (int)kOOB, 0, 0, 0);
    }
  }
  const int64_t b_n = a.inter / 2, bs_n = a.inter / 32;
  const int64_t b_e = (int64_t)a.hidden * b_n, bs_e = (int64_t)a.hidden * bs_n;
  const bool s_dword = ((bs_n | reinterpret_cast<uintptr_t>(a.ws)) & 3) == 0;
  const uint32_t sshift = s_dword ? 8u * grp : 0u;
  const i32x4 rH = make_rsrc(a.h, (uint32_t)(routes * a.inter * (int64_t)sizeof(T)));
  const uint32_t hoff = c16 < nrows ? (uint32_t)((r0 + c16) * a.inter * (int64_t)sizeof(T)) : kOOB;
  const uint32_t boff = col_ok ? (uint32_t)(col * b_n) : kOOB;
  const uint32_t soff = col_ok ? (uint32_t)(col * bs_n) : kOOB;

  f32x4 acc[kRG];
#pragma unroll
  for (int q = 0; q < kRG; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nunits = (a.inter + 127) >> 7;
  for (int u0 = wk * U; u0 < nunits; u0 += WK * U) {
    i32x4 braw[kRG][U];
    uint32_t sdw[kRG][U];
#pragma unroll
    for (int q = 0; q < kRG; ++q) {
      if (e[q] >= 0) {
        const i32x4 rB = make_rsrc(a.w + e[q] * b_e, (uint32_t)b_e);
        const i32x4 rS = make_rsrc(a.ws + e[q] * bs_e, (uint32_t)bs_e);
        const uint32_t so = soff + (uint32_t)(u0 * 4);
        if (s_dword) {
          if (U == 4) {
            const i32x4 v = buf_load16(rS, so);
#pragma unroll
            for (int uu = 0; uu < U; ++uu) sdw[q][uu] = (uint32_t)v[uu];
          } else {
            const i32x2 v = buf_load8(rS, so);
#pragma unroll
            for (int uu = 0; uu < U; ++uu) sdw[q][uu] = (uint32_t)v[uu];
          }
        } else {
#pragma unroll
          for (int uu = 0; uu < U; ++uu) sdw[q][uu] = buf_load_u8(rS, so + 4 * uu + grp);
        }
#pragma unroll
        for (int uu = 0; uu < U; ++uu) {
          const int k0 = (u0 + uu) * 128 + grp * 32;
          braw[q][uu] = buf_load16(rB, k0 < a.inter ? boff + (uint32_t)(k0 >> 1) : kOOB);
        }
      } else {
#pragma unroll
        for (int uu = 0; uu < U; ++uu) {
          braw[q][uu] = i32x4{0, 0, 0, 0};
          sdw[q][uu] = 0;
        }
      }
    }
    V8 hf[U][4];
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      const int k0 = (u0 + uu) * 128 + grp * 32;
      const uint32_t o =
          (k0 < a.inter && hoff != kOOB) ? hoff + (uint32_t)(k0 * (int)sizeof(T)) : kOOB;
#pragma unroll
      for (int j = 0; j < 4; ++j) hf[uu][j] = __builtin_bit_cast(V8, buf_load16(rH, o + 16 * j));
    }
#pragma unroll
    for (int q = 0; q < kRG; ++q) {
      if (e[q] < 0) continue;
#pragma unroll
      for (int uu = 0; uu < U; ++uu) {
        // K past the end: weights read as zero; the scale is forced to 1 so
        // bytes of the next row (possibly NaN) cannot leak in
        const bool k_ok = (u0 + uu) * 128 + grp * 32 < a.inter;
        const float sc = e8m0_scale(k_ok ? (sdw[q][uu] >> sshift) & 0xFFu : 127u);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[q] = mfma16(Decode<T>::run((uint32_t)braw[q][uu][j], sc), hf[uu][j], acc[q]);
      }
    }
  }

  // lane l holds D[column (l/16)*4 + i][route l%16]; route c16 belongs to
  // wave c16 / kRG as its accumulator c16 % kRG
  f32x4 res = acc[0];
#pragma unroll
  for (int q = 1; q < kRG; ++q)
    if ((c16 % kRG) == q) res = acc[q];
  if (c16 / kRG == rw) red[wk][lane] = res;
  wait_vmcnt<0>();  // route_wt has landed
  __syncthreads();

  for (int idx = threadIdx.x; idx < tpt * 16; idx += RW * WK * 64) {
    const int tl = idx >> 4;
    const int c = idx & 15;
    if (c >= cw) continue;
    const int64_t t = t0 + tl;
    if (t >= a.m) continue;
    float total = 0.f;
    for (int k = 0; k < a.top_k; ++k) {
      const int rho = tl * a.top_k + k;
      if (!((valid >> rho) & 1)) continue;  // expert outside [0, E)
      const int l = (c >> 2) * 16 + rho;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < WK; ++w) v += red[w][l][c & 3];
      total += to_f32(from_f32<T>(v * route_wt[rho]));
    }
    static_cast<T*>(a.out)[t * a.hidden + blockIdx.x * cw + c] = from_f32<T>(total);
  }
}

template <typename T, int RW>
int launch_rw(const DownArgs& a, int wk, int u, dim3 grid, hipStream_t st) {
  if (u == 4) {
    switch (wk) {
      case 1: moe_down_topk<T, RW, 1, 4><<<grid, RW * 64, 0, st>>>(a); break;
      case 2: moe_down_topk<T, RW, 2, 4><<<grid, RW * 128, 0, st>>>(a); break;
      default: moe_down_topk<T, RW, 4, 4><<<grid, RW * 256, 0, st>>>(a); break;
    }
  } else {
    switch (wk) {
      case 1: moe_down_topk<T, RW, 1, 2><<<grid, RW * 64, 0, st>>>(a); break;
      case 2: moe_down_topk<T, RW, 2, 2><<<grid, RW * 128, 0, st>>>(a); break;
      default: moe_down_topk<T, RW, 4, 2><<<grid, RW * 256, 0, st>>>(a); break;
    }
  }
  return launch_status("moe down+top-k launch");
}

template <typename T>
int launch_typed(const DownArgs& a, hipStream_t st) {
  const int tpt = a.tpt;
  const int rows = tpt * a.top_k;
  const int rw = (rows + kRG - 1) / kRG;
  const int units = (a.inter + 127) / 128;
  // U = 2 units per trip (U = 4 doubles the weight registers and halves
  // occupancy); WK waves split K, at most 4, more trips beyond 8 units
  const int u = 2;
  int wk = (units + u - 1) / u;
  wk = wk <= 1 ? 1 : (wk <= 2 ? 2 : 4);
  const int64_t gy = (a.m + tpt - 1) / tpt;
  if (gy > 65535) {
    set_error("moe down+top-k: too many token tiles (%lld)", (long long)gy);
    return MXFP4_ERR_VALUE;
  }
  dim3 grid((unsigned)(a.hidden / a.cw), (unsigned)gy);
  // When the grid holds more waves than are resident at once (16 per CU
  // at this kernel's ~114 VGPRs), two K waves with up to two trips each
  // beat three or four with one (MoE layer M=8: 42.9 -> 40.0 us; M=1,
  // resident either way, stays on four: 15.1 vs 16.3 us with two)
  if (wk > 2 && (int64_t)grid.x * grid.y * rw * wk > (int64_t)kModelCUs * 16) wk = 2;
  switch (rw) {
    case 1: return launch_rw<T, 1>(a, wk, u, grid, st);
    case 2: return launch_rw<T, 2>(a, wk, u, grid, st);
    case 3: return launch_rw<T, 3>(a, wk, u, grid, st);
    default: return launch_rw<T, 4>(a, wk, u, grid, st);
  }
}

}  // namespace

int launch_moe_down_topk(const void* h, const uint8_t* w2, const uint8_t* s2,
                         const float* topk_weights, const void* topk_ids, int ids64, int64_t m,
                         int top_k, int64_t hidden, int64_t inter, int num_experts, void* out,
                         int dtype, hipStream_t st) {
  if (top_k < 1 || top_k > 16 || hidden % 16 || inter % 32) {
    set_error("moe down+top-k: unsupported shape (top_k %d, hidden %lld, inter %lld)", top_k,
              (long long)hidden, (long long)inter);
    return MXFP4_ERR_VALUE;
  }
  DownArgs a;
  a.h = h;
  a.w = w2;
  a.ws = s2;
  a.route_w = topk_weights;
  a.ids = topk_ids;
  a.out = out;
  a.m = m;
  a.top_k = top_k;
  a.hidden = (int32_t)hidden;
  a.inter = (int32_t)inter;
  a.num_experts = num_experts;
  a.ids64 = ids64;
  // one token per tile: hidden / 16 x m workgroups of ceil(top_k / 4) x WK
  // waves (more tokens per tile would mean fewer, longer workgroups)
  a.tpt = 1;
  // 8 columns per workgroup when 16 would give fewer workgroups than CUs
  // (M=1: 128 -> 256 workgroups; MoE layer at M=1: 15.4 -> 15.1 us)
  a.cw = (hidden / 16) * m < kModelCUs ? 8 : 16;
  if (m == 0) return MXFP4_OK;
  return dtype == MXFP4_DT_BF16 ? launch_typed<__bf16>(a, st) : launch_typed<_Float16>(a, st);
}

}  // namespace mx
