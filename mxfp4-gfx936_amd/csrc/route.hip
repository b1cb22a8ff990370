// MoE router on the device: softmax over the experts, top-k, optional
// renormalisation -- the step that produces the topk_weights / topk_ids the
// MoE layer consumes (vllm:233-265), built the way the reference tests build
// them (test:242-244: softmax -> torch.topk) and, with renormalisation, the
// way the MoE benchmark configuration does (softmax -> top-k -> w / sum w).
//
// L lanes per token row (16 when E <= 256 and k <= 16: four rows per wave;
// else 64); lane l of a row holds the logits of experts l, l + L, ...
// Selection compares logits, not probabilities: softmax is monotonic, so the
// top-k of the probabilities is the top-k of the logits, with no rounding in
// between.  k rounds of an argmax over the row's lanes, ties to the lower
// expert id; slot r of the result is the r-th largest.  A few rows take as
// long as one chain of k argmax reductions, hence DPP for the cross-lane
// steps (below).  Weights:
//   p_i = exp(l_i - max) / sum_j exp(l_j - max)
//   renormalised: p_i / sum_{s selected} p_s = exp(l_i - max) / sum_s exp(l_s - max)
// (the full denominator cancels).  FP32 throughout; the sums run as a wave
// reduction, so they differ from a sequential sum by a few ulps.
#include <climits>
#include <math.h>

#include "common.h"

namespace mx {
namespace {

// Cross-lane steps through DPP (a VALU operand modifier) rather than LDS
// permutes: row_shr:1/2/4/8 gather each 16-lane row into its lane 15,
// row_bcast:15 / row_bcast:31 carry rows 0-2 into lane 63, which holds the
// wave's result; a source lane outside the row (or a row not in the mask)
// yields `old`, the operation's identity.
constexpr int kShr1 = 0x111, kShr2 = 0x112, kShr4 = 0x114, kShr8 = 0x118;
constexpr int kBcast15 = 0x142, kBcast31 = 0x143;
// row_ror:n rotates within each 16-lane row: combining with rotations by
// 1, 2, 4, 8 leaves the row's result in every lane of the row
constexpr int kRor1 = 0x121, kRor2 = 0x122, kRor4 = 0x124, kRor8 = 0x128;

template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dppf(float old, float v) {
  return __int_as_float(dpp<CTRL, ROWS>(__float_as_int(old), __float_as_int(v)));
}

// sum over the row of L lanes (16 or 64), returned to every lane of the row
template <int L>
__device__ __forceinline__ float row_sum(float v) {
  if constexpr (L == 16) {
    v += dppf<kRor1, 0xF>(0.f, v);
    v += dppf<kRor2, 0xF>(0.f, v);
    v += dppf<kRor4, 0xF>(0.f, v);
    v += dppf<kRor8, 0xF>(0.f, v);
    return v;
  }
  v += dppf<kShr1, 0xF>(0.f, v);
  v += dppf<kShr2, 0xF>(0.f, v);
  v += dppf<kShr4, 0xF>(0.f, v);
  v += dppf<kShr8, 0xF>(0.f, v);
  v += dppf<kBcast15, 0xA>(0.f, v);
  v += dppf<kBcast31, 0xC>(0.f, v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// (logit, expert) pair: larger logit first, then lower expert id (a total
// order); bi == INT_MAX is "none"
__device__ __forceinline__ void take_better(float& best, int& bi, float ov, int oi) {
  if (oi != INT_MAX && (bi == INT_MAX || ov > best || (ov == best && oi < bi))) {
    best = ov;
    bi = oi;
  }
}

template <int CTRL, int ROWS>
__device__ __forceinline__ void argmax_step(float& best, int& bi) {
  const float ov = dppf<CTRL, ROWS>(-INFINITY, best);
  const int oi = dpp<CTRL, ROWS>(INT_MAX, bi);
  take_better(best, bi, ov, oi);
}

// argmax over the row of L lanes, returned to every lane of the row
template <int L>
__device__ __forceinline__ void row_argmax(float& best, int& bi) {
  if constexpr (L == 16) {
    argmax_step<kRor1, 0xF>(best, bi);
    argmax_step<kRor2, 0xF>(best, bi);
    argmax_step<kRor4, 0xF>(best, bi);
    argmax_step<kRor8, 0xF>(best, bi);
  } else {
    argmax_step<kShr1, 0xF>(best, bi);
    argmax_step<kShr2, 0xF>(best, bi);
    argmax_step<kShr4, 0xF>(best, bi);
    argmax_step<kShr8, 0xF>(best, bi);
    argmax_step<kBcast15, 0xA>(best, bi);
    argmax_step<kBcast31, 0xC>(best, bi);
    best = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best), 63));
    bi = __builtin_amdgcn_readlane(bi, 63);
  }
}

template <int L, int J, typename ID>
__global__ __launch_bounds__(256) void route_topk(const float* __restrict__ logits, int64_t m,
                                                  int ne, int64_t ld, int top_k, int renorm,
                                                  float* __restrict__ w_out,
                                                  ID* __restrict__ id_out) {
  static_assert(L == 16 || L == 64, "16 or 64 lanes per row");
  const int lane = threadIdx.x & (L - 1);  // lane within the row
  const int64_t row = (int64_t)blockIdx.x * (256 / L) + threadIdx.x / L;
  if (row >= m) return;  // whole rows of lanes; no barriers
  const float* lr = logits + row * ld;
  float v[J];
#pragma unroll
  for (int j = 0; j < J; ++j) v[j] = lane + L * j < ne ? lr[lane + L * j] : -INFINITY;

  uint32_t taken = 0;  // bit j: expert lane + L j already selected
  float mine = -INFINITY;  // slot `lane` (lanes < top_k): logit and expert
  int mine_id = 0;
  float top = 0.f;  // the row's largest logit (first argmax pass)
  for (int r = 0; r < top_k; ++r) {
    // the lane's best unselected expert (ascending j: ties keep the lower id)
    float best = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = lane + L * j;
      if (e < ne && !((taken >> j) & 1u) && (bi == INT_MAX || v[j] > best)) {  // ties: lower j
        best = v[j];
        bi = e;
      }
    }
    row_argmax<L>(best, bi);
    if (r == 0) top = best;
    if (lane == r) {
      mine = best;
      mine_id = bi;
    }
    if ((bi & (L - 1)) == lane) taken |= 1u << (bi / L);
  }

  const float ex = lane < top_k ? expf(mine - top) : 0.f;
  float denom;
  if (renorm) {
    denom = row_sum<L>(ex);
  } else {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (lane + L * j < ne) s += expf(v[j] - top);
    denom = row_sum<L>(s);
  }
  if (lane < top_k) {
    w_out[row * top_k + lane] = ex / denom;
    id_out[row * top_k + lane] = (ID)mine_id;
  }
}

template <int L, typename ID>
void launch_rows(const float* logits, int64_t m, int ne, int64_t ld, int top_k, int renorm,
                 float* w, ID* ids, hipStream_t st) {
  constexpr int R = 256 / L;  // rows per workgroup
  const unsigned grid = (unsigned)((m + R - 1) / R);
  const int j = (ne + L - 1) / L;
  if (j <= 1) route_topk<L, 1, ID><<<grid, 256, 0, st>>>(logits, m, ne, ld, top_k, renorm, w, ids);
  else if (j <= 2) route_topk<L, 2, ID><<<grid, 256, 0, st>>>(logits, m, ne, ld, top_k, renorm, w, ids);
  else if (j <= 4) route_topk<L, 4, ID><<<grid, 256, 0, st>>>(logits, m, ne, ld, top_k, renorm, w, ids);
  else if (j <= 8) route_topk<L, 8, ID><<<grid, 256, 0, st>>>(logits, m, ne, ld, top_k, renorm, w, ids);
  else route_topk<L, 16, ID><<<grid, 256, 0, st>>>(logits, m, ne, ld, top_k, renorm, w, ids);
}

template <typename ID>
int launch_route(const float* logits, int64_t m, int ne, int64_t ld, int top_k, int renorm,
                 float* w, ID* ids, hipStream_t st) {
  // 16 lanes per row (4 rows per wave) while a row's logits fit 16 per
  // lane and its slots one per lane
  if (ne <= 256 && top_k <= 16) launch_rows<16>(logits, m, ne, ld, top_k, renorm, w, ids, st);
  else launch_rows<64>(logits, m, ne, ld, top_k, renorm, w, ids, st);
  return launch_status("router launch");
}

}  // namespace
}  // namespace mx

extern "C" int mxfp4_moe_route(const float* logits, int64_t m, int num_experts,
                               int64_t row_stride, int top_k, int renormalize,
                               float* topk_weights, void* topk_ids, int ids_dtype, void* stream) {
  using namespace mx;
  if (ids_dtype != MXFP4_DT_I32 && ids_dtype != MXFP4_DT_I64) {
    set_error("router: topk_ids must be int32 or int64 (dtype code %d)", ids_dtype);
    return MXFP4_ERR_TYPE;
  }
  if (m < 0 || num_experts < 1 || num_experts > 1024 || top_k < 1 || top_k > num_experts ||
      top_k > 64 || row_stride < num_experts) {
    set_error("router: invalid sizes (m %lld, experts %d, top_k %d, row stride %lld)",
              (long long)m, num_experts, top_k, (long long)row_stride);
    return MXFP4_ERR_VALUE;
  }
  if ((m + 3) / 4 > 0x7FFFFFFF) {
    set_error("router: too many rows (%lld)", (long long)m);
    return MXFP4_ERR_VALUE;
  }
  if (m == 0) return MXFP4_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (ids_dtype == MXFP4_DT_I64)
    return launch_route(logits, m, num_experts, row_stride, top_k, renormalize != 0, topk_weights,
                        static_cast<int64_t*>(topk_ids), st);
  return launch_route(logits, m, num_experts, row_stride, top_k, renormalize != 0, topk_weights,
                      static_cast<int32_t*>(topk_ids), st);
}
