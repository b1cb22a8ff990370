// Arguments shared by the routed / dense MXFP4 GEMM kernels.
//
// One argument block describes both the dense linear (no routing metadata:
// output row i reads activation row i) and the routed grouped GEMM of the
// MoE operator (soft:65-173 / aiter:28-364 semantics): padded position p of
// `sorted_ids` names route r = sorted_ids[p]; r >= num_valid is padding;
// the block of `block_m` positions containing p belongs to expert
// expert_ids[p / block_m] (-1 = not on this device: write zeros); the
// activation row is r / top_k and the output row is r.
#pragma once

#include "common.h"

namespace mx {

enum Epilogue {
  EPI_STORE = 0,     // c = T(acc * alpha [* route_w] [+ bias])
  EPI_SILU_MUL = 1,  // gate/up column pairs -> h = silu(g) * u, rounded like vllm:249-252
  EPI_PARTIAL = 2,   // FP32 partial sums of one K slice (split K, dense only)
  EPI_STORE_F32 = 3, // c = float(acc * alpha [* route_w] [+ bias]): bf16 A, C in FP32 (prefill tiles)
};

struct GemmArgs {
  const void* a;        // activations (T), packed u8 or FP8
  const uint8_t* a_mx;  // A scales [a_rows, k/32] (packed / FP8 A; FP8: may be null = 1)
  int64_t a_rows;       // activation rows addressable through `a`
  int64_t lda;          // A row stride, elements (bytes for packed A)
  int64_t lda_mx;       // A scale row stride, bytes
  const uint8_t* b;     // packed weights, expert-major
  const uint8_t* bs;    // E8M0 weight scales
  int64_t b_e, b_n;     // byte strides: expert, row
  int64_t bs_e, bs_n;
  void* c;
  int64_t ldc;  // output row stride, elements
  const int32_t* sorted_ids;       // nullptr => dense rows
  const int32_t* expert_ids;
  const int32_t* num_post_padded;  // device scalar
  const float* a_scale;            // [1] or nullptr
  const float* b_scale;            // [E] or nullptr
  const float* route_w;            // [num_valid] or nullptr
  const void* bias;                // [n] of T or nullptr (dense)
  int64_t m;          // dense: rows; routed: capacity of sorted_ids (em)
  int64_t num_valid;  // routed: route count (sentinel >= num_valid)
  int32_t n;          // output columns
  int32_t k;          // reduction length (multiple of 32)
  int32_t top_k;      // activation row = route / top_k
  int32_t block_m;    // rows per expert block in sorted_ids
  int32_t inter;      // SiLU epilogue: row offset of the `up` half in B
  int32_t num_experts;  // routed: experts in b; other expert ids act as -1
  // Direct routing (skinny kernel, 16-row blocks): instead of sorted
  // metadata, the top-k ids themselves ([num_valid], int32 or int64).
  // Workgroup row r handles route r if it is the 0th, 16th, ... route of
  // its expert, together with the next 15 routes of that expert.
  const void* route_ids;
  int32_t ids64;
  // direct routing: a route whose id is outside [0, num_experts) writes
  // zeros to its output row (the soft op, every row of C written) instead
  // of being skipped (the MoE layer, whose combine skips it)
  int32_t zero_dropped;
  // Split K (dense, plain epilogue): `splitk` K slices, slice s written as
  // FP32 to splitk_ws + s * m * n, then summed by splitk_reduce.
  float* splitk_ws;
  int32_t splitk;
  // Optional prepacked copy of the weights (prepack.hip), read by the
  // direct-to-LDS prefill kernels instead of b / bs: pre_b = fragment-ordered
  // nibbles [E][G][K/64][512 B], pre_s = the high halves of the FP32 scale
  // operands [E][G][K/64][16 rows][2]; G = 16-row groups; per-expert byte
  // strides.
  const uint8_t* pre_b;
  const uint16_t* pre_s;
  int64_t pre_b_e, pre_s_e;
  // set on the copy a prefill kernel receives: b / bs / b_e / bs_e are then
  // the prepacked arrays
  int32_t prepacked;
  // block-scaled (W4A4) GEMMs: activation format, 0 = packed E2M1, 1 = FP8
  // E4M3, 2 = FP8 E5M2 (FP8 rows are k bytes)
  int32_t a_fp8;
  // routed plain epilogues: scale as the reference's safe MoE path rounds
  // (ref_scaled) instead of once
  int32_t ref_round;
};

// MFMA operand format code of the block-scaled f8f6f4 instructions for
// GemmArgs::a_fp8 (0 -> E2M1 = 4, 1 -> E4M3 = 0, 2 -> E5M2 = 1).
constexpr int mfma_fmt_of(int a_fp8) { return a_fp8 == 0 ? 4 : a_fp8 - 1; }

// Bytes of the prepacked layout of `experts` weight matrices of `rows` x k
// (k % 64 == 0): nibble blocks, then scale operands.
__host__ __device__ inline int64_t prepacked_groups(int64_t rows) { return (rows + 15) / 16; }
__host__ __device__ inline int64_t prepacked_nibble_bytes(int64_t rows, int64_t k) {
  return prepacked_groups(rows) * (k / 64) * 512;
}
__host__ __device__ inline int64_t prepacked_scale_bytes(int64_t rows, int64_t k) {
  return prepacked_groups(rows) * (k / 64) * 64;
}

// Per-row routing lookup used by every kernel.
struct RowInfo {
  int64_t out_row;  // output row (route id or dense row)
  int64_t a_row;    // activation row
  bool valid;
};

__device__ __forceinline__ RowInfo row_info(const GemmArgs& g, int64_t pos) {
  RowInfo ri;
  if (g.sorted_ids == nullptr) {
    ri.valid = pos < g.m;
    ri.out_row = pos;
    ri.a_row = pos;
  } else {
    const int32_t r = g.sorted_ids[pos];
    ri.valid = (r >= 0) && (r < g.num_valid);
    ri.out_row = r;
    ri.a_row = ri.valid ? (r / g.top_k) : 0;
  }
  return ri;
}

// Expert of the routed block holding padded position `pos`; ids outside
// [0, num_experts) are treated as -1 (zeros) instead of addressing memory
// beyond the weights.
__device__ __forceinline__ int block_expert(const GemmArgs& g, int64_t pos) {
  const int e = g.expert_ids[pos / g.block_m];
  return (e >= 0 && e < g.num_experts) ? e : -1;
}

// Number of padded rows in use (routed: read from the device scalar).
__device__ __forceinline__ int64_t rows_in_use(const GemmArgs& g) {
  if (g.sorted_ids == nullptr) return g.m;
  int64_t npp = *g.num_post_padded;
  return npp < g.m ? npp : g.m;
}

// Tile order of the direct-to-LDS kernels; workgroup i runs on XCD i % 8.
// Dense: each XCD gets a contiguous range of tiles, walked in groups of 4
// row blocks, keeping its A rows and B columns L2-resident.  Routed: the
// grid covers the capacity of sorted_ids (nbm rounded up to a multiple of
// 8) but only the first ceil(num_post_padded / bm_rows) row blocks are
// live; those are split into 8 contiguous ranges of equal size, one per
// XCD, each XCD walking all column tiles of a row block before the next.
// Consecutive row blocks mostly belong to one expert, so an expert's
// weights are fetched into few L2s, and every XCD gets an equal share of
// the live rows.  Returns false for workgroups past the live range.
__device__ __forceinline__ bool tile_of(const GemmArgs& g, int bm_rows, int nbm, int nbn, int& bm,
                                        int& bn, int idx, int nwg) {
  const int x = idx % 8, i = idx / 8;
  if (g.sorted_ids) {
    const int live = (int)((rows_in_use(g) + bm_rows - 1) / bm_rows);
    const int lo = (int)((int64_t)live * x / 8), hi = (int)((int64_t)live * (x + 1) / 8);
    bm = lo + i / nbn;
    bn = i % nbn;
    return bm < hi;
  }
  const int per = nwg / 8, rem = nwg % 8;
  const int pid = x * per + (x < rem ? x : rem) + i;
  constexpr int GROUP = 4;
  const int first_m = (pid / (GROUP * nbn)) * GROUP;
  const int gsize = (nbm - first_m) < GROUP ? (nbm - first_m) : GROUP;
  bm = first_m + (pid % (GROUP * nbn)) % gsize;
  bn = (pid % (GROUP * nbn)) / gsize;
  return (int64_t)bm * bm_rows < g.m;
}

__device__ __forceinline__ float scalar_alpha(const GemmArgs& g, int expert) {
  float a = g.a_scale ? g.a_scale[0] : 1.0f;
  if (g.b_scale) a *= g.b_scale[expert];
  return a;
}

// The reference's safe MoE path in compute dtype OutT (soft:487-494) takes
// the GEMM's result in OutT, multiplies it by a_scale and rounds to OutT,
// then by b_scale[e] and rounds to OutT; the route weight (an FP32 tensor)
// then multiplies in FP32 and the store rounds.  With g.ref_round the
// plain routed epilogues follow that sequence: the FP32 sum goes through
// ref_scaled and the epilogue's own scalar becomes 1.  (By default the sum
// is multiplied by a_scale * b_scale[e] and rounded once, as the
// reference's Triton kernel does, soft:167-173.)  Identity roundings for
// OutT = float.
template <typename OutT>
__device__ __forceinline__ float ref_scaled(const GemmArgs& g, float acc, int expert) {
  float v = to_f32(from_f32<OutT>(acc));
  if (g.a_scale) v = to_f32(from_f32<OutT>(v * g.a_scale[0]));
  if (g.b_scale) v = to_f32(from_f32<OutT>(v * g.b_scale[expert]));
  return v;
}

// ref_scaled over a tile's accumulators (expert >= 0); the epilogue's own
// scalar is then 1.
template <typename OutT, int FM, int FN>
__device__ __forceinline__ void ref_pass(const GemmArgs& g, int expert, f32x4 (&acc)[FM][FN]) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = ref_scaled<OutT>(g, acc[i][j][e], expert);
}

// Host-side launchers (gemm_w4a16.hip, gemm_w4a4.hip).
int launch_w4a16(const GemmArgs& g, int dtype, int epi, hipStream_t st);
// Direct-to-LDS prefill kernel (gemm_w4a16_pf.hip): tile configurations.
enum PfConfig {
  PF_128x256 = 0,  // 1 x 4 waves of 128 x 64
  PF_128x128 = 1,  // 1 x 4 waves of 128 x 32
  PF_64x128 = 2,   // 1 x 4 waves of 64 x 32, 3 stages
  PF_32x128 = 3,   // 1 x 4 waves of 32 x 32, 3 stages
  PF_128x320 = 4,  // 1 x 4 waves of 128 x 80 (plain store epilogue only)
  PF_256x320 = 5,  // 2 x 4 waves of 128 x 80, one per CU (dense, plain store only)
  PF_256x256 = 6,  // 2 x 4 waves of 128 x 64, one per CU (dense, plain store only)
  PF_64x256 = 7,   // 1 x 4 waves of 64 x 64, 3 stages (routed 64-row blocks)
  PF_32x256 = 8,   // 1 x 4 waves of 32 x 64, 3 stages (routed 32-row blocks)
  PF_32x384 = 9,   // 1 x 4 waves of 32 x 96, 2 stages (routed 32-row blocks, SiLU)
  PF_32x512 = 10,  // 1 x 4 waves of 32 x 128, 2 stages (routed 32-row blocks)
  PF_64x384 = 11,  // 1 x 4 waves of 64 x 96, 2 stages (routed 64-row blocks, SiLU)
};
bool pf_supported(const GemmArgs& g, int elem_bytes);
// The prepacked weights of g (pre_b / pre_s) can replace b / bs.
bool pf_prepacked_usable(const GemmArgs& g);
// Compute units of the current device (cached per device; 0 if unknown).
int device_cus();
int pf_choose(const GemmArgs& g, int epi);
int launch_w4a16_pf(const GemmArgs& g, int dtype, int epi, int cfg, hipStream_t st);
// Split-K plan for a dense plain-epilogue GEMM whose tiles would not fill
// the chip: the tile configuration and slice count (1 = no split).
struct SplitPlan {
  int cfg, splits;
};
SplitPlan splitk_plan(int64_t m, int64_t k, int64_t n);
// Rows per skinny block (1 or 2 x 16) the dense W4A16 GEMM of these sizes
// runs with, 0 for the prefill kernels; split_ok: a split-K workspace is given.
int dense_skinny_rows(int64_t m, int64_t k, int64_t n, bool split_ok);
int64_t splitk_ws_bytes(int64_t m, int64_t k, int64_t n);
// Sums the FP32 slices, adds the bias and rounds to T (dtype) into g.c.
int launch_splitk_reduce(const GemmArgs& g, int dtype, hipStream_t st);
int launch_w4a4(const GemmArgs& g, int out_dtype, hipStream_t st);
// Direct-to-LDS W4A4 kernel (gemm_w4a4_pf.hip).
enum P4Config {
  P4_256x256 = 0,  // 2 x 4 waves of 128 x 64, 3 stages
  P4_128x128 = 1,  // 1 x 4 waves of 128 x 32
  P4_64x128 = 2,   // 1 x 4 waves of 64 x 32
  P4_32x128 = 3,   // 1 x 4 waves of 32 x 32 (routed 32-row blocks)
};
bool p4_supported(const GemmArgs& g);
int p4_choose(const GemmArgs& g, int out_dtype);  // -1: not applicable
int launch_w4a4_pf(const GemmArgs& g, int out_dtype, int cfg, hipStream_t st);
int launch_f32_reference(const GemmArgs& g, int a_dtype, hipStream_t st);
// MoE decode: down projection fused with the top-k combine (moe_decode.hip);
// h holds the m * top_k routes' rows of width inter in route order.
int launch_moe_down_topk(const void* h, const uint8_t* w2, const uint8_t* s2,
                         const float* topk_weights, const void* topk_ids, int ids64, int64_t m,
                         int top_k, int64_t hidden, int64_t inter, int num_experts, void* out,
                         int dtype, hipStream_t st);

}  // namespace mx
