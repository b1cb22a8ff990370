/*
 * libmxfp4_gfx950 -- C ABI of the MI355X (gfx950) MXFP4 backend.
 *
 * Drop-in replacement for the `moe_op_mxfp4_soft` operator surface of
 * lutianshu824/mxfp4-gfx936.  Reference paths below are relative to that
 * repository:
 *   soft  = src/aiter/ops/triton/moe_op_mxfp4_soft.py
 *   aiter = integration/aiter/moe_op_mxfp4.py
 *   vllm  = integration/vllm/vllm_mxfp4_gfx936.py
 *   test  = tests/test_moe_mxfp4_soft.py
 *
 * Conventions
 *   - Every pointer argument is device memory on the current HIP device,
 *     except where a comment says otherwise.  The caller owns all memory; the
 *     library allocates nothing on the device and never synchronises the host.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     All work is enqueued asynchronously on it, in order.
 *   - Packed MXFP4: two E2M1 codes per byte, low nibble = even K index;
 *     one E8M0 byte per 32 K values (value 2^(s-127), s = 255 is NaN).
 *   - Rows are K-contiguous; *_row_stride arguments are in elements of the
 *     tensor (bytes for uint8 tensors).  Packed/activation rows and their base
 *     pointers must be 16-byte aligned.
 *   - Every entry point returns MXFP4_OK (0) or an error class below and
 *     leaves a message for mxfp4_last_error().  Argument errors are detected
 *     before anything is enqueued.
 */
#ifndef MXFP4_GFX950_H_
#define MXFP4_GFX950_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error classes; the Python layer raises the exception named beside each,
 * matching the reference's conventions (soft:283-294, 317-329, 398-407). */
enum {
  MXFP4_OK = 0,
  MXFP4_ERR_TYPE = 1,            /* TypeError: unsupported dtype */
  MXFP4_ERR_VALUE = 2,           /* ValueError: shapes, K divisibility */
  MXFP4_ERR_NOT_IMPLEMENTED = 3, /* NotImplementedError: swizzled scales */
  MXFP4_ERR_RUNTIME = 4,         /* RuntimeError: unsupported metadata */
  MXFP4_ERR_HIP = 5              /* RuntimeError: HIP launch/runtime failure */
};

/* Element types. */
enum {
  MXFP4_DT_F32 = 0,
  MXFP4_DT_BF16 = 1,
  MXFP4_DT_F16 = 2,
  MXFP4_DT_U8 = 3, /* packed E2M1 pairs */
  MXFP4_DT_I32 = 4,
  MXFP4_DT_I64 = 5,
  MXFP4_DT_F8E4M3 = 6, /* OCP FP8 E4M3 (torch.float8_e4m3fn) */
  MXFP4_DT_F8E5M2 = 7  /* OCP FP8 E5M2 (torch.float8_e5m2) */
};

/* Quantizer rounding modes for mxfp4_quant. */
enum {
  MXFP4_QUANT_TIES_AWAY = 0, /* the reference test quantizer, test:28-60 */
  MXFP4_QUANT_RNE = 1        /* OCP MX: E = floor(log2 amax) - 2, E2M1 RNE */
};

/* Message of the last failing call on this host thread ("" if none). */
const char* mxfp4_last_error(void);

/* ABI version of this library (MXFP4_ABI_VERSION). */
#define MXFP4_ABI_VERSION 1
int mxfp4_abi_version(void);

/*
 * dequant_mxfp4(packed, block_scales, dtype) -- soft:277-307.
 * packed u8 [rows, k/2], scales u8 [rows, k/32] -> out [rows, k] of out_dtype
 * (F32, BF16 or F16), contiguous.  Bit-exact with the reference: the FP32
 * product LUT[code] * 2^(s-127) rounded to out_dtype with RNE; s = 255 gives
 * the canonical NaN (0x7FC00000 / 0x7FC0 / 0x7E00).  k % 32 == 0.
 */
int mxfp4_dequant(const uint8_t* packed, int64_t packed_row_stride, const uint8_t* scales,
                  int64_t scale_row_stride, int64_t rows, int64_t k, void* out, int out_dtype,
                  void* stream);

/*
 * linear_mxfp4_soft(x, packed, block_scales, bias) -- soft:310-376.
 * x [m, k] (BF16 or F16, row stride x_row_stride elements), W packed u8
 * [n, k/2], S u8 [n, k/32] (both contiguous) -> out [m, n] contiguous, same
 * dtype as x:  out = x . dequant(W, S)^T (+ bias), FP32 accumulation, one
 * rounding.  bias (optional, NULL for none) is [n] of x's dtype.
 * k % 128 == 0 (soft:326-327).
 */
int mxfp4_linear_w4a16(const void* x, int x_dtype, int64_t m, int64_t k, int64_t x_row_stride,
                       const uint8_t* packed, const uint8_t* scales, int64_t n, const void* bias,
                       void* out, void* stream);

/*
 * The same operation (soft:310-376) with a caller-provided device workspace
 * of at least the bytes mxfp4_linear_w4a16_workspace_size(m, k, n, &bytes)
 * reports, 16-byte aligned.  A non-zero size means the GEMM is too small to
 * fill the GPU: K is then split into slices whose FP32 partial sums go
 * through the workspace and are added in a fixed order (deterministic, but
 * not bitwise equal to the unsplit sum).  workspace may be NULL (no split).
 */
int mxfp4_linear_w4a16_workspace_size(int64_t m, int64_t k, int64_t n, int64_t* bytes);
int mxfp4_linear_w4a16_ws(const void* x, int x_dtype, int64_t m, int64_t k, int64_t x_row_stride,
                          const uint8_t* packed, const uint8_t* scales, int64_t n,
                          const void* bias, void* out, void* workspace, int64_t workspace_bytes,
                          void* stream);

/*
 * Prepacked weights -- the offline repack that aiter:189-205, 229-248 leave
 * to the kernel's own swizzled scale layouts (soft:398-399 refuses them), done
 * once at weight load (vllm:68-70, process_weights_after_loading).  packed
 * u8 [experts, rows, k/2] and scales u8 [experts, rows, k/32] (contiguous,
 * packed 4-byte aligned) -> pre_b [experts][ceil(rows/16)][k/64][512 B]
 * and pre_s [experts][ceil(rows/16)][k/64][16][2] u16, sizes from
 * mxfp4_prepack_w4a16_size, both 16-byte aligned.  Per 16-row group and
 * 64-deep K step, pre_b holds the nibbles in the order the prefill kernels
 * read their MFMA fragments (lane l: bytes s*32 + j*16 + (l/16)*4 .. +3 of
 * row l % 16, j = 0, 1) and pre_s the high halves of the conversion scale
 * operands ((byte << 7) | 0x40: the float (byte << 23) | 0x400000).  Rows
 * past `rows` are zero.  k % 64 == 0.  A copy is valid for the weights it
 * was made from: after they change, prepack again.
 */
int mxfp4_prepack_w4a16_size(int64_t experts, int64_t rows, int64_t k, int64_t* nibble_bytes,
                             int64_t* scale_bytes);
int mxfp4_prepack_w4a16(const uint8_t* packed, const uint8_t* scales, int64_t experts,
                        int64_t rows, int64_t k, uint8_t* pre_b, uint16_t* pre_s, void* stream);

/*
 * mxfp4_linear_w4a16_ws (soft:310-376) that also takes the prepacked copy
 * of (packed, scales) made by mxfp4_prepack_w4a16 with experts = 1, rows =
 * n.  The prefill kernels then read pre_b / pre_s instead of packed /
 * scales; the result is bitwise equal.  pre_b and pre_s are both NULL (the
 * plain call) or both set.
 */
int mxfp4_linear_w4a16_pre(const void* x, int x_dtype, int64_t m, int64_t k, int64_t x_row_stride,
                           const uint8_t* packed, const uint8_t* scales, const uint8_t* pre_b,
                           const uint16_t* pre_s, int64_t n, const void* bias, void* out,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Dense W4A4: both operands packed MXFP4, on gfx950's block-scaled MFMA
 * (the packed-A semantics of aiter:206-214, 329-338 with one expert).
 * a u8 [m, k/2], a_mx u8 [m, k/32], b u8 [n, k/2], b_mx u8 [n, k/32] (all
 * contiguous) -> out [m, n] of out_dtype (BF16, F16 or F32).  k % 32 == 0.
 */
int mxfp4_linear_w4a4(const uint8_t* a, const uint8_t* a_mx, int64_t m, int64_t k,
                      const uint8_t* b, const uint8_t* b_mx, int64_t n, void* out, int out_dtype,
                      void* stream);

/*
 * Routing metadata on the device -- the format of vllm:119-146 (consumed as
 * in soft:101-108).  topk_ids [num_routes] (I32 or I64; route r = token *
 * top_k + slot) -> sorted_ids (route ids grouped by ascending expert,
 * ascending inside an expert, each expert padded to block_m with the
 * sentinel num_routes), expert_ids (one per block), num_post_padded[0] =
 * number of entries used in sorted_ids.  Ids outside [0, num_experts) are
 * dropped (their rows are left untouched by the GEMMs, as in soft:478-481).
 * Deterministic.  Capacities come from mxfp4_moe_align_sizes; `workspace`
 * must hold align_workspace_bytes bytes.
 */
int mxfp4_moe_align_sizes(int64_t num_routes, int num_experts, int block_m, int64_t* max_sorted,
                          int64_t* max_blocks, int64_t* align_workspace_bytes);
int mxfp4_moe_align(const void* topk_ids, int ids_dtype, int64_t num_routes, int num_experts,
                    int block_m, int32_t* sorted_ids, int32_t* expert_ids,
                    int32_t* num_post_padded, void* workspace, int64_t workspace_bytes,
                    void* stream);

/*
 * Router -- the topk_weights / topk_ids the MoE layer consumes (vllm:233-265),
 * built as the reference tests build them (test:242-244: softmax over the
 * experts, then torch.topk) and, with renormalize != 0, divided by their sum
 * (the MoE benchmark configuration).  logits F32 [m, num_experts] (row
 * stride in elements) -> topk_weights F32 [m, top_k] and topk_ids (I32 or
 * I64) [m, top_k], contiguous; slot r holds the r-th most probable expert,
 * ties to the lower expert id.  Logits must be finite.  num_experts <= 1024,
 * 1 <= top_k <= min(num_experts, 64).
 */
int mxfp4_moe_route(const float* logits, int64_t m, int num_experts, int64_t row_stride,
                    int top_k, int renormalize, float* topk_weights, void* topk_ids, int ids_dtype,
                    void* stream);

/*
 * Routed grouped GEMM -- the compute of fused_moe_mxfp4_soft, soft:379-494,
 * and of AITER's fused_moe_mxfp4, aiter:28-364.
 *   a: activations [a_rows, k]: BF16/F16/F32 (a_dtype), or packed u8
 *      [a_rows, k/2] with a_mx u8 [a_rows, k/32] (a_dtype = MXFP4_DT_U8), or
 *      OCP FP8 [a_rows, k] (a_dtype = MXFP4_DT_F8E4M3 / F8E5M2; the e4m3 /
 *      e5m2 formats aiter:11-20 maps into tl.dot_scaled) with a_mx u8
 *      [a_rows, k/32] or NULL (every scale 1) -- packed and FP8 A run on the
 *      block-scaled f8f6f4 MFMA, each product A * 2^(sa-127) * B * 2^(sb-127)
 *      exact, FP32 accumulation.
 *   b u8 [num_experts, n, k/2], b_mx u8 [num_experts, n, k/32], contiguous.
 *   c: output rows indexed by route id, c + route * c_row_stride, of c_dtype
 *      (BF16, F16 or F32; the compute type of soft:405-407).  BF16 / F16 A
 *      must match c_dtype, except with F32 c, where they are widened
 *      exactly (BF16 A on blocks of 32k rows: the bf16 MFMA's exact
 *      products, FP32 sums; otherwise the FP32 MFMA).
 *   For each block i < num_post_padded[0] / block_m with expert
 *   e = expert_ids[i] and each route r = sorted_ids[i*block_m + j] <
 *   num_valid:  c[r, :] = a[r / top_k] . dequant(b[e])^T * a_scale[0] *
 *   b_scale[e] (* topk_weights[r] if mul_routed_weight), rounded once to
 *   c_dtype.  mul_routed_weight is a bit set: bit 0 multiplies the route
 *   weights; bit 1 (no counterpart in the reference's Triton kernels)
 *   scales as the reference's safe path rounds, soft:487-494: the sum
 *   rounded to c_dtype, times a_scale[0] rounded to c_dtype, times
 *   b_scale[e] rounded to c_dtype, times the route weight in FP32, then
 *   rounded.  Expert -1 writes zeros (aiter:156-172); so does any other id
 *   outside [0, num_experts).  Rows not named by the metadata are not
 *   written.  a_scale / b_scale may be NULL (= 1).  block_m % 16 == 0;
 *   k % 32 == 0; em = capacity of sorted_ids; expert_ids holds em / block_m
 *   entries, any of which may be read.
 */
int mxfp4_moe_gemm(const void* a, int a_dtype, int64_t a_rows, int64_t a_row_stride,
                   const uint8_t* a_mx, const uint8_t* b, const uint8_t* b_mx,
                   int64_t num_experts, int64_t n, int64_t k, void* c, int c_dtype,
                   int64_t c_row_stride, const float* a_scale, const float* b_scale,
                   const float* topk_weights, int mul_routed_weight, const int32_t* sorted_ids,
                   const int32_t* expert_ids, const int32_t* num_post_padded, int64_t em,
                   int block_m, int64_t num_valid, int top_k, void* stream);
/* mxfp4_moe_gemm with a prepacked copy of b / b_mx (mxfp4_prepack_w4a16 of
 * the same num_experts x n x k weights, 16-byte aligned), which the W4A16
 * prefill kernels read instead; bitwise the same c.  pre_b = pre_s = NULL is
 * mxfp4_moe_gemm.  b / b_mx are still required (the decode kernels and the
 * W4A4 / FP32 paths read them).  The reference has no such argument: it is
 * what the soft op's and AITER's entries (soft:379, aiter:300) use when the
 * caller has registered a prepacked copy of B. */
int mxfp4_moe_gemm_pre(const void* a, int a_dtype, int64_t a_rows, int64_t a_row_stride,
                       const uint8_t* a_mx, const uint8_t* b, const uint8_t* b_mx,
                       const uint8_t* pre_b, const uint16_t* pre_s, int64_t num_experts,
                       int64_t n, int64_t k, void* c, int c_dtype, int64_t c_row_stride,
                       const float* a_scale, const float* b_scale, const float* topk_weights,
                       int mul_routed_weight, const int32_t* sorted_ids,
                       const int32_t* expert_ids, const int32_t* num_post_padded, int64_t em,
                       int block_m, int64_t num_valid, int top_k, void* stream);

/*
 * fused_moe_mxfp4_soft(A, B, C, A_scale, B_scale, A_mx_scale, B_mx_scale,
 * topk_weights, topk_ids, ...) -- soft:379-494, safe semantics, in one call
 * (the routing metadata arguments, which soft:466 ignores, are not taken).
 * a, a_mx, b, b_mx, a_scale, b_scale, topk_weights, mul_routed_weight as in
 * mxfp4_moe_gemm; topk_ids I32/I64 [m, top_k]; c [m, top_k, n] contiguous,
 * 16-byte aligned, of c_dtype.  Every element of c is written: for each
 * (t, s) with e = topk_ids[t, s] in [0, num_experts)
 *   c[t, s, :] = a[t] . dequant(b[e])^T * a_scale[0] * b_scale[e]
 *                (* topk_weights[t, s] if mul_routed_weight),
 * FP32 accumulation, one rounding; every other row is zero (soft:476: C is
 * zero-filled first -- here only the rows no GEMM row covers are written
 * with zeros, which gives the same C).  Routing is built on the device; no
 * host synchronisation.  `workspace` (16-byte aligned) must hold
 * mxfp4_fused_moe_workspace_size bytes.  num_experts <= 1024.
 */
int mxfp4_fused_moe_workspace_size(int64_t m, int top_k, int64_t num_experts, int a_dtype,
                                   int c_dtype, int64_t* bytes);
int mxfp4_fused_moe(const void* a, int a_dtype, int64_t a_rows, int64_t a_row_stride,
                    const uint8_t* a_mx, const uint8_t* b, const uint8_t* b_mx,
                    int64_t num_experts, int64_t n, int64_t k, void* c, int c_dtype,
                    const float* a_scale, const float* b_scale, const float* topk_weights,
                    int mul_routed_weight, const void* topk_ids, int ids_dtype, int64_t m,
                    int top_k, void* workspace, int64_t workspace_bytes, void* stream);
/* mxfp4_fused_moe with a prepacked copy of b / b_mx, as mxfp4_moe_gemm_pre
 * (bitwise the same c; with the copy the routing blocks follow the MoE
 * layer's 16 / 32 / 64-row rule, which the workspace size covers). */
int mxfp4_fused_moe_pre(const void* a, int a_dtype, int64_t a_rows, int64_t a_row_stride,
                        const uint8_t* a_mx, const uint8_t* b, const uint8_t* b_mx,
                        const uint8_t* pre_b, const uint16_t* pre_s, int64_t num_experts,
                        int64_t n, int64_t k, void* c, int c_dtype, const float* a_scale,
                        const float* b_scale, const float* topk_weights, int mul_routed_weight,
                        const void* topk_ids, int ids_dtype, int64_t m, int top_k,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The vLLM MoE layer, vllm:233-265 (silu only):
 *   gu = moe(x, w13)                  [m, top_k, 2*inter] rounded to x's dtype
 *   h  = silu(gu[..., :inter]) * gu[..., inter:]   (rounded as the reference)
 *   d  = moe(h, w2) * topk_weights    [m*top_k, hidden]
 *   out = sum over top_k of d          [m, hidden], FP32 sum, one rounding
 * x [m, hidden] BF16/F16 contiguous; w13 u8 [E, 2*inter, hidden/2],
 * s13 u8 [E, 2*inter, hidden/32], w2 u8 [E, hidden, inter/2],
 * s2 u8 [E, hidden, inter/32]; topk_weights F32 [m, top_k]; topk_ids I32/I64
 * [m, top_k].  SiLU*mul is fused into the gate_up epilogue and the route
 * weight into the down epilogue.  `workspace` must hold
 * mxfp4_moe_layer_workspace_size bytes (routing metadata + intermediates).
 */
int mxfp4_moe_layer_workspace_size(int64_t m, int top_k, int num_experts, int64_t hidden,
                                   int64_t inter, int64_t* bytes);
int mxfp4_moe_layer(const void* x, int x_dtype, int64_t m, int64_t hidden, const uint8_t* w13,
                    const uint8_t* s13, const uint8_t* w2, const uint8_t* s2, int num_experts,
                    int64_t inter, const float* topk_weights, const void* topk_ids, int ids_dtype,
                    int top_k, void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mxfp4_moe_layer (vllm:233-265) with the prepacked copies of w13 / s13
 * (rows = 2*inter, k = hidden) and w2 / s2 (rows = hidden, k = inter) from
 * mxfp4_prepack_w4a16 with experts = num_experts.  Each pair is both NULL
 * or both set; the result is bitwise equal to mxfp4_moe_layer's.
 */
int mxfp4_moe_layer_pre(const void* x, int x_dtype, int64_t m, int64_t hidden, const uint8_t* w13,
                        const uint8_t* s13, const uint8_t* pre13_b, const uint16_t* pre13_s,
                        const uint8_t* w2, const uint8_t* s2, const uint8_t* pre2_b,
                        const uint16_t* pre2_s, int num_experts, int64_t inter,
                        const float* topk_weights, const void* topk_ids, int ids_dtype, int top_k,
                        void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mxfp4_moe_layer without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The layer's workspace is a fixed device array of
 * MXFP4_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs
 * on until the process ends; nothing is allocated per call.  Returns
 * MXFP4_ERR_VALUE when mxfp4_moe_layer_workspace_size exceeds that size
 * (with E=128, top-8, hidden 2048 and inter 768: up to ~700 tokens).  Calls that overlap on one GPU share the array and race: issue
 * them on one stream, or order them.  Otherwise as mxfp4_moe_layer.
 */
#define MXFP4_NOALLOC_SCRATCH_BYTES (32LL << 20)
int mxfp4_moe_layer_noalloc(const void* x, int x_dtype, int64_t m, int64_t hidden,
                            const uint8_t* w13, const uint8_t* s13, const uint8_t* w2,
                            const uint8_t* s2, int num_experts, int64_t inter,
                            const float* topk_weights, const void* topk_ids, int ids_dtype,
                            int top_k, void* out, void* stream);

/*
 * MXFP4 activation quantizer (the step before W4A4).  x [rows, k] (BF16,
 * F16 or F32, row stride in elements) -> packed u8 [rows, k/2] and
 * scales u8 [rows, k/32], contiguous.  mode MXFP4_QUANT_TIES_AWAY
 * reproduces the reference test quantizer bit for bit (test:28-60);
 * MXFP4_QUANT_RNE is the OCP MX rule.  k % 32 == 0.
 */
int mxfp4_quant(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t x_row_stride,
                int mode, uint8_t* packed, uint8_t* scales, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFP4_GFX950_H_ */
