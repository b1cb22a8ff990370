/*
 * CPU oracle, C part: an independent integer restatement of the byte-level
 * MXFP4 functions.  TEST INFRASTRUCTURE ONLY -- built by oracle/build.py into
 * oracle/_build/libmxfp4_oracle.so and loaded by tests/, smoke() and the
 * cpu_baseline leg of bench.py as a checker.  Nothing in the product links it.
 *
 * Reference lines restated (paths in lutianshu824/mxfp4-gfx936):
 *   soft = src/aiter/ops/triton/moe_op_mxfp4_soft.py
 *   vllm = integration/vllm/vllm_mxfp4_gfx936.py
 *   test = tests/test_moe_mxfp4_soft.py
 *
 * The numpy oracle computes dequant as LUT * ldexp(1, s - 127) in FP32 and
 * lets the FPU round; this file instead builds every output bit pattern from
 * the E2M1 fields and the E8M0 exponent with integer arithmetic, so the two
 * derivations check each other over all 16 x 256 (code, scale) pairs.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

enum { ORACLE_F32 = 0, ORACLE_BF16 = 1, ORACLE_F16 = 2 };

/* E2M1 magnitude code m (1..7) = mant * 2^exp2 with mant in {1, 1.5}:
 * 0.5=1*2^-1, 1=1*2^0, 1.5=1.5*2^0, 2=1*2^1, 3=1.5*2^1, 4=1*2^2, 6=1.5*2^2
 * (soft:12-29). */
static const int kE2M1Exp[8] = {0, -1, 0, 0, 1, 1, 2, 2};
static const int kE2M1Half[8] = {0, 0, 0, 1, 0, 1, 0, 1}; /* mant == 1.5 */

/* soft:295-307 for one element: value = E2M1[code] * 2^(s-127) in FP32,
 * NaN (0x7FC00000) when s == 255; exact except overflow to +-inf. */
uint32_t oracle_dequant_elem_f32(unsigned code, unsigned s) {
  if (s == 255) return 0x7FC00000u;
  uint32_t sign = (uint32_t)(code >> 3) << 31;
  unsigned m = code & 7;
  if (m == 0) return sign;
  int be = (int)s + kE2M1Exp[m]; /* biased FP32 exponent of the product */
  if (be >= 255) return sign | 0x7F800000u;
  if (be >= 1) return sign | ((uint32_t)be << 23) | ((uint32_t)kE2M1Half[m] << 22);
  /* be in {0, -1}: subnormal, value = mant * 2^(be-127) = (2*mant) * 2^(be+21) ulps */
  uint32_t twice_mant = kE2M1Half[m] ? 3u : 2u;
  return sign | (twice_mant << (be + 21));
}

uint16_t oracle_dequant_elem_bf16(unsigned code, unsigned s) {
  /* every FP32 product above has at most two significant bits, so its low
   * half is zero and the bf16 conversion is a plain truncation (NaN stays
   * the canonical 0x7FC0). */
  return (uint16_t)(oracle_dequant_elem_f32(code, s) >> 16);
}

/* float16 RNE of mant * 2^x, mant in {1, 1.5}, built from integers. */
uint16_t oracle_dequant_elem_f16(unsigned code, unsigned s) {
  if (s == 255) return 0x7E00;
  uint16_t sign = (uint16_t)((code >> 3) << 15);
  unsigned m = code & 7;
  if (m == 0) return sign;
  int x = (int)s - 127 + kE2M1Exp[m];
  if (x >= 16) return sign | 0x7C00; /* >= 65536 rounds to inf */
  if (x >= -14) return sign | (uint16_t)((x + 15) << 10) | (uint16_t)(kE2M1Half[m] << 9);
  /* subnormal: value / 2^-24 = (2*mant) * 2^(x+23), rounded half to even */
  uint32_t num = kE2M1Half[m] ? 3u : 2u;
  int sh = x + 23;
  uint32_t q;
  if (sh >= 0) {
    q = num << sh;
  } else {
    int r = -sh;
    if (r > 8) {
      q = 0;
    } else {
      uint32_t rem = num & ((1u << r) - 1u), half = 1u << (r - 1);
      q = num >> r;
      if (rem > half || (rem == half && (q & 1u))) q++;
    }
  }
  return sign | (uint16_t)q;
}

/* dequant_mxfp4(packed[rows, k/2], scales[rows, k/32], dtype) (soft:277-307),
 * rows contiguous.  out holds uint32 (f32) or uint16 (bf16/f16) patterns. */
int oracle_dequant(const uint8_t* packed, const uint8_t* scales, int64_t rows, int64_t k,
                   int dtype, void* out) {
  if (k % 32) return 1;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < k; ++i) {
      uint8_t byte = packed[r * (k / 2) + i / 2];
      unsigned code = (i & 1) ? (byte >> 4) : (byte & 15); /* low nibble = even k */
      unsigned s = scales[r * (k / 32) + i / 32];
      int64_t o = r * k + i;
      if (dtype == ORACLE_F32) ((uint32_t*)out)[o] = oracle_dequant_elem_f32(code, s);
      else if (dtype == ORACLE_BF16) ((uint16_t*)out)[o] = oracle_dequant_elem_bf16(code, s);
      else if (dtype == ORACLE_F16) ((uint16_t*)out)[o] = oracle_dequant_elem_f16(code, s);
      else return 2;
    }
  }
  return 0;
}

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* The reference test quantizer (test:28-60), one row of k floats. */
static void quant_row_ties_away(const float* x, int64_t k, uint8_t* packed, uint8_t* scales) {
  for (int64_t b = 0; b < k / 32; ++b) {
    const float* blk = x + b * 32;
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) { float a = fabsf(blk[j]); if (a > amax) amax = a; }
    uint32_t ab = (f32_bits(amax) + 0x200000u) & 0xFF800000u; /* test:37 */
    float amax_r = bits_f32(ab);
    float e = (amax_r == 0.f) ? -127.f : floorf(log2f(amax_r)) - 2.f; /* test:38 */
    if (e < -127.f) e = -127.f;
    if (e > 127.f) e = 127.f;
    float inv = ldexpf(1.f, -(int)e);
    uint8_t codes[32];
    for (int j = 0; j < 32; ++j) {
      uint32_t q = f32_bits(blk[j] * inv);               /* test:39-41 */
      uint32_t sign = q & 0x80000000u;
      int32_t ex = (int32_t)((q >> 23) & 0xFF);
      int32_t mant = (int32_t)(q & 0x7FFFFF);
      if (ex < 127) {                                      /* test:45-50 */
        int sh = 127 - ex - 1;
        mant = sh < 32 ? ((0x400000 | (mant >> 1)) >> sh) : 0;
      }
      ex = (ex > 126 ? ex : 126) - 126;                    /* test:51 */
      int32_t comb = (((ex << 2) | (mant >> 21)) + 1) >> 1; /* test:52 */
      int32_t mag = comb < 7 ? comb : 7;                   /* test:53 */
      codes[j] = (uint8_t)(((sign >> 28) & 0xF) | (uint32_t)mag);
    }
    for (int j = 0; j < 32; j += 2) packed[b * 16 + j / 2] = (uint8_t)(codes[j] | (codes[j + 1] << 4));
    scales[b] = (uint8_t)(((int)e + 127) & 0xFF);          /* test:57 */
  }
}

/* OCP MX quantizer: E = floor(log2 amax) - 2, E2M1 round-half-even, +-6 saturation. */
static void quant_row_rne(const float* x, int64_t k, uint8_t* packed, uint8_t* scales) {
  static const double grid[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
  for (int64_t b = 0; b < k / 32; ++b) {
    const float* blk = x + b * 32;
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) { float a = fabsf(blk[j]); if (a > amax) amax = a; }
    int e;
    if (amax == 0.f) {
      e = -127;
    } else if (isinf(amax)) {
      e = 127; /* floor(log2(inf)) - 2 saturates, as in numpy and test:38 */
    } else {
      uint32_t ab = f32_bits(amax);
      int ex = (int)((ab >> 23) & 0xFF);
      int fl;
      if (ex) {
        fl = ex - 127;
      } else { /* subnormal: floor(log2) from the top set bit */
        uint32_t mm = ab & 0x7FFFFF; int top = 31 - __builtin_clz(mm);
        fl = top - 149;
      }
      e = fl - 2;
      if (e < -127) e = -127;
      if (e > 127) e = 127;
    }
    uint8_t codes[32];
    for (int j = 0; j < 32; ++j) {
      double q = ldexp((double)blk[j], -e);
      double mag = fabs(q);
      int c;
      if (mag >= 6.0) {
        c = 7;
      } else {
        c = 0;
        for (int i = 1; i < 8; ++i) {
          if (mag >= grid[i]) { c = i; continue; }
          double dlo = mag - grid[i - 1], dhi = grid[i] - mag;
          c = (dhi < dlo || (dhi == dlo && (i % 2 == 0))) ? i : i - 1;
          break;
        }
      }
      codes[j] = (uint8_t)(c | (signbit(blk[j]) ? 8 : 0));
    }
    for (int j = 0; j < 32; j += 2) packed[b * 16 + j / 2] = (uint8_t)(codes[j] | (codes[j + 1] << 4));
    scales[b] = (uint8_t)(e + 127);
  }
}

/* mode 0: reference test quantizer (ties away); mode 1: OCP RNE. */
int oracle_quant(const float* x, int64_t rows, int64_t k, int mode, uint8_t* packed,
                 uint8_t* scales) {
  if (k % 32) return 1;
  for (int64_t r = 0; r < rows; ++r) {
    if (mode == 0) quant_row_ties_away(x + r * k, k, packed + r * (k / 2), scales + r * (k / 32));
    else quant_row_rne(x + r * k, k, packed + r * (k / 2), scales + r * (k / 32));
  }
  return 0;
}

/* vllm:119-146 with ids outside [0, num_experts) dropped: experts ascending,
 * route ids ascending inside an expert, chunks of block_m padded with the
 * sentinel n.  Returns the number of blocks; sorted_ids must hold
 * n + num_experts * block_m entries, expert_ids n + num_experts. */
int64_t oracle_make_routing(const int64_t* ids, int64_t n, int num_experts, int block_m,
                            int32_t* sorted_ids, int32_t* expert_ids) {
  int64_t pos = 0, blocks = 0;
  for (int e = 0; e < num_experts; ++e) {
    int64_t in_block = 0;
    for (int64_t r = 0; r < n; ++r) {
      if (ids[r] != e) continue;
      if (in_block == 0) expert_ids[blocks++] = e;
      sorted_ids[pos++] = (int32_t)r;
      if (++in_block == block_m) in_block = 0;
    }
    if (in_block) while (in_block++ < block_m) sorted_ids[pos++] = (int32_t)n;
  }
  return blocks;
}
