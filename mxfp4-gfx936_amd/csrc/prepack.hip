// Prepacked ("fragment-ordered") copy of MXFP4 weights for the prefill GEMMs.
//
// The direct-to-LDS prefill kernels (gemm_w4a16_pf.hip) stage a tile's
// weights 64 K at a time.  In the checkpoint layout (row-major nibbles
// [rows, K/2], E8M0 bytes [rows, K/32]) a lane's MFMA fragment is one dword
// of a 32-byte row segment and its scale one byte, and every scale needs a
// shift/or to become the conversion's scale operand.  The prepacked copy
// stores, per expert, per 16-row group g and per 64-deep stage s:
//
//   nibbles  [E][G][K/64][64 lanes][2 dwords]   512 bytes per (g, s)
//     lane l, dword j = bytes s*32 + j*16 + (l/16)*4 .. +3 of row g*16 + l%16
//     (j = the stage's first / second 32-deep half)
//   scales   [E][G][K/64][16 rows][2] uint16     64 bytes per (g, s)
//     row r, j = the high half of the conversion's scale operand for E8M0
//     byte 2s + j of row g*16 + r: (byte << 7) | 0x40, i.e. the float
//     (byte << 23) | 0x400000 without its all-zero low half
//
// so a fragment is 8 consecutive bytes and its two scales one dword in LDS:
// one conflict-free ds_read_b64 per fragment pair, one dword read and a
// shift / mask per scale pair.  Rows past the end of the matrix (the last
// group of a row count that is not a multiple of 16) are zero nibbles.
// Same bits in, same MFMA inputs: GEMMs on the prepacked copy are bitwise
// equal to GEMMs on the checkpoint layout.
#include "gemm.h"

namespace mx {
namespace {

// One thread per 8-byte lane slot of a nibble block; threads of lanes 0-15
// also write their row's two scale operand halves.
__global__ __launch_bounds__(256) void prepack_w4a16(const uint8_t* __restrict__ packed,
                                                     const uint8_t* __restrict__ scales,
                                                     int64_t experts, int64_t rows, int64_t k,
                                                     uint2* __restrict__ pre_b,
                                                     uint32_t* __restrict__ pre_s) {
  const int64_t nk = k / 64;
  const int64_t groups = prepacked_groups(rows);
  const int64_t total = experts * groups * nk * 64;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int l = (int)(i & 63);
    const int64_t blk = i >> 6;  // (e, g, s) block index
    const int64_t s = blk % nk;
    const int64_t eg = blk / nk;
    const int64_t e = eg / groups;
    const int64_t row = (eg % groups) * 16 + (l & 15);
    uint2 v{0u, 0u};
    uint32_t sb0 = 127, sb1 = 127;
    if (row < rows) {
      const uint8_t* wr = packed + (e * rows + row) * (k / 2) + s * 32 + (l >> 4) * 4;
      // 4-byte aligned: K / 2 and s * 32 are multiples of 4
      v.x = *reinterpret_cast<const uint32_t*>(wr);
      v.y = *reinterpret_cast<const uint32_t*>(wr + 16);
      const uint8_t* sr = scales + (e * rows + row) * (k / 32) + s * 2;
      sb0 = sr[0];
      sb1 = sr[1];
    }
    pre_b[i] = v;
    // the two 16-bit halves, block 2s first (the lower address)
    if (l < 16) pre_s[blk * 16 + l] = ((sb0 << 7) | 0x40u) | (((sb1 << 7) | 0x40u) << 16);
  }
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mxfp4_prepack_w4a16_size(int64_t experts, int64_t rows, int64_t k,
                                        int64_t* nibble_bytes, int64_t* scale_bytes) {
  if (nibble_bytes == nullptr || scale_bytes == nullptr || experts < 1 || rows < 1 || k <= 0 ||
      k % 64 != 0) {
    set_error("prepack size: invalid arguments (experts %lld, rows %lld, k %lld)",
              (long long)experts, (long long)rows, (long long)k);
    return MXFP4_ERR_VALUE;
  }
  *nibble_bytes = experts * prepacked_nibble_bytes(rows, k);
  *scale_bytes = experts * prepacked_scale_bytes(rows, k);
  return MXFP4_OK;
}

extern "C" int mxfp4_prepack_w4a16(const uint8_t* packed, const uint8_t* scales, int64_t experts,
                                   int64_t rows, int64_t k, uint8_t* pre_b, uint16_t* pre_s,
                                   void* stream) {
  if (experts < 1 || rows < 1 || k <= 0 || k % 64 != 0 || k > 0x7FFFFFFF) {
    set_error("prepack: invalid sizes (experts %lld, rows %lld, k %lld; K must be a multiple "
              "of 64)",
              (long long)experts, (long long)rows, (long long)k);
    return MXFP4_ERR_VALUE;
  }
  if (packed == nullptr || scales == nullptr || pre_b == nullptr || pre_s == nullptr ||
      (reinterpret_cast<uintptr_t>(packed) & 3) || (reinterpret_cast<uintptr_t>(pre_b) & 15) ||
      (reinterpret_cast<uintptr_t>(pre_s) & 15)) {
    set_error("prepack: weights must be 4-byte and the prepacked arrays 16-byte aligned");
    return MXFP4_ERR_VALUE;
  }
  const int64_t total = experts * prepacked_groups(rows) * (k / 64) * 64;
  const int64_t blocks = (total + 255) / 256 < 16384 ? (total + 255) / 256 : 16384;
  prepack_w4a16<<<(unsigned)blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      packed, scales, experts, rows, k, reinterpret_cast<uint2*>(pre_b),
      reinterpret_cast<uint32_t*>(pre_s));
  return launch_status("prepack launch");
}
