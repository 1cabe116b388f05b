// GGUF block formats and their device layouts.
//
// GGUF storage (decoded by backend/core/llm_quant.c:70-142):
//   Q4_0 18 B / 32: d f16 @0, qs[16] @2; element j<16 low nibble of qs[j],
//        j>=16 high nibble of qs[j-16]; w = d*(q-8).
//   Q8_0 34 B / 32: d f16 @0, qs int8[32] @2; w = d*q.
//   Q4_K 144 B / 256: d @0, dmin @2, scales[12] @4, qs[128] @16; sub-block g
//        (32 elements) uses the low (g even) or high (g odd) nibble of
//        qs[(g/2)*32 + l]; w = d*sc[g]*q - dmin*m[g] with 6-bit sc/m packed
//        in scales[12].
//   Q6_K 210 B / 256: ql[128] @0, qh[64] @128, sc int8[16] @192, d @208;
//        element n = 128h + 32q + l has
//        q6 = ((ql[64h + 32(q&1) + l] >> 4(q>>1)) & 15)
//             | (((qh[32h + l] >> 2q) & 3) << 4),
//        w = d * sc[n/16] * (q6 - 32).
//
// Device layouts keep exactly the GGUF byte count. F32/F16/BF16 are uploaded
// unchanged. For the block formats the kernels give each lane one "unit" of
// a row (64 elements of a K-quant superblock, or one 32-element Q8_0/Q4_0
// block), so the matrix is stored as field planes indexed by (row, unit):
// lane u's slice of a field sits at (row * U + u) * size, and the 64 lanes of
// a wavefront read one contiguous span per load instruction. U = units per
// row. Planes, each over all rows:
//   Q4_K (U = cols/64, unit 4s+p): qa 16 B = qs[32p..+16), qb 16 B =
//        qs[32p+16..+16), slice 4 B = sc(2p) | m(2p)<<6 | sc(2p+1)<<12 |
//        m(2p+1)<<18 | byte p of (d, dmin) << 24
//   Q6_K (U = cols/64, unit 4s+2h+l16): a = ql[64h+16*l16..+16),
//        b = ql[64h+32+16*l16..+16), c = qh[32h+16*l16..+16) (16 B each),
//        sc 4 B (byte q = sc[8h+2q+l16]), then d 2 B per superblock
//   Q8_0 (U = cols/32): qa = qs[0..16), qb = qs[16..32), d 2 B
//   Q4_0 (U = cols/32): q = qs[0..16), d 2 B
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace fy {

enum : unsigned { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q6_K = 14, BF16 = 30 };

struct format_info {
    unsigned block;    // elements per block
    unsigned bytes;    // GGUF bytes per block
};

inline bool format_of(unsigned type, format_info *f)
{
    switch (type) {
    case F32: *f = {1, 4}; return true;
    case F16: case BF16: *f = {1, 2}; return true;
    case Q4_0: *f = {32, 18}; return true;
    case Q8_0: *f = {32, 34}; return true;
    case Q4_K: *f = {256, 144}; return true;
    case Q6_K: *f = {256, 210}; return true;
    default: return false;
    }
}

// Host-side byte permutation GGUF -> device layout (see the header comment); pack.cpp.
void pack_planes(uint8_t *dst, const uint8_t *src, unsigned type, size_t rows, size_t cols);

}  // namespace fy
