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
// unchanged. The block formats are stored in tiles of 32 rows, the M (or N)
// extent of one gfx950 MFMA: tile t holds rows 32t.. (R rows, R = 32 except
// possibly in the last tile) at byte 32 * t * row_bytes. A tile is a sequence
// of column groups of 256 (a K-quant superblock, or eight Q8_0/Q4_0 blocks;
// the last Q8_0/Q4_0 group may hold nb < 8 blocks), group g at
// g * group_bytes * R. Inside a group every field is stored row-minor
// ([field][row]), so the 64 lanes of a wavefront that own 32 rows x 2
// halves read one contiguous 1 KiB span per 16-byte load. Row r of the tile:
//   Q4_K (144 R): for units p < 4 (sub-blocks 2p, 2p+1): qa at 32R p + 16r
//        = qs[32p..+16), qb at 32R p + 16R + 16r = qs[32p+16..+16); slices at
//        128R + 16r, four words, word p = sc(2p) | m(2p)<<6 | sc(2p+1)<<12 |
//        m(2p+1)<<18 | byte p of (d, dmin) << 24.
//   Q6_K (210 R; the 16-byte fields of group g at 208R g, the d values of
//        all groups after them): for units p = 2h + l16 < 4 (elements
//        128h + 32q + 16 l16 + i, q < 4, i < 16): la at 48R p + 16r =
//        ql[64h+16 l16..+16), lb at 48R p + 16R + 16r = ql[64h+32+16 l16..+16),
//        qh at 48R p + 32R + 16r = qh[32h+16 l16..+16); sc at 192R + 16r, word
//        p byte q = sc[8h + 2q + l16]; d of group g at 208R G + 2R g + 2r
//        (G groups per row).
//   Q8_0 (34 R nb): qs[16h..16h+16) of block j at 32R j + 16R h + 16r; then
//        a full group (nb = 8) stores row r's eight d at 256R + 16r, a short
//        one d of block j at 32R nb + 2R j + 2r.
//   Q4_0 (18 R nb): a full group stores units p < 4 (blocks 2p, 2p+1) like
//        Q4_K: half h at 32R p + 16R h + 16r, byte n = element 16h + n of
//        block 2p (low nibble) | of block 2p + 1 (high nibble), then row r's
//        eight d at 128R + 16r. A short group keeps qs of block j at
//        16R j + 16r and d at 16R nb + 2R j + 2r.
// Every 16-byte field starts 16-byte aligned (tile and group offsets are
// multiples of 16); 2-byte scales are read one per lane.
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

constexpr int kTileRows = 32;
constexpr int kGroupCols = 256;

// Bytes per row of one column group (a full one; a short last Q8_0/Q4_0
// group has nb * block bytes).
inline unsigned group_row_bytes(unsigned type)
{
    switch (type) {
    case Q4_K: return 144;
    case Q6_K: return 210;
    case Q8_0: return 8 * 34;
    case Q4_0: return 8 * 18;
    default: return 0;
    }
}

// GGUF bytes per row, usable in device code.
template <unsigned T>
constexpr size_t tiled_row_bytes(int cols)
{
    return T == Q4_K ? (size_t)(cols / 256) * 144 : T == Q6_K ? (size_t)(cols / 256) * 210
         : T == Q8_0 ? (size_t)(cols / 32) * 34 : (size_t)(cols / 32) * 18;
}

// Host-side byte permutation GGUF -> device layout (see the header comment); pack.cpp.
void pack_tiles(uint8_t *dst, const uint8_t *src, unsigned type, size_t rows, size_t cols);

}  // namespace fy
