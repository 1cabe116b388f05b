// Host conversion of GGUF block storage into the tiled device layout
// described in formats.h. A pure byte permutation: the device matrix has
// exactly the GGUF byte count and every quant, scale and minimum is kept bit
// for bit.
#include "formats.h"
#include <string.h>

namespace fy {
namespace {

// Q4_K sub-block scales and minimums as backend/core/llm_quant.c:249-250
// unpacks them from scales[12].
void q4k_scales(const uint8_t *sc, unsigned (&scale)[8], unsigned (&minimum)[8])
{
    for (unsigned g = 0; g < 8; ++g) {
        if (g < 4) {
            scale[g] = sc[g] & 63u;
            minimum[g] = sc[g + 4] & 63u;
        } else {
            scale[g] = (sc[g + 4] & 15u) | ((unsigned)(sc[g - 4] >> 6) << 4);
            minimum[g] = (sc[g + 4] >> 4) | ((unsigned)(sc[g] >> 6) << 4);
        }
    }
}

// One row's group (GGUF bytes `b`) into a group of R rows at `g`, row r.
void pack_q4k(uint8_t *g, const uint8_t *b, size_t R, size_t r)
{
    unsigned scale[8], minimum[8];
    q4k_scales(b + 4, scale, minimum);
    for (unsigned p = 0; p < 4; ++p) {
        memcpy(g + 32 * R * p + 16 * r, b + 16 + 32 * p, 16);
        memcpy(g + 32 * R * p + 16 * R + 16 * r, b + 32 + 32 * p, 16);
        const uint32_t slice = scale[2 * p] | minimum[2 * p] << 6 | scale[2 * p + 1] << 12 |
            minimum[2 * p + 1] << 18 | (uint32_t)b[p] << 24;
        memcpy(g + 128 * R + 16 * r + 4 * p, &slice, 4);
    }
}

// `dd` is where this group's d values start (after every group's fields).
void pack_q6k(uint8_t *g, uint8_t *dd, const uint8_t *b, size_t R, size_t r)
{
    for (unsigned h = 0; h < 2; ++h)
        for (unsigned l16 = 0; l16 < 2; ++l16) {
            const unsigned p = 2 * h + l16;
            memcpy(g + 48 * R * p + 16 * r, b + 64 * h + 16 * l16, 16);
            memcpy(g + 48 * R * p + 16 * R + 16 * r, b + 64 * h + 32 + 16 * l16, 16);
            memcpy(g + 48 * R * p + 32 * R + 16 * r, b + 128 + 32 * h + 16 * l16, 16);
            for (unsigned q = 0; q < 4; ++q) g[192 * R + 16 * r + 4 * p + q] = b[192 + 8 * h + 2 * q + l16];
        }
    memcpy(dd + 2 * r, b + 208, 2);
}

// Q8_0 / Q4_0: `b` holds nb consecutive GGUF blocks of the row. A full group
// (nb = 8) stores Q8_0 quants block by block in two halves of 16 columns,
// Q4_0 quants in units of two blocks (byte n of half h of unit p: element
// 16h + n of block 2p in the low nibble, of block 2p + 1 in the high one),
// and the row's eight scales together; a short group keeps each block's
// bytes (Q8_0 again in halves) and the scales block by block.
void pack_q8q4(uint8_t *g, const uint8_t *b, size_t R, size_t r, size_t nb, size_t quant)
{
    if (nb == 8) {
        for (size_t j = 0; j < 8; ++j) {
            const uint8_t *blk = b + j * (quant + 2);
            memcpy(g + 8 * quant * R + 16 * r + 2 * j, blk, 2);
            if (quant == 32)
                for (size_t h = 0; h < 2; ++h) memcpy(g + 32 * R * j + 16 * R * h + 16 * r, blk + 2 + 16 * h, 16);
        }
        if (quant == 16) {
            // Element e of a Q4_0 block: low nibble of qs[e] (e < 16), else the
            // high nibble of qs[e - 16].
            auto nib = [&](size_t j, size_t e) -> uint8_t {
                const uint8_t *qs = b + j * 18 + 2;
                return e < 16 ? (qs[e] & 15) : (qs[e - 16] >> 4);
            };
            for (size_t p = 0; p < 4; ++p)
                for (size_t h = 0; h < 2; ++h)
                    for (size_t n = 0; n < 16; ++n)
                        g[32 * R * p + 16 * R * h + 16 * r + n] =
                            (uint8_t)(nib(2 * p, 16 * h + n) | nib(2 * p + 1, 16 * h + n) << 4);
        }
        return;
    }
    for (size_t j = 0; j < nb; ++j) {
        const uint8_t *blk = b + j * (quant + 2);
        if (quant == 32)
            for (size_t h = 0; h < 2; ++h) memcpy(g + 32 * R * j + 16 * R * h + 16 * r, blk + 2 + 16 * h, 16);
        else
            memcpy(g + 16 * R * j + 16 * r, blk + 2, 16);
        memcpy(g + quant * R * nb + 2 * R * j + 2 * r, blk, 2);
    }
}

}  // namespace

void pack_tiles(uint8_t *dst, const uint8_t *src, unsigned type, size_t rows, size_t cols)
{
    format_info f;
    if (!format_of(type, &f)) return;
    const size_t row_bytes = cols / f.block * f.bytes;
    const unsigned gb = group_row_bytes(type);
    if (!gb) {
        memcpy(dst, src, rows * row_bytes);
        return;
    }
    const size_t groups = (cols + kGroupCols - 1) / kGroupCols;
    for (size_t t = 0; t * kTileRows < rows; ++t) {
        const size_t R = rows - t * kTileRows < (size_t)kTileRows ? rows - t * kTileRows : kTileRows;
        uint8_t *tile = dst + t * kTileRows * row_bytes;
        for (size_t r = 0; r < R; ++r) {
            const uint8_t *row = src + (t * kTileRows + r) * row_bytes;
            for (size_t g = 0; g < groups; ++g) {
                const uint8_t *b = row + g * gb;
                switch (type) {
                case Q4_K: pack_q4k(tile + g * gb * R, b, R, r); break;
                case Q6_K: pack_q6k(tile + g * 208 * R, tile + 208 * R * groups + 2 * R * g, b, R, r); break;
                default: {
                    const size_t blocks = cols / 32, nb = blocks - 8 * g < 8 ? blocks - 8 * g : 8;
                    pack_q8q4(tile + g * gb * R, b, R, r, nb, type == Q8_0 ? 32 : 16);
                }
                }
            }
        }
    }
}

}  // namespace fy
