// Host conversion of GGUF block storage into the device layout described in
// formats.h. A pure byte permutation: the device matrix has exactly the GGUF
// byte count and every quant, scale and minimum is kept bit for bit.
#include "formats.h"
#include <string.h>

namespace fy {
namespace {

// Q4_K: unit u = 4*s + p (superblock s, nibble pair p) of row r.
//   qa[r][u] = qs[32p .. 32p+16), qb[r][u] = qs[32p+16 .. 32p+32)
//   slice[r][u] = sc(2p) | m(2p) << 6 | sc(2p+1) << 12 | m(2p+1) << 18
//                 | byte p of (d, dmin) << 24
// with the 6-bit sc/m decoded as in backend/core/llm_quant.c:249-250.
void pack_q4k(uint8_t *dst, const uint8_t *src, size_t rows, size_t cols)
{
    const size_t U = cols / 64, n = rows * U;
    uint8_t *qa = dst, *qb = dst + 16 * n;
    uint32_t *slice = (uint32_t *)(dst + 32 * n);
    for (size_t r = 0; r < rows; ++r) {
        for (size_t s = 0; s < cols / 256; ++s) {
            const uint8_t *b = src + (r * (cols / 256) + s) * 144, *sc = b + 4;
            unsigned scale[8], minimum[8];
            for (unsigned g = 0; g < 8; ++g) {
                if (g < 4) {
                    scale[g] = sc[g] & 63u;
                    minimum[g] = sc[g + 4] & 63u;
                } else {
                    scale[g] = (sc[g + 4] & 15u) | ((unsigned)(sc[g - 4] >> 6) << 4);
                    minimum[g] = (sc[g + 4] >> 4) | ((unsigned)(sc[g] >> 6) << 4);
                }
            }
            for (unsigned p = 0; p < 4; ++p) {
                const size_t u = r * U + 4 * s + p;
                memcpy(qa + 16 * u, b + 16 + 32 * p, 16);
                memcpy(qb + 16 * u, b + 32 + 32 * p, 16);
                slice[u] = scale[2 * p] | minimum[2 * p] << 6 | scale[2 * p + 1] << 12 |
                    minimum[2 * p + 1] << 18 | (uint32_t)b[p] << 24;
            }
        }
    }
}

// Q6_K: unit u = 4*s + 2*h + l16 of row r covers elements
// 128h + 32q + 16*l16 + i (q < 4, i < 16):
//   a[r][u] = ql[64h + 16*l16 ..+16), b[r][u] = ql[64h + 32 + 16*l16 ..+16)
//   c[r][u] = qh[32h + 16*l16 ..+16)
//   sc[r][u] = byte q = sc[8h + 2q + l16]
//   d[r][s] = d
void pack_q6k(uint8_t *dst, const uint8_t *src, size_t rows, size_t cols)
{
    const size_t ns = cols / 256, U = 4 * ns, n = rows * U;
    uint8_t *a = dst, *b = dst + 16 * n, *c = dst + 32 * n, *sc = dst + 48 * n, *d = dst + 52 * n;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t s = 0; s < ns; ++s) {
            const uint8_t *blk = src + (r * ns + s) * 210;
            for (unsigned h = 0; h < 2; ++h)
                for (unsigned l16 = 0; l16 < 2; ++l16) {
                    const size_t u = r * U + 4 * s + 2 * h + l16;
                    memcpy(a + 16 * u, blk + 64 * h + 16 * l16, 16);
                    memcpy(b + 16 * u, blk + 64 * h + 32 + 16 * l16, 16);
                    memcpy(c + 16 * u, blk + 128 + 32 * h + 16 * l16, 16);
                    for (unsigned q = 0; q < 4; ++q) sc[4 * u + q] = blk[192 + 8 * h + 2 * q + l16];
                }
            memcpy(d + 2 * (r * ns + s), blk + 208, 2);
        }
    }
}

// Q8_0 / Q4_0: unit = one 32-element block of row r.
//   Q8_0: qa[r][u] = qs[0..16), qb[r][u] = qs[16..32), d[r][u]
//   Q4_0: q[r][u] = qs[0..16), d[r][u]
void pack_q8q4(uint8_t *dst, const uint8_t *src, unsigned type, size_t rows, size_t cols)
{
    const size_t n = rows * (cols / 32), quant = type == Q8_0 ? 32 : 16, stride = quant + 2;
    uint8_t *d = dst + quant * n;
    for (size_t u = 0; u < n; ++u) {
        const uint8_t *blk = src + u * stride;
        memcpy(d + 2 * u, blk, 2);
        memcpy(dst + 16 * u, blk + 2, 16);
        if (type == Q8_0) memcpy(dst + 16 * n + 16 * u, blk + 18, 16);
    }
}

}  // namespace

void pack_planes(uint8_t *dst, const uint8_t *src, unsigned type, size_t rows, size_t cols)
{
    switch (type) {
    case Q4_K: pack_q4k(dst, src, rows, cols); break;
    case Q6_K: pack_q6k(dst, src, rows, cols); break;
    case Q8_0: case Q4_0: pack_q8q4(dst, src, type, rows, cols); break;
    default: {
        format_info f;
        if (format_of(type, &f)) memcpy(dst, src, rows * (cols / f.block) * f.bytes);
    }
    }
}

}  // namespace fy
