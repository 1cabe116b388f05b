// Host conversion of GGUF block storage into the 16-byte aligned plane layout
// described in formats.h. A pure byte permutation: no value changes.
#include "formats.h"
#include <string.h>

namespace fy {

void pack_planes(uint8_t *dst, const uint8_t *src, unsigned type, size_t rows, size_t cols)
{
    if (type == Q8_0 || type == Q4_0) {
        const size_t blocks = rows * (cols / 32);
        const size_t quant = type == Q8_0 ? 32 : 16, stride = quant + 2;
        uint8_t *qs = dst, *ds = dst + blocks * quant;
        for (size_t b = 0; b < blocks; ++b) {
            const uint8_t *block = src + b * stride;
            memcpy(ds + 2 * b, block, 2);
            memcpy(qs + quant * b, block + 2, quant);
        }
    } else if (type == Q6_K) {
        const size_t blocks = rows * (cols / 256);
        uint8_t *q = dst, *sc = dst + blocks * 192, *d = dst + blocks * 208;
        for (size_t b = 0; b < blocks; ++b) {
            const uint8_t *block = src + b * 210;
            memcpy(q + 192 * b, block, 192);
            memcpy(sc + 16 * b, block + 192, 16);
            memcpy(d + 2 * b, block + 208, 2);
        }
    } else {
        format_info f;
        if (format_of(type, &f)) memcpy(dst, src, rows * (cols / f.block) * f.bytes);
    }
}

}  // namespace fy
