/* TEST INFRASTRUCTURE ONLY: the parity oracle of the quantized matrix path.
 *
 * A plain-C restatement of the reference CPU path, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's CPU-baseline leg as the oracle.
 * Nothing in the product (fyodor_amd/) links, loads or calls it.
 *
 * Each function follows the reference file:line it names, including the
 * order and rounding of every floating-point operation, so its outputs are
 * bit-identical to the reference scalar kernel when built like it
 * (C17, no FMA contraction, SSE2 scalar float).
 *
 * Pinning (see tests/test_oracle.py):
 *  - orc_half / orc_round_f16: all 65,536 encodings against an independent
 *    ldexp closed form and every round-to-nearest-even tie
 *    (backend/tests/test_kv_precision.c:10-46);
 *  - orc_value: Q4_K/Q6_K blocks built from logical scales by an encoder
 *    independent of the decoder (backend/tests/test_architectures.c:229-300),
 *    exact constant-row fixtures for Q4_0/Q8_0
 *    (backend/tests/test_generation.c:79-103);
 *  - orc_matvec: bit-exact against golden vectors written by the reference's
 *    own nya_llm_matvec compiled from its sources (tests/golden/), and
 *    against exact power-of-two dot products;
 *  - orc_matvec_double: brute-force double sums on tiny inputs;
 *  - orc_dequant: element for element equal to orc_value. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_BF16 = 30 };

/* backend/core/llm_quant.c:5-39: exact binary16 -> binary32. */
float orc_half(const unsigned char *p)
{
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    const uint32_t sign = (h & 0x8000u) << 16;
    int exponent = (int)((h >> 10) & 31u);
    uint32_t fraction = h & 1023u, bits;
    if (exponent == 0 && fraction == 0) {
        bits = sign;
    } else if (exponent == 0) {
        /* Subnormal: normalise the fraction. */
        exponent = 1;
        while (!(fraction & 1024u)) { fraction <<= 1; --exponent; }
        bits = sign | ((uint32_t)(exponent + 112) << 23) | ((fraction & 1023u) << 13);
    } else if (exponent == 31) {
        bits = sign | 0x7F800000u | (fraction << 13);
    } else {
        bits = sign | ((uint32_t)(exponent + 112) << 23) | (fraction << 13);
    }
    float value;
    memcpy(&value, &bits, sizeof(value));
    return value;
}

/* backend/core/llm_quant.c:46-67: round to binary16 (ties to even), expand. */
float orc_round_f16(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    const uint32_t sign = (bits >> 16) & 0x8000u, magnitude = bits & 0x7FFFFFFFu;
    uint32_t half;
    if (magnitude >= 0x7F800000u) {
        half = magnitude == 0x7F800000u ? 0x7C00u : 0x7E00u;
    } else if (magnitude >= 0x477FF000u) {
        half = 0x7C00u;
    } else if (magnitude < 0x33000000u) {
        half = 0;
    } else {
        const uint32_t exponent = magnitude >> 23;
        const uint32_t shift = exponent < 113u ? 126u - exponent : 13u;
        const uint32_t mantissa = (magnitude & 0x7FFFFFu) | (exponent < 113u ? 0x800000u : 0u);
        uint32_t rounded = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1u), mid = 1u << (shift - 1u);
        if (rest > mid || (rest == mid && (rounded & 1u))) ++rounded;
        half = exponent < 113u ? rounded : ((exponent - 112u) << 10) + rounded;
    }
    const uint16_t h = (uint16_t)(sign | half);
    const unsigned char b[2] = {(unsigned char)h, (unsigned char)(h >> 8)};
    return orc_half(b);
}

/* 6-bit scale and minimum of Q4_K sub-block g (backend/core/llm_quant.c:75-76). */
static void q4k_scale(const unsigned char *s, size_t g, unsigned *sc, unsigned *mn)
{
    if (g < 4) {
        *sc = s[g] & 63u;
        *mn = s[g + 4] & 63u;
    } else {
        *sc = (s[g + 4] & 15u) | ((unsigned)(s[g - 4] >> 6) << 4);
        *mn = (s[g + 4] >> 4) | ((unsigned)(s[g] >> 6) << 4);
    }
}

/* 6-bit Q6_K quant of element n, minus 32 (backend/core/llm_quant.c:81-84). */
static int q6k_quant(const unsigned char *b, size_t n)
{
    const size_t h = n / 128, q = n % 128 / 32, l = n % 32;
    const unsigned lo = b[h * 64 + q % 2 * 32 + l], hi = b[128 + h * 32 + l];
    return (int)(((lo >> (q / 2 * 4)) & 15u) | (((hi >> (q * 2)) & 3u) << 4)) - 32;
}

/* backend/core/llm_quant.c:70-142: one element of a row-major GGUF tensor. */
float orc_value(const unsigned char *data, unsigned type, size_t index)
{
    switch (type) {
    case T_F32: {
        float v;
        memcpy(&v, data + index * 4, 4);
        return v;
    }
    case T_F16:
        return orc_half(data + index * 2);
    case T_BF16: {
        const unsigned char *p = data + index * 2;
        const uint32_t bits = ((uint32_t)p[0] | ((uint32_t)p[1] << 8)) << 16;
        float v;
        memcpy(&v, &bits, 4);
        return v;
    }
    case T_Q8_0: {
        const unsigned char *b = data + index / 32 * 34;
        int8_t q;
        memcpy(&q, b + 2 + index % 32, 1);
        return orc_half(b) * q;
    }
    case T_Q4_0: {
        const unsigned char *b = data + index / 32 * 18;
        const size_t at = index % 32;
        const unsigned packed = b[2 + at % 16];
        const int q = at < 16 ? (int)(packed & 15u) : (int)(packed >> 4);
        return orc_half(b) * (float)(q - 8);
    }
    case T_Q4_K: {
        const unsigned char *b = data + index / 256 * 144;
        const size_t at = index % 256, g = at / 32;
        unsigned sc, mn;
        q4k_scale(b + 4, g, &sc, &mn);
        const unsigned q = (b[16 + g / 2 * 32 + at % 32] >> (g % 2 * 4)) & 15u;
        return orc_half(b) * (float)sc * (float)q - orc_half(b + 2) * (float)mn;
    }
    case T_Q6_K: {
        const unsigned char *b = data + index / 256 * 210;
        const size_t at = index % 256;
        int8_t sc;
        memcpy(&sc, b + 192 + at / 16, 1);
        return orc_half(b + 208) * (float)sc * (float)q6k_quant(b, at);
    }
    default:
        return 0.0f;
    }
}

/* Bytes of one stored row. */
static size_t row_bytes(unsigned type, size_t cols)
{
    switch (type) {
    case T_F32: return cols * 4;
    case T_F16: case T_BF16: return cols * 2;
    case T_Q4_0: return cols / 32 * 18;
    case T_Q8_0: return cols / 32 * 34;
    case T_Q4_K: return cols / 256 * 144;
    case T_Q6_K: return cols / 256 * 210;
    default: return 0;
    }
}

/* One output of the scalar reference, backend/core/llm_quant.c:161-311. */
static float scalar_row(const unsigned char *r, unsigned type, const float *x, size_t cols)
{
    if (type == T_F32) {
        /* :161-182 accumulates F32 rows in double. */
        double sum = 0.0;
        for (size_t k = 0; k < cols; ++k) {
            float w;
            memcpy(&w, r + 4 * k, 4);
            sum += (double)w * x[k];
        }
        return (float)sum;
    }
    float sum = 0.0f;
    if (type == T_F16 || type == T_BF16) {
        for (size_t k = 0; k < cols; ++k) sum += orc_value(r, type, k) * x[k];
    } else if (type == T_Q8_0) {
        /* :206-234: (scale * q) * x, one block after another. */
        for (size_t b = 0; b < cols / 32; ++b) {
            const unsigned char *blk = r + 34 * b;
            const float scale = orc_half(blk);
            for (size_t i = 0; i < 32; ++i) {
                int8_t q;
                memcpy(&q, blk + 2 + i, 1);
                sum += scale * (float)q * x[32 * b + i];
            }
        }
    } else if (type == T_Q4_K) {
        /* :245-255: (factor * q - bias) * x per element. */
        for (size_t b = 0; b < cols / 256; ++b) {
            const unsigned char *blk = r + 144 * b;
            const float d = orc_half(blk), dmin = orc_half(blk + 2);
            for (size_t g = 0; g < 8; ++g) {
                unsigned sc, mn;
                q4k_scale(blk + 4, g, &sc, &mn);
                const float factor = d * (float)sc, bias = dmin * (float)mn;
                const unsigned char *qs = blk + 16 + g / 2 * 32;
                const unsigned shift = (unsigned)(g % 2 * 4);
                for (size_t l = 0; l < 32; ++l)
                    sum += (factor * (float)((qs[l] >> shift) & 15u) - bias) * x[256 * b + 32 * g + l];
            }
        }
    } else if (type == T_Q6_K) {
        /* :256-270: sixteen groups of sixteen, factor * q * x. */
        for (size_t b = 0; b < cols / 256; ++b) {
            const unsigned char *blk = r + 210 * b;
            const float d = orc_half(blk + 208);
            for (size_t g = 0; g < 16; ++g) {
                int8_t sc;
                memcpy(&sc, blk + 192 + g, 1);
                const float factor = d * (float)sc;
                for (size_t j = 0; j < 16; ++j)
                    sum += factor * (float)q6k_quant(blk, 16 * g + j) * x[256 * b + 16 * g + j];
            }
        }
    } else if (type == T_Q4_0) {
        /* :278-311: low and high nibble of each byte, interleaved. */
        for (size_t b = 0; b < cols / 32; ++b) {
            const unsigned char *blk = r + 18 * b;
            const float scale = orc_half(blk);
            for (size_t i = 0; i < 16; ++i) {
                const unsigned packed = blk[2 + i];
                const float low = (float)((int)(packed & 15u) - 8), high = (float)((int)(packed >> 4) - 8);
                sum += scale * low * x[32 * b + i];
                sum += scale * high * x[32 * b + i + 16];
            }
        }
    }
    return sum;
}

/* backend/core/llm_quant.c:145-312 with no compute context: y = W x. */
void orc_matvec(float *y, const unsigned char *w, unsigned type, const float *x, size_t cols, size_t rows)
{
    const size_t stride = row_bytes(type, cols);
    for (size_t r = 0; r < rows; ++r) y[r] = scalar_row(w + r * stride, type, x, cols);
}

/* backend/tests/test_quant_kernels.c:13-25: double sum of decoded products
 * and the sum of their magnitudes, per row. */
void orc_matvec_double(double *sum, double *magnitude, const unsigned char *w, unsigned type,
    const float *x, size_t cols, size_t rows)
{
    const size_t stride = row_bytes(type, cols);
    for (size_t r = 0; r < rows; ++r) {
        double s = 0.0, m = 0.0;
        for (size_t k = 0; k < cols; ++k) {
            const double p = (double)orc_value(w + r * stride, type, k) * x[k];
            s += p;
            m += fabs(p);
        }
        sum[r] = s;
        magnitude[r] = m;
    }
}

/* Batch-major matmul through the scalar rows: Y[b][r] (what the reference
 * runs per token when a provider declines, backend/core/llm_cpu_prefill.inc:8). */
typedef struct job {
    float *y;
    const unsigned char *w;
    const float *x;
    unsigned type;
    size_t cols, rows, batch, begin, end;
} job;

static void *run_job(void *opaque)
{
    const job *j = opaque;
    const size_t stride = row_bytes(j->type, j->cols);
    for (size_t r = j->begin; r < j->end; ++r)
        for (size_t b = 0; b < j->batch; ++b)
            j->y[b * j->rows + r] = scalar_row(j->w + r * stride, j->type, j->x + b * j->cols, j->cols);
    return NULL;
}

/* The same, with rows split over `threads` POSIX threads (the CPU baseline
 * "port"); results do not depend on the thread count. Returns 0 on success. */
int orc_matmul(float *y, const unsigned char *w, unsigned type, const float *x, size_t cols, size_t rows,
    size_t batch, int threads)
{
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = (int)rows;
    job jobs[256];
    pthread_t ids[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; ++t) {
        jobs[t] = (job){y, w, x, type, cols, rows, batch, rows * (size_t)t / (size_t)threads,
            rows * (size_t)(t + 1) / (size_t)threads};
    }
    int started = 0;
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&ids[t], NULL, run_job, &jobs[t])) break;
        started = t;
    }
    run_job(&jobs[0]);
    for (int t = started + 1; t < threads; ++t) run_job(&jobs[t]);
    for (int t = 1; t <= started; ++t) pthread_join(ids[t], NULL);
    return 0;
}

/* The decoded weights of a whole matrix, out[r * cols + k] = orc_value of
 * element k of row r (backend/core/llm_quant.c:70-142), rows split over
 * `threads` POSIX threads. The tests form the double-precision sums of the
 * reference kernel contract (backend/tests/test_quant_kernels.c:13-25) for
 * large batches from these values with a BLAS product. Returns 0. */
typedef struct dequant_job {
    float *out;
    const unsigned char *w;
    unsigned type;
    size_t cols, begin, end;
} dequant_job;

static void *run_dequant(void *opaque)
{
    const dequant_job *j = opaque;
    const size_t stride = row_bytes(j->type, j->cols);
    for (size_t r = j->begin; r < j->end; ++r)
        for (size_t k = 0; k < j->cols; ++k) j->out[r * j->cols + k] = orc_value(j->w + r * stride, j->type, k);
    return NULL;
}

int orc_dequant(float *out, const unsigned char *w, unsigned type, size_t rows, size_t cols, int threads)
{
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = (int)rows;
    if (threads > 256) threads = 256;
    dequant_job jobs[256];
    pthread_t ids[256];
    for (int t = 0; t < threads; ++t)
        jobs[t] = (dequant_job){out, w, type, cols, rows * (size_t)t / (size_t)threads,
            rows * (size_t)(t + 1) / (size_t)threads};
    int started = 0;
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&ids[t], NULL, run_dequant, &jobs[t])) break;
        started = t;
    }
    run_dequant(&jobs[0]);
    for (int t = started + 1; t < threads; ++t) run_dequant(&jobs[t]);
    for (int t = 1; t <= started; ++t) pthread_join(ids[t], NULL);
    return 0;
}
