// Host-side launchers of the gfx950 kernels (called by abi.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fy {

// Y[n][rows] = sum_k W[row][k] * X[n][k] for n < batch, W in the device
// layout.
// F32 / F16 / BF16 weights (dense.hip).
hipError_t launch_dense(unsigned type, const uint8_t *w, const float *x, float *y,
    int rows, int cols, int batch, hipStream_t stream);
// Q4_0 / Q8_0 / Q4_K / Q6_K weights in the tiled layout (smalln.hip), batch
// 1..8; x must be 16-byte aligned. Batches of 2..8 need smalln_workspace
// bytes of 16-byte-aligned device scratch (batch 1 needs none).
size_t smalln_workspace(int cols, int batch);
hipError_t launch_smalln(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, int batch,
    void *workspace, hipStream_t stream);

// Batch-1 matvec with the eight block dots of a 256-column group chained
// through one MFMA accumulator (matvec.hip); matvec_supported tells which
// requests it takes (the others run on launch_smalln). x must be 16-byte
// aligned.
bool matvec_supported(unsigned type, int rows, int cols);
const char *matvec_kernel(unsigned type, int rows, int cols);
hipError_t launch_matvec(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    hipStream_t stream);
// The same product of silu(gate) * up (elementwise, formed as each group of
// the vector is loaded): the decoder's gated SiLU folded into its down
// product. Shapes that run on the row-balanced kernel only (up to two tiles
// per CU for Q4_K); gate and up 16-byte aligned.
bool matvec_gated_supported(unsigned type, int rows, int cols);
// One token's product of the decoder's normalized residual: h = x + r (r
// may be null), xn = RMS-normalized h times g (the norm step's arithmetic and
// order), y = W xn, and h written to hout by one workgroup. Up to 32 rows per
// CU, cols up to 4096.
bool matvec_normed_supported(unsigned type, int rows, int cols);
hipError_t launch_matvec_normed(unsigned type, const uint8_t *w, const float *x, const float *r, const float *g,
    float *hout, float eps, float *y, int rows, int cols, hipStream_t stream);
// The same over the q|k|v rows with rope_qkv's rotary step in its epilogue:
// y as rope_qkv leaves it (q rotated), k and v into the cache slot of
// positions[0]. Rows per CU even. The matrix holds q|k|v rows
// [row0, row0 + rows) (row0 even): all of them, or one part.
bool matvec_normed_rope_supported(unsigned type, int rows, int cols);
hipError_t launch_matvec_normed_rope(unsigned type, const uint8_t *w, const float *x, const float *r, const float *g,
    float *hout, float eps, float *y, int rows, int cols, int row0, const int *positions, const float *freq,
    float *keys, float *values, int qd, int kvd, int width, int capacity, hipStream_t stream);
// The same rotary product of h * g with the norm's scale on the row sums,
// from the partial sums of squares of launch_matvec_residual (before the
// rotary step); the shapes of matvec_normed_rope_supported.
hipError_t launch_matvec_scaled_rope(unsigned type, const uint8_t *w, const float *hn, const double *parts, float eps,
    float *y, int rows, int cols, int row0, const int *positions, const float *freq, float *keys, float *values,
    int qd, int kvd, int width, int capacity, hipStream_t stream);
// Both rotary products over q|k|v rows stored as two matrices (q|k of
// type0, then v of type1: Q4_K and Q6_K) in one launch, the CUs split
// between them by bytes: the scaled form where parts is given (x = h * g),
// else the normed form (x the residual, r, g, hout as there).
bool matvec_rope_pair_supported(unsigned type0, int rows0, unsigned type1, int rows1, int cols);
hipError_t launch_matvec_rope_pair(unsigned type0, const uint8_t *w0, int rows0, unsigned type1, const uint8_t *w1,
    int rows1, int cols, const float *x, const float *r, const float *g, float *hout, const double *parts, float eps,
    float *y, const int *positions, const float *freq, float *keys, float *values, int qd, int kvd, int width,
    int capacity, hipStream_t stream);
// The gate|up product of one token with rows interleaved in 16-row blocks
// (gate rows, then their up rows) and silu(gate) * up as its output: Q4_K on
// the one-workgroup-per-tile kernel (more than 32 rows per CU), one column
// chunk.
bool matvec_swiglu_supported(unsigned type, int rows, int cols);
hipError_t launch_matvec_swiglu(unsigned type, const uint8_t *w, const float *x, float *hidden, int rows, int cols,
    hipStream_t stream);
// The same with Gemma's GELU gate (the shapes of matvec_swiglu_supported).
hipError_t launch_matvec_geglu(unsigned type, const uint8_t *w, const float *x, float *hidden, int rows, int cols,
    hipStream_t stream);
// The same of h * g with the norm's scale on the row sums, from the
// partial sums of squares of launch_matvec_residual.
bool matvec_swiglu_scaled_supported(unsigned type, int rows, int cols);
hipError_t launch_matvec_swiglu_scaled(unsigned type, const uint8_t *w, const float *hn, const double *parts,
    float eps, float *hidden, int rows, int cols, hipStream_t stream);
// One token's product added into the residual in place, with h * g and the
// partial sums of squares of h (256 doubles) for the next product.
bool matvec_residual_supported(unsigned type, int rows, int cols);
hipError_t launch_matvec_residual(unsigned type, const uint8_t *w, const float *x, float *res, const float *g,
    float *hn, double *parts, int rows, int cols, hipStream_t stream);
hipError_t launch_matvec_gated(unsigned type, const uint8_t *w, const float *gate, const float *up, float *y,
    int rows, int cols, hipStream_t stream);
// Batches of 2..8 on the same row-balanced layout, the activation digits made
// inside the kernel (matvec.hip); no workspace. x must be 16-byte aligned.
bool smalln_rows_supported(unsigned type, int rows, int cols, int batch);
hipError_t launch_smalln_rows(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    int batch, hipStream_t stream);

// Activation digits of `batch` tokens x `cols` columns (row stride ldx) in
// the layout of blockdot.h for np token slots (smalln.hip).
hipError_t launch_quantize_x(const float *x, int ldx, int cols, int batch, int np, uint8_t *dig, float2 *meta,
    hipStream_t stream);

// Batches above 8 with quantized weights: Q4_K / Q8_0 / Q4_0 on fp16 MFMA
// (prefill_f16.hip), Q6_K on int8 MFMA (prefill.hip). The launch needs
// prefill_workspace bytes of 16-byte-aligned device scratch; prefill_kernel
// names the GEMM kernel.
size_t prefill_workspace(unsigned type, int cols, int batch);
hipError_t launch_prefill(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, int batch,
    void *workspace, hipStream_t stream);
const char *prefill_kernel(unsigned type);

bool prefill_f16_supported(unsigned type);
size_t prefill_f16_workspace(int cols, int batch);
hipError_t launch_prefill_f16(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    int batch, void *workspace, hipStream_t stream);

// Dense F32 / F16 / BF16 batches above 8 as one GEMM on the fp32 matrix cores
// (dense.hip).
// Batches of matrices with few row tiles split the columns over several
// workgroups; their partial sums need dense_gemm_workspace bytes.
bool dense_gemm_supported(unsigned type, int rows, int cols, int batch);
size_t dense_gemm_workspace(int rows, int cols, int batch);
hipError_t launch_dense_gemm(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    int batch, void *workspace, size_t workspace_bytes, hipStream_t s);
// Plain 16-byte-per-thread device copy (dense.hip), for counter calibration.
hipError_t launch_copy(uint4 *dst, const uint4 *src, size_t count, hipStream_t stream);
// Plain streaming read of `count` 16-byte elements, one workgroup per CU
// (dense.hip); `sink` holds kReadSinkWords words.
constexpr int kReadSinkWords = 1024;
hipError_t launch_read(const uint4 *src, size_t count, unsigned *sink, hipStream_t stream);
// The same read in other shapes (dense.hip): `waves` wavefronts per
// workgroup, `depth` 16-byte loads in flight per lane, `per_cu` workgroups
// per CU, `mode` 0 non-temporal loads, 1 default cache policy, 2 into LDS.
hipError_t launch_read_shaped(const uint4 *src, size_t count, unsigned *sink, int waves, int depth, int per_cu,
    int mode, hipStream_t stream);
// Vector steps of the resident decoder (resident.hip) over `count` tokens,
// fp32 device vectors, token i's row at i times the row's stride (floats):
// the decode step ids written (step[0] token, step[1] position); rows
// tokens[i] of a GGUF-layout matrix decoded (row_bytes its stored size)
// times scale; x += r (when r is given) then out = RMS-normalized x times w
// (w may be null); the same with r RMS-normalized times post first and x
// scaled by oscale after the add (n <= kPostNormMax); rotary encoding at
// positions[i] (q rotated in place, k rotated into its slot of `keys`, v
// copied into `values`, both [capacity][kv_heads * width]); the Gemma form
// (per-head RMS norms of q, k and v, then the half-split rotation of q and
// k; width <= 512; k null: q only); causal attention of each token's
// `heads` query heads (width <= 512) over positions [0, positions[i]], the
// last `window` of them when window > 0 (scores: count x heads x max_length
// scratch, used past 8192 positions); out = silu(gate) * up or
// gelu(gate) * up; logits x = cap tanh(x / cap).
constexpr int kPostNormMax = 16384;
hipError_t launch_set_step(uint32_t *step, uint32_t token, int position, hipStream_t stream);
hipError_t launch_embed(const uint8_t *w, unsigned type, size_t row_bytes, int rows, const uint32_t *tokens, int count,
    int cols, float *out, float scale, hipStream_t stream);
hipError_t launch_rms_norm(float *x, const float *r, const float *w, float *out, int n, int count, float eps,
    hipStream_t stream);
hipError_t launch_post_norm(float *x, const float *r, const float *post, float oscale, const float *w, float *out,
    int n, int count, float eps, hipStream_t stream);
hipError_t launch_rope_qkv(float *q, int q_stride, const float *k, int k_stride, const float *v, int v_stride,
    int count, int heads, int kv_heads, int width, const float *freq, const int *positions, int capacity, float *keys,
    float *values, hipStream_t stream);
hipError_t launch_head_norm_rope(float *q, int q_stride, const float *k, int k_stride, const float *v, int v_stride,
    int count, int heads, int kv_heads, int width, const float *q_norm, const float *k_norm, float eps,
    const float *freq, const int *positions, int capacity, float *keys, float *values, hipStream_t stream);
hipError_t launch_softcap(float *x, size_t n, float cap, hipStream_t stream);
// Attention split over the cached positions (resident.hip): `splits`
// workgroups per (KV head, token), then their combination; partials:
// count * heads * splits * (width + 2) floats.
bool attention_split_supported(int heads, int kv_heads, int width, int max_length, int splits);
hipError_t launch_attention_split(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *partials, const int *positions, int count, int heads, int kv_heads, int width, int max_length, int window,
    int splits, float scale, hipStream_t s);
hipError_t launch_attention(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *scores, const int *positions, int count, int heads, int kv_heads, int width, int max_length, int window,
    float scale, hipStream_t stream);
hipError_t launch_silu_mul(const float *gate, int gate_stride, const float *up, int up_stride, float *out, int n,
    int count, hipStream_t stream);
hipError_t launch_gelu_mul(const float *gate, int gate_stride, const float *up, int up_stride, float *out, int n,
    int count, hipStream_t stream);
hipError_t launch_silu_pairs(const float *gu, float *out, int n, int count, hipStream_t stream);
hipError_t launch_gelu_pairs(const float *gu, float *out, int n, int count, hipStream_t stream);
// The greedy choice of each of `count` rows of n logits (first largest among
// the entries not masked; 0xFFFFFFFF for a row with a NaN or +inf, or
// without a finite candidate).
hipError_t launch_greedy(const float *logits, int n, int count, const uint32_t *mask, uint32_t *ids,
    hipStream_t stream);

// Compute units of the current device (counted once per device).
int device_cu_count();

}  // namespace fy
