/* C ABI of the gfx950 quantized matrix kernel library (libfyodor_hip.so).
 *
 * The ROCm provider (fyodor_amd/rocm/rocm.c) resolves these symbols with
 * dlopen/dlsym, the same way the reference provider resolves the HIP runtime
 * and rocBLAS (rocm/rocm.c:155-166, rocm/abi.h:8-26). They replace the one
 * rocBLAS call on the reference path, rocblas_sgemm(T,N) over host-expanded
 * F32 weights (rocm/rocm.c:123-128), with kernels that read the GGUF block
 * formats directly.
 *
 * Conventions follow the reference's versioned GPU-library bridge
 * (CUDA/cutlass/bridge.h:1-23): device addresses and the stream are passed as
 * uintptr_t and stay owned by the caller; the library never allocates,
 * frees or synchronizes them. Return codes:
 *     0  enqueued on the stream (or, for queries, answered);
 *     1  declined before anything was enqueued (unsupported type or shape);
 *    <0  HIP failure after a possible enqueue; the caller must treat its
 *        device state as failed and recompute the whole request elsewhere.
 *
 * Layouts (backend/include/compute.h:80-83, rocm/rocm.c:124-126):
 *     W  [rows][cols] in the device weight layout: the GGUF row-major
 *        block storage itself, or its nya_hip_weight_pack permutation;
 *     X  [batch][cols] fp32, each batch entry contiguous;
 *     Y  [batch][rows] fp32.
 */
#ifndef FYODOR_HIP_H
#define FYODOR_HIP_H
#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define NYA_HIP_EXPORT __attribute__((visibility("default")))
#else
#define NYA_HIP_EXPORT
#endif
#ifdef __cplusplus
extern "C" {
#endif

#define NYA_HIP_ABI_VERSION 2U

/* GGML storage type IDs (backend/core/llm_internal.h:11-19). */
enum {
    NYA_HIP_F32 = 0, NYA_HIP_F16 = 1, NYA_HIP_Q4_0 = 2, NYA_HIP_Q8_0 = 8,
    NYA_HIP_Q4_K = 12, NYA_HIP_Q6_K = 14, NYA_HIP_BF16 = 30
};

/* Version handshake, as nya_cutlass_abi_version (CUDA/cutlass/bridge.h:17).
 * Returns NYA_HIP_ABI_VERSION. */
NYA_HIP_EXPORT unsigned nya_hip_abi_version(void);

/* Device bytes of a [rows][cols] matrix of `type`. This always equals its
 * GGUF storage size: the device layout only moves bytes. Replaces the F32
 * size from nya_vendor_matrix (backend/core/vendor.c:59-80), which the
 * reference uploads after host expansion. Returns 0, or 1 for an unsupported
 * type or shape (cols not a multiple of the block, a zero or
 * above-INT_MAX dimension, a size_t overflow, or a Q4_0/Q8_0/Q4_K/Q6_K
 * matrix the kernels cannot address: above INT32_MAX bytes or rows above
 * 2^26 columns). Every other entry point declines the same shapes. */
NYA_HIP_EXPORT int nya_hip_weight_bytes(unsigned type, size_t rows, size_t cols, size_t *bytes);

/* Whether the device layout of `type` differs from GGUF storage:
 * 0 the GGUF bytes are uploaded as they are (F32, F16, BF16);
 * 1 they must first pass through nya_hip_weight_pack (Q4_0, Q8_0, Q4_K,
 *   Q6_K, whose blocks are regrouped into per-lane field planes so that
 *   every kernel load instruction reads one contiguous span);
 * -1 unsupported type. */
NYA_HIP_EXPORT int nya_hip_weight_layout(unsigned type);

/* Host-side (CPU) conversion of GGUF bytes `src` into the device layout at
 * `dst`, both host memory of nya_hip_weight_bytes bytes, not overlapping.
 * Replaces the host F32 decode of the reference weight upload
 * (rocm/rocm.c:90-94, backend/core/vendor.c:81-85) with a byte
 * permutation of the same size. Returns 0, or 1 when unsupported. */
NYA_HIP_EXPORT int nya_hip_weight_pack(void *dst, const void *src, unsigned type,
    size_t rows, size_t cols);

/* Device workspace that nya_hip_matmul needs for this request (0 when none).
 * Returns 0, or 1 when the request is unsupported. */
NYA_HIP_EXPORT int nya_hip_workspace_bytes(unsigned type, size_t rows, size_t cols,
    size_t batch, size_t *bytes);

/* Enqueue Y = X * W^T for batch >= 1 (replaces rocm/rocm.c:127-128).
 * batch 1 is the decode matvec, batch 2..8 the small-N path and larger
 * batches the prefill GEMM. `workspace` holds at least the bytes reported
 * by nya_hip_workspace_bytes for the same arguments (it may be 0 then). */
NYA_HIP_EXPORT int nya_hip_matmul(uintptr_t w, unsigned type, size_t rows, size_t cols,
    uintptr_t x, uintptr_t y, size_t batch, uintptr_t workspace, size_t workspace_bytes,
    uintptr_t stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): Y = X * W^T exactly as nya_hip_matmul with its
 * workspace (same kernels, same results per token), but the kernels'
 * scratch is a fixed device array of NYA_HIP_STATIC_SCRATCH_BYTES inside
 * this library, one per GPU, held until the process ends; the call
 * allocates and frees nothing. Prefill batches (above 8 tokens) run in
 * token chunks whose scratch fits the array; where not even a 64-token
 * chunk fits (rows of about 254k columns and more) the batch runs as
 * 8-token launches, which is what nya_hip_matmul does with a workspace
 * shorter than it asks for (then the results equal that call's, not the
 * GEMM's). Returns 0, 1 when declined (the rules of nya_hip_matmul), <0 on
 * a HIP failure; NYA_HIP_STATUS_SCRATCH is kept for callers that test for
 * it and is not returned. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race and must be serialized by the caller; the array keeps the
 * last call's contents, which no call reads before writing. */
#define NYA_HIP_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
#define NYA_HIP_STATUS_SCRATCH 2
NYA_HIP_EXPORT int nya_hip_matmul_static(uintptr_t w, unsigned type, size_t rows, size_t cols,
    uintptr_t x, uintptr_t y, size_t batch, uintptr_t stream);

/* Name of the main kernel nya_hip_matmul launches for these arguments, as it
 * appears in a rocprofv3 kernel trace, or NULL when unsupported. Diagnostic
 * only; it launches nothing. */
NYA_HIP_EXPORT const char *nya_hip_kernel_name(unsigned type, size_t rows, size_t cols, size_t batch);

/* Diagnostics, no counterpart in the reference: enqueue a plain device copy
 * of `bytes` (a multiple of 16, 16-byte aligned pointers) with one 16-byte
 * load and one 16-byte store per element, used to calibrate HBM read/write
 * byte counters (rocprofv3 FETCH_SIZE / WRITE_SIZE) against a known size. */
NYA_HIP_EXPORT int nya_hip_copy(uintptr_t dst, uintptr_t src, size_t bytes, uintptr_t stream);

/* Diagnostics, no counterpart in the reference: enqueue a plain streaming
 * read of `bytes` (a multiple of 16, 16-byte aligned) with non-temporal
 * 16-byte loads, one workgroup per compute unit over a contiguous share and
 * nothing computed: the HBM read time a decode matvec of the same bytes can
 * approach. `sink` (4-byte aligned, NYA_HIP_READ_SINK_BYTES) receives at most
 * a few words and is otherwise left as it is. */
#define NYA_HIP_READ_SINK_BYTES 4096
NYA_HIP_EXPORT int nya_hip_read(uintptr_t src, size_t bytes, uintptr_t sink, uintptr_t stream);

/* Diagnostics, no counterpart in the reference: the same plain read in
 * another shape, to measure which read structure streams a given size
 * fastest. `waves` wavefronts per workgroup and `depth` 16-byte loads in
 * flight per lane, as one of the pairs 4x32, 4x16, 8x16, 8x8, 16x8, 16x4;
 * `per_cu` (1..4) workgroups per compute unit; `mode` 0 non-temporal loads
 * into registers, 1 loads with the default cache policy, 2 loads straight
 * into LDS (buffer_load_dwordx4 ... lds), 3 as 0 followed by an output store
 * of 56 words per workgroup (the store every real kernel ends with) at
 * sink + 256 bytes per workgroup: for mode 3 `sink` holds
 * NYA_HIP_READ_STORE_SINK_BYTES. Returns 1 for any other shape. */
#define NYA_HIP_READ_STORE_SINK_BYTES ((size_t)1 << 20)
NYA_HIP_EXPORT int nya_hip_read_shaped(uintptr_t src, size_t bytes, uintptr_t sink, int waves, int depth,
    int per_cu, int mode, uintptr_t stream);

/* The vector steps of the decoder over `count` tokens (1..65535) at once,
 * for a provider that keeps a whole model's token forward on the device (the
 * resident plan of backend/include/compute.h:37-51; the reference's CUDA
 * provider runs the same steps as its own kernels,
 * CUDA/resident.inc:466-578). All vectors are fp32 device arrays (4-byte
 * aligned), token i's row at i times the row length; token ids (uint32) and
 * positions (int32) are device arrays, so the same calls serve every token.
 * Each call enqueues one kernel and returns 0, 1 when declined (null or
 * misaligned pointers, zero or out-of-range sizes), <0 on a HIP failure.
 * Each restates one step of the engine's CPU token forward,
 * backend/core/llm_cpu.c:424-578 (its LLaMA and Gemma branches). */

/* step[0] = token (uint32), step[1] = position (int32), written on the
 * stream: the ids of one decode token for the calls below (tokens = step,
 * positions = step + 4 bytes, count 1), so a recorded sequence of those
 * calls serves every token. No counterpart in the reference (its CUDA plan
 * passes them as kernel arguments, CUDA/resident.inc:466-578). */
NYA_HIP_EXPORT int nya_hip_step(uintptr_t step, unsigned token, size_t position, uintptr_t stream);

/* out[i][cols] = row tokens[i] of a [rows][cols] matrix of `type` in GGUF
 * storage (not packed), decoded as nya_llm_tensor_value does
 * (backend/core/llm_quant.c:70-142), times scale: the token embedding
 * gather (backend/core/llm_cpu.c:71-80, :452-453; Gemma's scale sqrt(d),
 * :453, 1 otherwise). An id past the matrix gives a zero row. */
NYA_HIP_EXPORT int nya_hip_embed(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t tokens,
    size_t count, uintptr_t out, float scale, uintptr_t stream);

/* Per token row of n: when residual is nonzero, x += residual first (x is
 * written back); then out = x * s * weight with
 * s = 1 / sqrt(sum x^2 / n + epsilon), the sum of squares in double, weight
 * 0 meaning ones (backend/core/llm_cpu.c:83-104; the residual add of :514
 * folded in). */
NYA_HIP_EXPORT int nya_hip_rms_norm(uintptr_t x, uintptr_t residual, uintptr_t weight, uintptr_t out, size_t n,
    size_t count, float epsilon, uintptr_t stream);

/* The residual add of a block whose branch carries its own norm (Gemma's
 * post-attention and post-feed-forward norms, backend/core/llm_cpu.c:514,
 * :531, :544-547), folded into the next norm step: per token row of n
 * (at most 16384), r' = residual * s_r * post with
 * s_r = 1 / sqrt(sum residual^2 / n + epsilon) (post 0: r' = residual;
 * residual 0: no add), x = (x + r') * output_scale written back (the
 * block's output scale, 1 where it has none), then out = x * s * weight as
 * nya_hip_rms_norm. The residual rows are read, not written. */
NYA_HIP_EXPORT int nya_hip_post_norm(uintptr_t x, uintptr_t residual, uintptr_t post, float output_scale,
    uintptr_t weight, uintptr_t out, size_t n, size_t count, float epsilon, uintptr_t stream);

/* The Gemma form of nya_hip_rope_qkv (backend/core/llm_cpu.c:487-500): each
 * head of width <= 512 is RMS-normalized on its own (q heads with q_norm,
 * k heads with k_norm, v heads without a weight; :360-363), then q and k
 * heads have their halves rotated, the pair (j, j + width / 2) by
 * p * frequencies[j] (:345-358): q in place, k into the key cache slot of
 * positions[i], v (normalized only) into the value slot. v may equal k
 * with the same stride (layers without a value matrix store the key's
 * projection as the value, :492). k = 0: the q heads only (layers that
 * read another layer's cache, :488-489); k_norm, keys and values are then
 * not used. A position outside [0, capacity) leaves everything alone. */
NYA_HIP_EXPORT int nya_hip_head_norm_rope(uintptr_t q, size_t q_stride, uintptr_t k, size_t k_stride, uintptr_t v,
    size_t v_stride, size_t count, size_t heads, size_t kv_heads, size_t width, uintptr_t q_norm, uintptr_t k_norm,
    float epsilon, uintptr_t frequencies, uintptr_t positions, size_t capacity, uintptr_t keys, uintptr_t values,
    uintptr_t stream);

/* x[i] = cap * tanh(x[i] / cap) over n logits: the final soft cap
 * (backend/core/llm_cpu.c:562-565). cap > 0. */
NYA_HIP_EXPORT int nya_hip_softcap(uintptr_t x, size_t n, float cap, uintptr_t stream);

/* The rotary step of each token i at position p = positions[i]: its q row
 * (q + i q_stride floats, `heads` heads of `width`) has the interleaved
 * pairs (2j, 2j+1) of every head rotated in place, and its k row
 * (k + i k_stride, kv_heads heads) rotated into keys + p kv_heads width, by
 * the angle p * frequencies[j] (backend/core/llm_cpu.c:298-324, angles
 * :429-432); its v row (v + i v_stride) is copied to
 * values + p kv_heads width — the token's slots of the layer's KV cache
 * ([capacity][kv_heads * width] each; the cache writes of :433-436). A
 * position outside [0, capacity) leaves the rows and the cache alone. */
NYA_HIP_EXPORT int nya_hip_rope_qkv(uintptr_t q, size_t q_stride, uintptr_t k, size_t k_stride, uintptr_t v,
    size_t v_stride, size_t count, size_t heads, size_t kv_heads, size_t width, uintptr_t frequencies,
    uintptr_t positions, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream);

/* Causal attention of each token (its q at q + i q_stride): for each of
 * `heads` heads (grouped onto kv_heads key/value heads, width at most 512),
 * scores q.k_t * scale over the cached positions t = 0 .. positions[i]
 * (at most max_length) of keys / values ([max_length][kv_heads * width]
 * rows), a softmax, and out[i] = sum_t p_t v_t (backend/core/llm_cpu.c:491-511).
 * window > 0 keeps the last `window` of those positions, as the engine
 * bounds a sliding layer's attention (:486-488); 0 keeps all. `scores` is
 * scratch of count * heads * max_length floats, needed (and used) only
 * when max_length exceeds 8192. */
NYA_HIP_EXPORT int nya_hip_attention(uintptr_t q, size_t q_stride, uintptr_t keys, uintptr_t values, uintptr_t out,
    uintptr_t scores, uintptr_t positions, size_t count, size_t heads, size_t kv_heads, size_t width,
    size_t max_length, size_t window, float scale, uintptr_t stream);

/* No counterpart in the reference's C engine (the reference's CUDA plan
 * splits long attention the same way, CUDA/resident.inc:119-133): the
 * attention of nya_hip_attention for long contexts, split over the cached
 * positions. `splits` workgroups per (KV head, token) each take a
 * contiguous share of the token's causal range for all the query heads
 * that share the KV head (every cached K and V row read once per token),
 * and a second launch combines their partial maxima, sums and weighted
 * values (out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M)): the same
 * softmax, with the exponentials rescaled per split. `partials` is scratch
 * of count * heads * splits * (width + 2) floats (16-byte aligned). Runs for
 * width 64, 128 or 256 with heads / kv_heads in {1, 2, 4, 8} (8 up to width
 * 128), or width 512 with heads / kv_heads in {1, 2};
 * ceil(max_length / splits) <= 1024, 16-byte aligned q, keys,
 * values and q_stride a multiple of 4; else returns 1. q == 0 queries the
 * shape (heads, kv_heads, width, max_length, splits): 0 where it runs. */
NYA_HIP_EXPORT int nya_hip_attention_split(uintptr_t q, size_t q_stride, uintptr_t keys, uintptr_t values,
    uintptr_t out, uintptr_t partials, uintptr_t positions, size_t count, size_t heads, size_t kv_heads, size_t width,
    size_t max_length, size_t window, size_t splits, float scale, uintptr_t stream);

/* out[i][j] = g / (1 + e^-g) * u with g = gate[i gate_stride + j],
 * u = up[i up_stride + j], out rows of n (backend/core/llm_cpu.c:336-341,
 * SiLU of the gate times the up product). For one token out may be gate
 * itself; for several it must not overlap either input. */
NYA_HIP_EXPORT int nya_hip_silu_mul(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride,
    uintptr_t out, size_t n, size_t count, uintptr_t stream);

/* The same with GELU's tanh form in place of SiLU, Gemma's gate
 * (backend/core/llm_cpu.c:329-341):
 * out = 0.5 g (1 + tanh(0.7978845608028654 (g + 0.044715 g^3))) u. */
NYA_HIP_EXPORT int nya_hip_gelu_mul(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride,
    uintptr_t out, size_t n, size_t count, uintptr_t stream);

/* No counterpart in the reference: one token's product of the decoder's
 * normalized residual, nya_hip_rms_norm folded into the product that reads
 * it. h = x + r (r = 0: h = x), xn = h * scale * norm with
 * scale = 1 / sqrt(sum h^2 / cols + eps) (backend/core/llm_cpu.c:83-104, the
 * sum in double in the norm step's order), y = W xn as nya_hip_matmul of one
 * column; with r, h is written to hout (cols floats, overlapping neither x nor
 * r: the norm step writes x in place, which this product cannot while its
 * other workgroups read x). y and hout equal nya_hip_rms_norm followed by
 * nya_hip_matmul bit for bit. For callers that run one decode token (the
 * resident plan): one launch fewer per block. w == 0 queries the shape: 0
 * where it runs (Q4_K, Q6_K, Q8_0, Q4_0 with cols a multiple of 256 up to
 * 4096 and at most 32 rows per CU), else 1; then also 1 for missing or
 * misaligned (16 bytes; y 4) vectors. */
NYA_HIP_EXPORT int nya_hip_matvec_normed(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t r, uintptr_t norm, float eps, uintptr_t hout, uintptr_t y, uintptr_t stream);

/* No counterpart in the reference: nya_hip_matvec_normed of the q|k|v rows
 * ((heads + 2 kv_heads) width of them: q, then k, then v) with
 * nya_hip_rope_qkv's rotary step of one token in its epilogue (frequencies,
 * positions, capacity, keys and values as there): y is left as the two
 * steps leave it (q rows rotated, k and v rows as produced) and the key and
 * value rows go into the cache slot of positions[0], bit for bit, for a
 * position in [0, capacity); outside it nothing is rotated or stored, as
 * there. W holds the q|k|v rows [first_row, first_row + rows): all of them
 * (first_row 0), or one part where the rows are stored in two matrices of
 * different types (q|k and v of a Q4_K_M model), one call per part
 * (first_row even; y is the part's own rows). One launch for the attention
 * norm, the q|k|v product and the rotary step of a decode token (one per
 * part). w == 0 queries the shape: as nya_hip_matvec_normed, with rows and
 * rows per CU even. */
NYA_HIP_EXPORT int nya_hip_matvec_normed_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row,
    uintptr_t x, uintptr_t r, uintptr_t norm, float eps, uintptr_t hout, uintptr_t y, uintptr_t positions,
    uintptr_t frequencies, size_t heads, size_t kv_heads, size_t width, size_t capacity, uintptr_t keys,
    uintptr_t values, uintptr_t stream);

/* No counterpart in the reference: both parts of q|k|v rows stored as two
 * matrices — q|k (rows0 rows of type0) and v (rows1 of type1): Q4_K and
 * Q6_K, a Q4_K_M model's value matrices — through the rotary product in one
 * launch, the CUs split between the parts by their bytes. With parts
 * nonzero, the scaled form of nya_hip_matvec_scaled_rope (x = hn; r, norm
 * and hout unused); else the normed form of nya_hip_matvec_normed_rope (x,
 * r, norm, hout as there). y receives all rows0 + rows1 = (heads +
 * 2 kv_heads) width rows and the cache slot of positions[0] the key and
 * value rows, as the two per-part calls leave them (bit for bit). w0 == 0
 * queries the shape (type0, rows0, type1, rows1, cols): 0 where it runs
 * (Q4_K then Q6_K, even row counts, cols a multiple of 256 up to 4096, at
 * most 32 rows per workgroup of either part), else 1. */
NYA_HIP_EXPORT int nya_hip_matvec_rope_pair(uintptr_t w0, unsigned type0, size_t rows0, uintptr_t w1, unsigned type1,
    size_t rows1, size_t cols, uintptr_t x, uintptr_t r, uintptr_t norm, uintptr_t hout, uintptr_t parts, float eps,
    uintptr_t y, uintptr_t positions, uintptr_t frequencies, size_t heads, size_t kv_heads, size_t width,
    size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream);

/* No counterpart in the reference: nya_hip_matvec_normed_rope of the decoder's
 * normalized residual from nya_hip_matvec_residual's outputs (the previous
 * block's down product): the q|k|v row sums of W hn times the norm's scale
 * s = 1 / sqrt(sum parts / cols + eps), then nya_hip_rope_qkv's rotary step
 * and cache store as there. Like nya_hip_matvec_swiglu_scaled, no workgroup
 * waits for a reduction over the row, and y meets the product's error bound
 * as nya_hip_rms_norm followed by the product and nya_hip_rope_qkv do, not
 * bit for bit. For callers that run one decode token (the resident plan):
 * the attention norm of every block after the first without a reduction in
 * each workgroup. first_row as there. w == 0 queries the shape: 0 where it
 * runs (the shapes of nya_hip_matvec_normed_rope), else 1; then also 1 for
 * missing or misaligned vectors (hn 16 bytes, parts 8, y and the rotary
 * arguments 4). */
NYA_HIP_EXPORT int nya_hip_matvec_scaled_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row,
    uintptr_t hn, uintptr_t parts, float eps, uintptr_t y, uintptr_t positions, uintptr_t frequencies, size_t heads,
    size_t kv_heads, size_t width, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream);

/* No counterpart in the reference: the gate|up product of one token with
 * the gated SiLU as its output. W (rows = 2 n, the library's layout) holds
 * the feed-forward gate and up rows interleaved in 16-row blocks: rows
 * 32 b .. 32 b + 15 are gate rows 16 b .. 16 b + 15, rows 32 b + 16 ..
 * 32 b + 31 their up rows. hidden[j] = silu(g_j) * u_j (as nya_hip_silu_pairs
 * forms it) with g_j, u_j the products of x with gate and up row j, equal bit
 * for bit to nya_hip_matmul of one column followed by nya_hip_silu_pairs;
 * each SiLU is formed once. For callers that lay out the matrix so (the
 * resident plan): one launch and one pass over the products fewer per block.
 * w == 0 queries the shape: 0 where it runs, 1 where it does not (Q4_K only,
 * rows a multiple of 32 and more than 32 per CU, cols a multiple of 256 up to
 * 16384); then also 1 for x or hidden missing or misaligned. */
NYA_HIP_EXPORT int nya_hip_matvec_swiglu(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t hidden, uintptr_t stream);

/* Partial sums of squares handed from nya_hip_matvec_residual to
 * nya_hip_matvec_swiglu_scaled: doubles. */
#define NYA_HIP_NORM_PARTS 256

/* No counterpart in the reference: one decode token's product added into the
 * decoder's residual, with what the next RMS norm needs, so that the next
 * product can take the norm without a step of its own. res[i] += (W x)[i] for
 * i < rows (the residual add of nya_hip_rms_norm, bit for bit: the product is
 * nya_hip_matmul's of one column), hn[i] = res[i] * norm[i] (the new res),
 * and parts[0 .. NYA_HIP_NORM_PARTS) the double sums of res[i]^2 over the
 * kernel's workgroups' rows, zeros past its last (their total is the norm's
 * sum of squares; the order differs from the norm step's). For callers that
 * run one decode token (the resident plan): the attention output product
 * with the feed-forward norm's inputs, read by nya_hip_matvec_swiglu_scaled.
 * w == 0 queries the shape: 0 where it runs (Q4_K, Q6_K, Q8_0, Q4_0 with
 * cols a multiple of 256 up to 20480, at most 64 rows per CU, on at most 256
 * CUs), else 1; then also 1 for missing or misaligned vectors (w, x: 16
 * bytes; res, norm, hn: 4; parts: 8) or hn or parts overlapping x, or hn
 * overlapping res. */
NYA_HIP_EXPORT int nya_hip_matvec_residual(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t res, uintptr_t norm, uintptr_t hn, uintptr_t parts, uintptr_t stream);

/* No counterpart in the reference: nya_hip_matvec_swiglu of the decoder's
 * normalized residual from nya_hip_matvec_residual's outputs, with the RMS
 * norm's scale s = 1 / sqrt(sum parts / cols + eps) (backend/core/llm_cpu.c:
 * 83-104) multiplying the gate and up row sums: hidden = silu(g) * u of
 * g, u = s (W hn), the same in every workgroup. The scale is one number, so
 * W (hn s) = s (W hn): no workgroup waits for a reduction over the row
 * before its products. hidden meets the product's error bound as
 * nya_hip_rms_norm followed by nya_hip_matvec_swiglu does, not bit for bit.
 * For callers that run one decode token (the resident plan): the
 * feed-forward norm's launch goes. w == 0 queries the shape: 0 where it runs
 * (nya_hip_matvec_swiglu's shapes), else 1; then also 1 for missing or
 * misaligned vectors (hn 16 bytes, parts 8, hidden 4). */
NYA_HIP_EXPORT int nya_hip_matvec_swiglu_scaled(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t hn,
    uintptr_t parts, float eps, uintptr_t hidden, uintptr_t stream);

/* No counterpart in the reference: nya_hip_matvec_swiglu with Gemma's GELU
 * gate (backend/core/llm_cpu.c:329-341) in place of SiLU:
 * hidden[j] = 0.5 g (1 + tanh(0.7978845608028654 (g + 0.044715 g^3))) u,
 * as nya_hip_gelu_pairs forms it, bit for bit with nya_hip_matmul of one
 * column followed by nya_hip_gelu_pairs. The shapes and the shape query of
 * nya_hip_matvec_swiglu. */
NYA_HIP_EXPORT int nya_hip_matvec_geglu(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t hidden, uintptr_t stream);

/* out[i][j] = silu(g) * u for row i of gu (count rows of 2 n floats holding
 * gate and up values in 16-element blocks: g = gu[i][32 (j / 16) + j % 16],
 * u 16 further), out rows of n (n a multiple of 16; out must not overlap gu);
 * silu(g) * u = g / (1 + e^-g) * u as nya_hip_silu_mul forms it. The
 * feed-forward step of the gate|up layout of nya_hip_matvec_swiglu for runs
 * of several tokens. */
NYA_HIP_EXPORT int nya_hip_silu_pairs(uintptr_t gu, uintptr_t out, size_t n, size_t count, uintptr_t stream);

/* The same with Gemma's GELU gate as nya_hip_gelu_mul forms it: the
 * feed-forward step of nya_hip_matvec_geglu's layout for runs of several
 * tokens. */
NYA_HIP_EXPORT int nya_hip_gelu_pairs(uintptr_t gu, uintptr_t out, size_t n, size_t count, uintptr_t stream);

/* No counterpart in the reference: the decoder's gated SiLU step (as
 * nya_hip_silu_mul computes it, backend/core/llm_cpu.c:336-341) folded into
 * the down product of one token. y = W v with v[j] = silu(gate[j]) * up[j],
 * j < cols, W as for nya_hip_matmul (the library's layout); v is formed as
 * each group of it is loaded, with the step's own operations, so y equals
 * nya_hip_silu_mul followed by nya_hip_matmul of one column bit for bit.
 * For callers that run one decode token (the resident plan): it saves one
 * launch per block. Returns 1 for shapes the row kernel does not take
 * (quantized types Q4_K / Q6_K / Q8_0 / Q4_0 only, and for Q4_K at most 64
 * rows per CU) and for gate / up not 16-byte aligned: the caller runs the
 * two steps instead. */
NYA_HIP_EXPORT int nya_hip_matvec_gated(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t gate,
    uintptr_t up, uintptr_t y, uintptr_t stream);

/* ids[i] = the greedy choice of row i of `count` rows of n fp32 logits
 * (logits + i n), as backend/core/llm_cpu.c:896-904 (nya_llm_sample at
 * temperature 0) picks it after the suppressed tokens are masked
 * (backend/core/llm_cpu.c:570-574): the first index of the largest value
 * among the entries whose bit in `mask` is clear (uint32 words, bit j % 32
 * of word j / 32; 0: none masked); 0xFFFFFFFF for a row holding a
 * non-finite value anywhere (the engine rejects non-finite model output
 * before masking) or with every entry masked. The resident plan's batched
 * verification of draft tokens downloads these ids instead of `count` rows
 * of logits. */
NYA_HIP_EXPORT int nya_hip_greedy(uintptr_t logits, size_t n, size_t count, uintptr_t mask, uintptr_t ids,
    uintptr_t stream);

#ifdef __cplusplus
}
#endif
#endif
