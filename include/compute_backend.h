/* Provider contract between the compute dispatch layer and one provider.
 *
 * Same struct tag, member order and member types as
 * backend/include/compute_backend.h:12-29, because the engine reads the
 * ROCm provider's table through this layout. No driver types cross it. */
#ifndef NYA_COMPUTE_BACKEND_H
#define NYA_COMPUTE_BACKEND_H
#include "compute.h"
#include <stdint.h>

struct nya_llm_context;
typedef struct nya_backend_interface {
    nya_backend_type type;
    const char *name;
    unsigned capabilities;
    void *(*create)(void);
    void (*destroy)(void *);
    int (*active)(const void *);
    int (*matvec)(void *, const void *, size_t, size_t, unsigned, const float *, float *);
    void *(*plan_create)(void *, const struct nya_llm_context *, size_t);
    void (*plan_free)(void *);
    int (*plan_token)(void *, uint32_t, size_t, int, float *);
    int (*plan_prefill)(void *, const uint32_t *, size_t, size_t, float *);
    void (*plan_stats)(const void *, nya_compute_stats *);
    int (*matmul)(void *, const void *, size_t, size_t, unsigned, const float *, float *, size_t);
    int (*attention_f32)(void *, const nya_compute_attention *);
    int (*plan_read_kv)(void *, size_t, size_t, size_t, float *, float *, size_t);
    void (*context_stats)(const void *, nya_compute_stats *);
} nya_backend_interface;

/* The ROCm provider's table (replaces rocm/rocm.c:193-199). Capabilities are
 * MATVEC | QUANTIZED | MATMUL | RESIDENT; the attention entry is NULL. */
const nya_backend_interface *nya_rocm_backend(void);

/* Entries of the ROCm provider that the engine's table has no slot for; they
 * take the handle its plan_create returned. Batched verification of draft
 * tokens: the forward of tokens [position, position + count) in one run and
 * the target's greedy choice after each (ids[i] for position + i + 1), the
 * count rows of logits too when `logits` is not NULL; 0 or -1 (the plan
 * retires, as after a failed plan_token). The most tokens one verification
 * takes; the plan's vocabulary size. No counterpart in the reference, whose
 * speculative decoding verifies with serial target steps
 * (backend/core/llm_cpu.c:1274-1305). */
int nya_rocm_plan_verify(void *plan, const uint32_t *tokens, size_t count, size_t position, uint32_t *ids,
    float *logits);
size_t nya_rocm_plan_verify_limit(const void *plan);
size_t nya_rocm_plan_vocabulary(const void *plan);

#endif
