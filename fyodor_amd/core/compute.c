/* Compute dispatch layer for the ROCm provider (backend/core/compute.c:1-152).
 *
 * The engine's own compute.c lists every compiled provider; this build
 * compiles one, the ROCm provider, so "rocm" is the only name that creates a
 * context. Every entry point forwards through the provider table and yields
 * -1 / NULL when the provider is missing or has failed, which is the signal
 * for the engine to run its CPU kernel (backend/core/llm_quant.c:159-160). */
#include "compute_backend.h"
#include <stdlib.h>
#include <string.h>

struct nya_compute_context { const nya_backend_interface *api; void *state; };
struct nya_compute_plan { const nya_backend_interface *api; void *state; };

static const nya_backend_interface *provider_named(const char *name)
{
    const nya_backend_interface *rocm = nya_rocm_backend();
    return name && !strcmp(name, rocm->name) ? rocm : NULL;
}

static int live(const nya_compute_context *c)
{
    return c && c->api->active(c->state);
}

nya_compute_context *nya_compute_create(void)
{
    return nya_compute_create_for(getenv("NYA_COMPUTE"));
}

/* backend/core/compute.c:40-46 */
int nya_compute_backend_known(const char *provider)
{
    static const char *const known[] = {"cpu", "cuda", "vulkan", "rocm", "mlx"};
    for (size_t i = 0; provider && i < sizeof(known) / sizeof(known[0]); ++i)
        if (!strcmp(provider, known[i])) return 1;
    return 0;
}

int nya_compute_backend_compiled(const char *provider)
{
    return provider_named(provider) != NULL;
}

/* backend/core/compute.c:59-72: NULL selects "cpu", which this build does
 * not compile, so the caller keeps its own CPU kernels. */
nya_compute_context *nya_compute_create_for(const char *selection)
{
    const nya_backend_interface *api = provider_named(selection ? selection : "cpu");
    if (!api) return NULL;
    nya_compute_context *c = calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->api = api;
    c->state = api->create();
    if (c->state) return c;
    free(c);
    return NULL;
}

void nya_compute_free(nya_compute_context *c)
{
    if (!c) return;
    c->api->destroy(c->state);
    free(c);
}

void nya_compute_context_stats(const nya_compute_context *c, nya_compute_stats *stats)
{
    if (!stats) return;
    memset(stats, 0, sizeof(*stats));
    if (c && c->api->context_stats) c->api->context_stats(c->state, stats);
}

const char *nya_compute_name(const nya_compute_context *c)
{
    return live(c) ? c->api->name : "cpu";
}

unsigned nya_compute_capabilities(const nya_compute_context *c)
{
    return live(c) ? c->api->capabilities : 0;
}

int nya_compute_matvec_typed(nya_compute_context *c, const void *w, size_t rows,
    size_t cols, unsigned type, const float *x, float *y)
{
    return live(c) ? c->api->matvec(c->state, w, rows, cols, type, x, y) : -1;
}

int nya_compute_matvec(nya_compute_context *c, const void *w, size_t rows, size_t cols,
    const float *x, float *y)
{
    return nya_compute_matvec_typed(c, w, rows, cols, 0, x, y);
}

int nya_compute_matmul_typed(nya_compute_context *c, const void *w, size_t rows, size_t cols,
    unsigned type, const float *x, float *y, size_t batch)
{
    return live(c) && c->api->matmul ? c->api->matmul(c->state, w, rows, cols, type, x, y, batch) : -1;
}

int nya_compute_attention_f32(nya_compute_context *c, const nya_compute_attention *a)
{
    return live(c) && c->api->attention_f32 ? c->api->attention_f32(c->state, a) : -1;
}

nya_compute_plan *nya_compute_plan_create(nya_compute_context *c,
    const struct nya_llm_context *model, size_t capacity)
{
    if (!live(c) || !c->api->plan_create) return NULL;
    nya_compute_plan *p = calloc(1, sizeof(*p));
    if (!p) return NULL;
    p->api = c->api;
    p->state = c->api->plan_create(c->state, model, capacity);
    if (p->state) return p;
    free(p);
    return NULL;
}

void nya_compute_plan_free(nya_compute_plan *p)
{
    if (!p) return;
    p->api->plan_free(p->state);
    free(p);
}

int nya_compute_plan_token(nya_compute_plan *p, unsigned int token, size_t position,
    int logits, float *output)
{
    return p ? p->api->plan_token(p->state, token, position, logits, output) : -1;
}

int nya_compute_plan_prefill(nya_compute_plan *p, const unsigned int *tokens, size_t count,
    size_t position, float *output)
{
    return p && p->api->plan_prefill ? p->api->plan_prefill(p->state, tokens, count, position, output) : -1;
}

void nya_compute_plan_stats(const nya_compute_plan *p, nya_compute_stats *stats)
{
    if (!stats) return;
    memset(stats, 0, sizeof(*stats));
    if (p && p->api->plan_stats) p->api->plan_stats(p->state, stats);
}

int nya_compute_plan_read_kv(nya_compute_plan *p, size_t layer, size_t position,
    size_t count, float *keys, float *values, size_t elements)
{
    return p && p->api->plan_read_kv ?
        p->api->plan_read_kv(p->state, layer, position, count, keys, values, elements) : -1;
}
