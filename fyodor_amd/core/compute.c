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

/* ---- batched verification and greedy speculative decoding ----------------
 * Extensions of this build (no slot in the engine's provider table): they
 * reach the ROCm provider's plan directly. */

static int rocm_plan(const nya_compute_plan *p)
{
    return p && p->api == nya_rocm_backend();
}

int nya_compute_plan_verify(nya_compute_plan *p, const unsigned int *tokens, size_t count,
    size_t position, unsigned int *ids, float *logits)
{
    return rocm_plan(p) ? nya_rocm_plan_verify(p->state, tokens, count, position, ids, logits) : -1;
}

size_t nya_compute_plan_verify_limit(const nya_compute_plan *p)
{
    return rocm_plan(p) ? nya_rocm_plan_verify_limit(p->state) : 0;
}

static int is_stop(unsigned int token, const unsigned int *stops, size_t stop_count)
{
    for (size_t i = 0; i < stop_count; ++i)
        if (stops[i] == token) return 1;
    return 0;
}

/* Runs committed tokens seq[from, to) through a plan (the prompt, or the
 * draft catching up on what the target accepted). */
static int catch_up(nya_compute_plan *p, const unsigned int *seq, size_t from, size_t to, float *scratch)
{
    if (to - from == 1) return p->api->plan_token(p->state, seq[from], from, 0, NULL);
    return p->api->plan_prefill(p->state, seq + from, to - from, from, scratch);
}

/* The engine's greedy speculative loop (backend/core/llm_cpu.c:1252-1317,
 * temperature 0, ordinary draft) with one target verification per round.
 * State between rounds: `pending`, the last emitted token, sits at position
 * P and is in neither cache yet; seq[0, P] holds the prompt and every
 * emitted token; the target's cache holds [0, P), the draft's
 * [0, draft_valid). A round: the draft catches up to P, proposes
 * p_0..p_{m-1} (running pending, p_0, .., p_{m-2} at P, P + 1, ..), the
 * target verifies [pending, p_0, .., p_{m-1}] at P, and its choices
 * ids[0..m] are emitted while the proposals match: ids[j] follows pending
 * and p_0..p_{j-1}, which is what the engine's target step j computes. */
int nya_compute_generate_greedy(nya_compute_plan *target, nya_compute_plan *draft,
    const unsigned int *prompt, size_t prompt_count, size_t window, size_t limit,
    const unsigned int *stops, size_t stop_count, unsigned int *out, size_t *out_count,
    nya_compute_speculation *stats)
{
    nya_compute_speculation st;
    memset(&st, 0, sizeof(st));
    if (out_count) *out_count = 0;
    if (stats) *stats = st;
    const size_t vocabulary = rocm_plan(target) ? nya_rocm_plan_vocabulary(target->state) : 0;
    size_t verify = nya_compute_plan_verify_limit(target);
    if (!vocabulary || !prompt || !prompt_count || !out || !out_count || !limit || window > 32 ||
        (stop_count && !stops) || prompt_count > SIZE_MAX / 8 || limit > SIZE_MAX / 8)
        return -1;
    if (!draft) window = 0;
    if (window && (!rocm_plan(draft) || nya_rocm_plan_vocabulary(draft->state) != vocabulary ||
                   !nya_compute_plan_verify_limit(draft)))
        return -1;
    if (window > verify - 1) window = verify - 1;
    for (size_t i = 0; i < prompt_count; ++i)
        if (prompt[i] >= vocabulary) return -1;
    for (size_t i = 0; i < stop_count; ++i)
        if (stops[i] >= vocabulary) return -1;
    unsigned int *seq = malloc((prompt_count + limit) * sizeof(*seq));
    float *scratch = malloc(vocabulary * sizeof(float));
    int result = -1;
    if (!seq || !scratch) goto done;
    memcpy(seq, prompt, prompt_count * sizeof(*seq));
    size_t P = prompt_count - 1, draft_valid = 0, generated = 0;
    /* The prompt but its last token; that one is the first pending token. */
    if (P > 0) {
        if (catch_up(target, seq, 0, P, scratch)) goto done;
        st.target_tokens += P;
        if (window) {
            if (catch_up(draft, seq, 0, P, scratch)) goto done;
            ++st.draft_steps;
            draft_valid = P;
        }
    }
    int stopped = 0;
    while (!stopped && generated < limit) {
        unsigned int batch[33], ids[33];
        size_t m = window < limit - generated ? window : limit - generated;
        batch[0] = seq[P];
        if (m) {
            if (draft_valid < P) {
                if (catch_up(draft, seq, draft_valid, P, scratch)) goto done;
                ++st.draft_steps;
            }
            /* Proposal i follows batch[0..i]: the draft's own greedy choice. */
            for (size_t i = 0; i < m; ++i) {
                unsigned int next;
                if (nya_compute_plan_verify(draft, &batch[i], 1, P + i, &next, NULL)) goto done;
                ++st.draft_steps;
                ++st.draft_tokens;
                batch[i + 1] = next;
                if (is_stop(next, stops, stop_count)) { m = i + 1; break; }
            }
            draft_valid = P + m;
        }
        if (nya_compute_plan_verify(target, batch, m + 1, P, ids, NULL)) goto done;
        ++st.rounds;
        st.target_tokens += m + 1;
        size_t j = 0;
        for (;;) {
            const unsigned int g = ids[j];
            out[generated++] = g;
            seq[P + 1 + j] = g;
            if (is_stop(g, stops, stop_count)) { stopped = 1; break; }
            if (generated == limit || j == m || batch[j + 1] != g) break;
            ++st.accepted;
            ++j;
        }
        P += 1 + j;
        if (draft_valid > P) draft_valid = P;
    }
    st.generated = generated;
    *out_count = generated;
    result = 0;
done:
    if (stats) *stats = st;
    free(seq);
    free(scratch);
    return result;
}
