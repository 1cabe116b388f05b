/* Compute dispatch layer for the ROCm provider (backend/core/compute.c:1-152).
 *
 * The engine's own compute.c lists every compiled provider; this library
 * compiles one, the ROCm provider, so "rocm" is the only name that creates a
 * context. Every entry point forwards through the provider table and yields
 * -1 / NULL when the provider is missing or has failed, which is the signal
 * for the engine to run its CPU kernel (backend/core/llm_quant.c:159-160). */
#include "compute_backend.h"
#include <math.h>
#include <stdint.h>
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

/* backend/core/compute.c:59-72: NULL selects "cpu", which this library does
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
 * Extensions of this library (no slot in the engine's provider table): they
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

/* ---- sampling at temperature > 0 -----------------------------------------
 * The engine's sampler (backend/core/llm_cpu.c:798-935) restated: its random
 * stream, its candidate order and its arithmetic (float logits and
 * probabilities, double masses), so that equal logits give equal tokens. */

/* One draw of the engine's stream (llm_cpu.c:798-808): an xorshift step,
 * the state times a 64-bit odd constant, its top 24 of 32 bits over 2^24. */
static float unit_draw(uint64_t *state)
{
    uint64_t v = *state;
    v ^= v >> 12;
    v ^= v << 25;
    v ^= v >> 27;
    *state = v;
    const uint32_t bits = (uint32_t)((v * UINT64_C(0x2545F4914F6CDD1D)) >> 32);
    return (float)(bits >> 8) / 16777216.0f;
}

typedef struct { float value; unsigned int token; } ranked;

/* Candidate order (llm_cpu.c:811-826): larger value first, then smaller id. */
static int ahead(const ranked *a, const ranked *b)
{
    return a->value > b->value || (a->value == b->value && a->token < b->token);
}

static int ranked_order(const void *l, const void *r)
{
    const ranked *a = l, *b = r;
    return ahead(a, b) ? -1 : ahead(b, a) ? 1 : 0;
}

/* h[0..k) is a heap whose root is the last of its candidates in order. */
static void keep_worst_on_top(ranked *h, size_t k, size_t i)
{
    for (;;) {
        size_t c = 2 * i + 1;
        if (c >= k) return;
        if (c + 1 < k && ahead(&h[c], &h[c + 1])) ++c;   /* the later child */
        if (ahead(&h[c], &h[i])) return;
        const ranked t = h[i];
        h[i] = h[c];
        h[c] = t;
        i = c;
    }
}

/* The sampling distribution (llm_cpu.c:847-888): the first top_k candidates
 * in order, exp((l - max) / T) each, cut after the shortest prefix holding
 * top_p of their mass, normalized; written densely over logits (zero
 * elsewhere) and, in order, to cand[0..*count). */
static int distribution(float *logits, size_t n, float temperature, float top_p, size_t top_k, ranked *cand,
    size_t *count)
{
    size_t kept = top_k == 0 || top_k > n ? n : top_k;
    if (!n || !(temperature > 0.0f)) return -1;
    for (size_t j = 0; j < n; ++j)
        if (isnan(logits[j]) || logits[j] == INFINITY) return -1;
    for (size_t j = 0; j < kept; ++j) cand[j] = (ranked){logits[j], (unsigned int)j};
    if (kept < n) {
        for (size_t j = kept / 2; j-- > 0;) keep_worst_on_top(cand, kept, j);
        for (size_t j = kept; j < n; ++j) {
            const ranked c = {logits[j], (unsigned int)j};
            if (ahead(&c, &cand[0])) {
                cand[0] = c;
                keep_worst_on_top(cand, kept, 0);
            }
        }
    }
    qsort(cand, kept, sizeof(*cand), ranked_order);
    const float top = cand[0].value;
    if (!isfinite(top)) return -1;
    double mass = 0.0, prefix = 0.0;
    for (size_t j = 0; j < kept; ++j) {
        cand[j].value = expf((cand[j].value - top) / temperature);
        mass += cand[j].value;
    }
    for (size_t j = 0; j < kept; ++j) {
        prefix += cand[j].value;
        if (prefix >= (double)top_p * mass) {
            kept = j + 1;
            break;
        }
    }
    if (!(prefix > 0.0) || !isfinite(prefix)) return -1;
    memset(logits, 0, n * sizeof(*logits));
    for (size_t j = 0; j < kept; ++j) {
        cand[j].value = (float)((double)cand[j].value / prefix);
        logits[cand[j].token] = cand[j].value;
    }
    *count = kept;
    return 0;
}

/* One token from the distribution of `logits` (llm_cpu.c:890-911), which it
 * leaves in place of the logits. */
static int sample_token(float *logits, size_t n, const nya_compute_sampling *s, uint64_t *rng, ranked *cand,
    unsigned int *token)
{
    size_t count;
    if (distribution(logits, n, s->temperature, s->top_p, s->top_k, cand, &count)) return -1;
    const double target = unit_draw(rng);
    double cdf = 0.0;
    for (size_t j = 0; j < count; ++j) {
        cdf += cand[j].value;
        if (target < cdf) {
            *token = cand[j].token;
            return 0;
        }
    }
    *token = cand[count - 1].token;
    return 0;
}

/* One token from a dense nonnegative vector (llm_cpu.c:915-932): the CDF in
 * double, falling back to the last positive entry. */
static int draw_dense(const float *w, size_t n, uint64_t *rng, unsigned int *token)
{
    double mass = 0.0, cdf = 0.0;
    size_t last = 0;
    for (size_t j = 0; j < n; ++j) {
        if (w[j] < 0.0f || !isfinite(w[j])) return -1;
        mass += w[j];
        if (w[j] > 0.0f) last = j;
    }
    if (!(mass > 0.0)) return -1;
    const double target = (double)unit_draw(rng) * mass;
    for (size_t j = 0; j < n; ++j) {
        cdf += w[j];
        if (target < cdf) {
            *token = (unsigned int)j;
            return 0;
        }
    }
    *token = (unsigned int)last;
    return 0;
}

/* The engine's speculative sampling loop (llm_cpu.c:1215-1317, ordinary
 * draft) over batched verification; state between rounds as in
 * nya_compute_generate_greedy. A round: the draft catches up to P and samples
 * p_0..p_{m-1} (its distributions kept as q_0..q_{m-1}), the target verifies
 * [pending, p_0, .., p_{m-1}] at P, and row j of the result is the target's
 * logits after pending and p_0..p_{j-1}: the engine's target step j. */
int nya_compute_generate_sampled(nya_compute_plan *target, nya_compute_plan *draft,
    const unsigned int *prompt, size_t prompt_count, size_t window, size_t limit,
    const nya_compute_sampling *sampling, const unsigned int *stops, size_t stop_count,
    unsigned int *out, size_t *out_count, nya_compute_speculation *stats)
{
    nya_compute_speculation st;
    memset(&st, 0, sizeof(st));
    if (out_count) *out_count = 0;
    if (stats) *stats = st;
    if (!sampling) return -1;
    const nya_compute_sampling s = *sampling;
    /* The engine's request bounds (llm_cpu.c:1174-1177). */
    if (!isfinite(s.temperature) || s.temperature < 0.0f || s.temperature > 5.0f || !isfinite(s.top_p) ||
        s.top_p <= 0.0f || s.top_p > 1.0f)
        return -1;
    if (s.temperature == 0.0f)
        return nya_compute_generate_greedy(target, draft, prompt, prompt_count, window, limit, stops, stop_count, out,
                                           out_count, stats);
    const size_t vocabulary = rocm_plan(target) ? nya_rocm_plan_vocabulary(target->state) : 0;
    const size_t verify = nya_compute_plan_verify_limit(target);
    if (!vocabulary || !prompt || !prompt_count || !out || !out_count || !limit || window > 32 ||
        (stop_count && !stops) || prompt_count > SIZE_MAX / 8 || limit > SIZE_MAX / 8 ||
        vocabulary > SIZE_MAX / sizeof(float) / 40)
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
    float *rows = malloc((window + 1) * vocabulary * sizeof(float));     /* the target's rows of a round */
    float *qs = malloc((window ? window : 1) * vocabulary * sizeof(float)); /* the draft's distributions */
    ranked *cand = malloc(vocabulary * sizeof(*cand));
    int result = -1;
    if (!seq || !rows || !qs || !cand) goto done;
    /* The engine's two streams (llm_cpu.c:1229-1232). */
    uint64_t rng = s.seed ? s.seed : UINT64_C(0x9E3779B97F4A7C15);
    uint64_t draft_rng = rng ^ UINT64_C(0xD1B54A32D192ED03);
    if (!draft_rng) draft_rng = 1;
    memcpy(seq, prompt, prompt_count * sizeof(*seq));
    size_t P = prompt_count - 1, draft_valid = 0, generated = 0;
    if (P > 0) {
        if (catch_up(target, seq, 0, P, rows)) goto done;
        st.target_tokens += P;
        if (window) {
            if (catch_up(draft, seq, 0, P, rows)) goto done;
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
                if (catch_up(draft, seq, draft_valid, P, rows)) goto done;
                ++st.draft_steps;
            }
            for (size_t i = 0; i < m; ++i) {
                float *q = qs + i * vocabulary;
                unsigned int next;
                if (nya_compute_plan_verify(draft, &batch[i], 1, P + i, ids, q)) goto done;
                ++st.draft_steps;
                if (sample_token(q, vocabulary, &s, &draft_rng, cand, &next)) goto done;
                ++st.draft_tokens;
                batch[i + 1] = next;
                if (is_stop(next, stops, stop_count)) { m = i + 1; break; }
            }
            draft_valid = P + m;
        }
        if (nya_compute_plan_verify(target, batch, m + 1, P, ids, rows)) goto done;
        ++st.rounds;
        st.target_tokens += m + 1;
        size_t emitted = 0;
        int rejected = 0;
        for (size_t j = 0; j < m && !stopped; ++j) {
            float *p = rows + j * vocabulary;
            const float *q = qs + j * vocabulary;
            unsigned int token = batch[j + 1];
            size_t count;
            if (distribution(p, vocabulary, s.temperature, s.top_p, s.top_k, cand, &count)) goto done;
            if (!(q[token] > 0.0f)) goto done;
            /* Accept x ~ q with probability min(1, p(x) / q(x)) (llm_cpu.c:1282-1290). */
            const int accepted = (double)unit_draw(&rng) * q[token] < p[token];
            if (!accepted) {
                for (size_t v = 0; v < vocabulary; ++v) p[v] = fmaxf(p[v] - q[v], 0.0f);
                if (draw_dense(p, vocabulary, &rng, &token)) goto done;
            } else {
                ++st.accepted;
            }
            out[generated++] = token;
            seq[P + 1 + emitted++] = token;
            if (is_stop(token, stops, stop_count)) stopped = 1;
            if (!accepted) { rejected = 1; break; }
        }
        /* After every proposal the target's next row gives one more token. */
        if (!rejected && !stopped && generated < limit) {
            unsigned int token;
            if (sample_token(rows + m * vocabulary, vocabulary, &s, &rng, cand, &token)) goto done;
            out[generated++] = token;
            seq[P + 1 + emitted++] = token;
            if (is_stop(token, stops, stop_count)) stopped = 1;
        }
        P += emitted;
        if (draft_valid > P) draft_valid = P;
    }
    st.generated = generated;
    *out_count = generated;
    result = 0;
done:
    if (stats) *stats = st;
    free(seq);
    free(rows);
    free(qs);
    free(cand);
    return result;
}
