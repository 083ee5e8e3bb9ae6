/* ctypes-facing shim around the reference C runtime (runtime/vault3.h API).
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile into oracle/_ref/libv3ref.so as one
 * translation unit with the reference's runtime/vault3.c (included from the reference tree); never
 * linked into the product.
 *
 * Provides: an aligned model buffer + v3_load (runtime/vault3.c:273-455), a state arena +
 * v3_state_init (:828-852), v3_step (:2034-2222), v3_set_pinned (:898-928), an optional persistent
 * thread pool implementing the v3_parallel_for_fn hook (runtime/vault3.h:103-106), a helper that
 * seeds the fixed-size state as it stands deep into a long stream (for timing at long context), and
 * read access to the resonance state and the model for the governor (runtime/vault3.h:180-216), and
 * direct calls of the static resonance / quarantine functions on constructed banks and rings.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* The runtime's translation unit itself, so that the shim can also reach the static resonance and
 * quarantine functions (runtime/vault3.c:1178-1831) for direct tests on constructed states. */
#include "vault3.c"

typedef struct pool pool_t;

typedef struct {
    v3_model m;
    v3_state s;
    uint8_t *buf;
    void *arena;
    size_t arena_size;
    pool_t *pool;
} ref_ctx;

/* ---------------------------------------------------------------- thread pool ---------------- */

struct pool {
    int n;
    pthread_t *th;
    pthread_mutex_t mu;
    pthread_cond_t cv_go, cv_done;
    uint64_t gen;
    int pending;
    int quit;
    v3_task_fn fn;
    void *arg;
    uint32_t total;
};

typedef struct {
    pool_t *p;
    int idx;
} worker_arg;

static void run_share(pool_t *p, int idx) {
    uint32_t per = (p->total + (uint32_t)p->n - 1u) / (uint32_t)p->n;
    uint32_t i0 = (uint32_t)idx * per, i1 = i0 + per;
    if (i1 > p->total) i1 = p->total;
    if (i0 < i1) p->fn(p->arg, i0, i1);
}

static void *worker(void *a) {
    worker_arg *wa = (worker_arg *)a;
    pool_t *p = wa->p;
    int idx = wa->idx;
    free(wa);
    uint64_t seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (!p->quit && p->gen == seen) pthread_cond_wait(&p->cv_go, &p->mu);
        if (p->quit) {
            pthread_mutex_unlock(&p->mu);
            return 0;
        }
        seen = p->gen;
        pthread_mutex_unlock(&p->mu);
        run_share(p, idx);
        pthread_mutex_lock(&p->mu);
        if (--p->pending == 0) pthread_cond_signal(&p->cv_done);
        pthread_mutex_unlock(&p->mu);
    }
}

static void pool_for(void *ctx, v3_task_fn fn, void *arg, uint32_t n) {
    pool_t *p = (pool_t *)ctx;
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->arg = arg;
    p->total = n;
    p->pending = p->n - 1;
    p->gen++;
    pthread_cond_broadcast(&p->cv_go);
    pthread_mutex_unlock(&p->mu);
    run_share(p, 0);
    pthread_mutex_lock(&p->mu);
    while (p->pending > 0) pthread_cond_wait(&p->cv_done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

static void pool_free(pool_t *p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->cv_go);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->n - 1; i++) pthread_join(p->th[i], 0);
    free(p->th);
    free(p);
}

static pool_t *pool_new(int n) {
    pool_t *p = (pool_t *)calloc(1, sizeof(pool_t));
    p->n = n;
    pthread_mutex_init(&p->mu, 0);
    pthread_cond_init(&p->cv_go, 0);
    pthread_cond_init(&p->cv_done, 0);
    p->th = (pthread_t *)calloc((size_t)n, sizeof(pthread_t));
    for (int i = 1; i < n; i++) {
        worker_arg *wa = (worker_arg *)malloc(sizeof(worker_arg));
        wa->p = p;
        wa->idx = i;
        pthread_create(&p->th[i - 1], 0, worker, wa);
    }
    return p;
}

/* ---------------------------------------------------------------- API -------------------------- */

ref_ctx *ref_open(const uint8_t *data, uint64_t size, int verify, int *err) {
    ref_ctx *c = (ref_ctx *)calloc(1, sizeof(ref_ctx));
    c->buf = (uint8_t *)aligned_alloc(64, (size + 63) & ~(uint64_t)63);
    memcpy(c->buf, data, size);
    int rc = v3_load(&c->m, c->buf, size, verify);
    if (rc != V3_OK) {
        *err = rc;
        free(c->buf);
        free(c);
        return 0;
    }
    c->arena_size = v3_state_arena_size(&c->m);
    c->arena = aligned_alloc(64, (c->arena_size + 63) & ~(size_t)63);
    rc = v3_state_init(&c->s, &c->m, c->arena, c->arena_size);
    if (rc != V3_OK) {
        *err = rc;
        free(c->arena);
        free(c->buf);
        free(c);
        return 0;
    }
    *err = 0;
    return c;
}

int ref_set_threads(ref_ctx *c, int n) {
    pool_free(c->pool);
    c->pool = 0;
    c->s.par_for = 0;
    c->s.par_ctx = 0;
    if (n > 1) {
        c->pool = pool_new(n);
        c->s.par_for = pool_for;
        c->s.par_ctx = c->pool;
    }
    return 0;
}

void ref_close(ref_ctx *c) {
    if (!c) return;
    pool_free(c->pool);
    free(c->arena);
    free(c->buf);
    free(c);
}

void ref_reset(ref_ctx *c) { v3_state_reset(&c->s); }

int ref_set_pinned(ref_ctx *c, uint32_t n) { return v3_set_pinned(&c->s, n); }

uint64_t ref_arena_bytes(ref_ctx *c) { return (uint64_t)c->arena_size; }

uint32_t ref_vocab(ref_ctx *c) { return c->m.vocab_size; }

int ref_step(ref_ctx *c, uint32_t tok, float *out) {
    const float *lg = v3_step(&c->s, tok);
    if (out) memcpy(out, lg, sizeof(float) * c->m.vocab_size);
    return 0;
}

/* Host-visible scalar state for cross-checks. */
void ref_state_info(ref_ctx *c, uint64_t *pos, uint32_t *n_pin, uint32_t *mem_cnt, uint32_t *seg_id_offset) {
    *pos = c->s.pos;
    *n_pin = c->s.n_pin;
    *mem_cnt = c->s.mem_cnt;
    *seg_id_offset = c->s.seg_id_offset;
}

/* Flags of the auto-pin and resonance machinery: pin_locked, seg_bias_active, n_uniq_segs. */
void ref_state_flags(ref_ctx *c, int *pin_locked, int *seg_bias_active, uint32_t *n_uniq_segs) {
    *pin_locked = c->s.pin_locked;
    *seg_bias_active = c->s.seg_bias_active;
    *n_uniq_segs = c->s.n_uniq_segs;
}

/* Set the segment budget of the state (v3_set_seg_budget, runtime/vault3.h:158-159). */
int ref_set_seg_budget(ref_ctx *c, uint32_t budget) { return v3_set_seg_budget(&c->s, budget); }

void ref_mem_pos(ref_ctx *c, uint64_t *out) {
    for (uint32_t i = 0; i < c->s.mem_cnt; i++) out[i] = c->s.mem_pos[i];
}

/* The bank's tokens and segment ids and the resonance biases over its mem_cnt slots (the values
 * v3_step computed for its last step; hop1 meaningful when seg_bias_active == 2). */
void ref_res_state(ref_ctx *c, uint32_t *mem_tok, uint32_t *mem_seg, float *arch, float *sup, float *hop1) {
    for (uint32_t i = 0; i < c->s.mem_cnt; i++) {
        mem_tok[i] = c->s.mem_tok[i];
        mem_seg[i] = c->s.mem_seg[i];
        arch[i] = c->s.seg_bias_arch[i];
        sup[i] = c->s.seg_bias_sup[i];
        hop1[i] = c->s.seg_bias_hop1[i];
    }
}

/* The token rings (W slots each) and the current chunk's segment scores. */
void ref_rings(ref_ctx *c, uint32_t *tok_prev, uint32_t *tok_cur, float *sc_cur) {
    uint32_t W = c->m.window;
    for (uint32_t i = 0; i < W; i++) {
        tok_prev[i] = c->s.tok_prev[i];
        tok_cur[i] = c->s.tok_cur[i];
        sc_cur[i] = c->s.sc_cur ? c->s.sc_cur[i] : 0.0f;
    }
}

/* The loaded model (for the governor entry points, runtime/vault3.h:211-216) and the governor's size. */
const v3_model *ref_model(ref_ctx *c) { return &c->m; }
uint64_t ref_gov_size(void) { return (uint64_t)sizeof(v3_governor); }

/* Copy one layer's KV field out of the state, as [G][rows][D] floats (rows = W for the window
 * fields 0-5, sink_cap for the sink fields 6-8, seg_cap for the segment fields 9-11; field order
 * k_prev k_cur v_prev v_cur kraw_prev kraw_cur k_sink_raw k_sink v_sink k_seg_raw k_seg v_seg).
 * Returns the number of rows, or -1. */
int64_t ref_state_field(ref_ctx *c, uint32_t layer, uint32_t field, float *out) {
    const v3_state *s = &c->s;
    const v3_model *m = &c->m;
    if (layer >= m->n_layers || field > 11) return -1;
    const v3_layer_state *L = &s->ls[layer];
    const float *src[12] = {L->k_prev, L->k_cur, L->v_prev, L->v_cur, L->kraw_prev, L->kraw_cur,
                            L->k_sink_raw, L->k_sink, L->v_sink, L->k_seg_raw, L->k_seg, L->v_seg};
    uint64_t rows = field < 6 ? m->window : field < 9 ? s->sink_cap : s->seg_cap;
    if (!src[field]) return rows ? -1 : 0;
    if (out) memcpy(out, src[field], sizeof(float) * m->n_kv_heads * rows * m->head_dim);
    return (int64_t)rows;
}

static uint64_t splitmix(uint64_t *x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void fill(float *p, uint64_t n, uint64_t *rng) {
    for (uint64_t i = 0; i < n; i++) {
        /* sum of the four 16-bit uniforms of one draw, centred and scaled to unit variance */
        const uint64_t z = splitmix(rng);
        double s = 0.0;
        for (int k = 0; k < 4; k++) s += ((double)((z >> (16 * k)) & 0xFFFFu) + 0.5) * (1.0 / 65536.0);
        p[i] = (float)((s - 2.0) * 1.7320508075688772);
    }
}

/* Put the state where a long stream leaves it: position `pos` (chunk index >= 2), `n_pin` sinks
 * locked, `mem_cnt` occupied segment-memory slots, every KV row filled with unit-variance values.
 * Steps taken from here stay inside the current chunk while pos % W < W - 1. */
int ref_seed_long_context(ref_ctx *c, uint64_t pos, uint32_t n_pin, uint32_t mem_cnt, uint64_t seed) {
    v3_state *s = &c->s;
    const v3_model *m = &c->m;
    uint64_t W = m->window, G = m->n_kv_heads, D = m->head_dim;
    if (pos < 2 * W || n_pin > s->sink_cap || mem_cnt > s->seg_budget) return -1;
    uint64_t rng = seed;
    for (uint32_t l = 0; l < m->n_layers; l++) {
        v3_layer_state *L = &s->ls[l];
        fill(L->k_prev, G * W * D, &rng); fill(L->k_cur, G * W * D, &rng);
        fill(L->v_prev, G * W * D, &rng); fill(L->v_cur, G * W * D, &rng);
        fill(L->kraw_prev, G * W * D, &rng); fill(L->kraw_cur, G * W * D, &rng);
        fill(L->k_sink_raw, G * s->sink_cap * D, &rng); fill(L->k_sink, G * s->sink_cap * D, &rng);
        fill(L->v_sink, G * s->sink_cap * D, &rng);
        if (s->seg_cap) {
            fill(L->k_seg_raw, G * s->seg_cap * D, &rng); fill(L->k_seg, G * s->seg_cap * D, &rng);
            fill(L->v_seg, G * s->seg_cap * D, &rng);
        }
    }
    s->pos = pos;
    s->n_pin = n_pin;
    s->pin_locked = 1;
    s->mem_cnt = mem_cnt;
    for (uint32_t i = 0; i < mem_cnt; i++) {
        s->mem_pos[i] = (uint64_t)i * 8u;
        s->mem_score[i] = 0.0f;
        s->mem_tok[i] = 0;
        s->mem_seg[i] = i / 16u;
    }
    s->n_uniq_segs = 0;   /* no shingles: resonance stays inactive */
    s->ema_ready = 1;
    return 0;
}

/* ---------------------------------------------------------------- direct resonance calls -------- */

/* Load a bank (mem_cnt <= seg_cap slots of tokens and segment ids) into the state and rebuild the
 * shingle index (rebuild_shingle_index, runtime/vault3.c:1178-1260); returns n_uniq_segs, or -1. */
int ref_res_load_bank(ref_ctx *c, const uint32_t *mem_tok, const uint32_t *mem_seg, uint32_t mem_cnt) {
    v3_state *s = &c->s;
    if (mem_cnt > s->seg_cap) return -1;
    for (uint32_t i = 0; i < mem_cnt; i++) {
        s->mem_tok[i] = mem_tok[i];
        s->mem_seg[i] = mem_seg[i];
        s->mem_pos[i] = i;
        s->mem_score[i] = 0.0f;
    }
    s->mem_cnt = mem_cnt;
    rebuild_shingle_index(s);
    return (int)s->n_uniq_segs;
}

/* One update_query_resonance (runtime/vault3.c:1426-1786) on given token rings (W slots each), ring
 * slot c, position and pin count over the loaded bank; returns seg_bias_active and copies the three
 * bias vectors (mem_cnt slots). */
int ref_res_update(ref_ctx *c, const uint32_t *tok_prev, const uint32_t *tok_cur, uint32_t ci, uint64_t pos,
                   uint32_t n_pin, float *arch, float *sup, float *hop1) {
    v3_state *s = &c->s;
    uint32_t W = c->m.window;
    for (uint32_t i = 0; i < W; i++) {
        s->tok_prev[i] = tok_prev[i];
        s->tok_cur[i] = tok_cur[i];
    }
    s->pos = pos;
    s->n_pin = n_pin;
    update_query_resonance(s, ci);
    for (uint32_t i = 0; i < s->mem_cnt; i++) {
        arch[i] = s->seg_bias_arch[i];
        sup[i] = s->seg_bias_sup[i];
        hop1[i] = s->seg_bias_hop1[i];
    }
    return s->seg_bias_active;
}

/* check_spoof_quarantine (runtime/vault3.c:1798-1831) on given rings. */
int ref_spoof(ref_ctx *c, const uint32_t *tok_prev, const uint32_t *tok_cur, uint32_t ci, uint64_t pos, uint32_t n_pin) {
    v3_state *s = &c->s;
    uint32_t W = c->m.window;
    for (uint32_t i = 0; i < W; i++) {
        s->tok_prev[i] = tok_prev[i];
        s->tok_cur[i] = tok_cur[i];
    }
    s->n_pin = n_pin;
    return check_spoof_quarantine(s, pos, ci);
}

/* The runtime's own v3_expf (fn 0), v3_erff (fn 1) and v3_geluf (fn 2) (runtime/vault3.c:104-129),
 * element-wise. */
void ref_math(int fn, const float *x, float *y, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) y[i] = fn == 0 ? v3_expf(x[i]) : fn == 1 ? v3_erff(x[i]) : v3_geluf(x[i]);
}

/* One update_segment_bank (runtime/vault3.c:1833-1915) on given evicted-chunk rings (W slots: scores,
 * local segment ids, tokens) and a given bank of mem_cnt slots, with the segment budget, pin count
 * and seg-id offset set first.  Returns the new mem_cnt (or -1 if the budget exceeds the state's
 * capacity) and copies the new bank and seg-id offset out.  The quarantine that v3_step applies before
 * the call (:2079-2088) is not part of this function: callers pass scores it leaves unchanged. */
int ref_seg_update(ref_ctx *c, uint64_t ev_chunk_idx, uint32_t n_pin, uint32_t seg_id_offset, uint32_t budget,
                   const float *sc_prev, const uint32_t *seg_prev, const uint32_t *tok_prev, uint32_t mem_cnt,
                   const uint64_t *mem_pos, const float *mem_score, const uint32_t *mem_tok, const uint32_t *mem_seg,
                   uint64_t *o_pos, float *o_score, uint32_t *o_tok, uint32_t *o_seg, uint32_t *o_offset) {
    v3_state *s = &c->s;
    uint32_t W = c->m.window;
    if (budget > s->seg_cap || mem_cnt > budget) return -1;
    s->seg_budget = budget;
    s->n_pin = n_pin;
    s->seg_id_offset = seg_id_offset;
    for (uint32_t t = 0; t < W; t++) {
        s->sc_prev[t] = sc_prev[t];
        s->seg_prev[t] = seg_prev[t];
        s->tok_prev[t] = tok_prev[t];
    }
    for (uint32_t i = 0; i < mem_cnt; i++) {
        s->mem_pos[i] = mem_pos[i];
        s->mem_score[i] = mem_score[i];
        s->mem_tok[i] = mem_tok[i];
        s->mem_seg[i] = mem_seg[i];
    }
    s->mem_cnt = mem_cnt;
    update_segment_bank(s, ev_chunk_idx);
    for (uint32_t i = 0; i < s->mem_cnt; i++) {
        o_pos[i] = s->mem_pos[i];
        o_score[i] = s->mem_score[i];
        o_tok[i] = s->mem_tok[i];
        o_seg[i] = s->mem_seg[i];
    }
    *o_offset = s->seg_id_offset;
    return (int)s->mem_cnt;
}
