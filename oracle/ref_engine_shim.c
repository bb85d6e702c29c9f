/* ref_engine_shim: drives the reference engine (compiled from its own
 * sources into oracle/_ref by oracle/Makefile, target `engine`) next to
 * this repository's batched prefill (siphon_amd/host/si_prefill.c) and
 * "hip" backend adapter, for tests/test_prefill.py. TEST INFRASTRUCTURE
 * ONLY; never shipped in the product.
 *
 * It is compiled with the reference's headers; the prefill and the adapter
 * are compiled against this repository's mirror of them (si_mirror.h,
 * si_engine_mirror.h), and the tests check that every field offset agrees
 * (re_layout here, re_mirror_layout in ref_engine_layout.c). The mirror's
 * si_backend has one more slot than the reference's, `gemm`, after
 * row_to_f32: backends given to the prefill here are declared with it
 * (with_gemm below); the reference CPU backend itself, which lacks it, is
 * only reached through gemv and row_to_f32.
 */
#include <stddef.h>

#include "siphon/engine.h"
#include "siphon/kernels.h"
#include "siphon/model.h"

/* the repository's prefill and adapter, declared with the reference's
 * types (same layouts) */
const float *si_engine_prefill(si_engine *e, const uint32_t *tokens, int64_t n);
int si_backend_hip_open(const char *lib_path, int device, si_backend **out);
void si_backend_hip_close(si_backend *be);
int si_backend_hip_place(si_backend *be, si_tensor *w);

typedef int (*gemm_fn)(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y,
                       si_tp *tp);

/* a reference si_backend followed by the gemm slot: the mirror's layout */
typedef struct {
    si_backend base;
    gemm_fn gemm;
} with_gemm;

/* ---- the reference CPU backend with the gemm slot the integration adds:
 * one reference gemv per row (the cpu_gemm fill of backend.c) ---------- */

static void cpu_gemv_fwd(si_backend *be, const si_tensor *w, const float *x, float *y,
                         int64_t n_out, si_tp *tp) {
    (void)be;
    si_backend *cpu = si_backend_cpu();
    cpu->gemv(cpu, w, x, y, n_out, tp);
}

static void cpu_row_fwd(si_backend *be, const si_tensor *w, uint64_t row, float *out) {
    (void)be;
    si_backend *cpu = si_backend_cpu();
    cpu->row_to_f32(cpu, w, row, out);
}

static int cpu_gemm_rows(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y,
                         si_tp *tp) {
    (void)be;
    si_backend *cpu = si_backend_cpu();
    const int64_t n_in = (int64_t)w->ne[0], n_out = (int64_t)w->ne[1];
    for (int64_t m = 0; m < M; m++) cpu->gemv(cpu, w, X + m * n_in, Y + m * n_out, n_out, tp);
    return SI_OK;
}

static with_gemm g_cpu_gemm = {{"cpu", SI_LOC_HOST, cpu_gemv_fwd, cpu_row_fwd}, cpu_gemm_rows};
/* the same with an empty gemm slot: the prefill makes one gemv per row */
static with_gemm g_cpu_nogemm = {{"cpu", SI_LOC_HOST, cpu_gemv_fwd, cpu_row_fwd}, NULL};

/* ---- a recorder in front of a backend's gemm: every call's operands and
 * result are kept for the tests to check against the oracle ----------- */

#define REC_MAX 256
typedef struct {
    const void *data;
    uint32_t type;
    int64_t n_in, n_out, M;
    float *X, *Y;
} rec_call;

static with_gemm *g_rec_inner;
static rec_call g_rec[REC_MAX];
static int g_nrec;

static void rec_gemv(si_backend *be, const si_tensor *w, const float *x, float *y, int64_t n_out,
                     si_tp *tp) {
    (void)be;
    g_rec_inner->base.gemv(&g_rec_inner->base, w, x, y, n_out, tp);
}

static void rec_row(si_backend *be, const si_tensor *w, uint64_t row, float *out) {
    (void)be;
    g_rec_inner->base.row_to_f32(&g_rec_inner->base, w, row, out);
}

static int rec_gemm(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y,
                    si_tp *tp) {
    (void)be;
    const int rc = g_rec_inner->gemm(&g_rec_inner->base, w, X, M, Y, tp);
    if (rc == SI_OK && g_nrec < REC_MAX) {
        rec_call *c = &g_rec[g_nrec++];
        c->data = w->data;
        c->type = w->type;
        c->n_in = (int64_t)w->ne[0];
        c->n_out = (int64_t)w->ne[1];
        c->M = M;
        c->X = si_xmalloc(sizeof(float) * (size_t)(M * c->n_in));
        c->Y = si_xmalloc(sizeof(float) * (size_t)(M * c->n_out));
        memcpy(c->X, X, sizeof(float) * (size_t)(M * c->n_in));
        memcpy(c->Y, Y, sizeof(float) * (size_t)(M * c->n_out));
    }
    return rc;
}

static with_gemm g_recorder = {{"rec", SI_LOC_HOST, rec_gemv, rec_row}, rec_gemm};

/* ---- entry points for ctypes ------------------------------------------ */

const char *re_errstr(void) { return si_errstr(); }

void *re_model_load(const char *path) {
    si_kern_init();
    si_model *m = NULL;
    return si_model_load(path, &m) == SI_OK ? m : NULL;
}

void re_model_free(void *m) { si_model_free(m); }

void *re_engine_create(void *m, int64_t n_ctx, int threads) {
    si_engine *e = NULL;
    return si_engine_create(m, n_ctx, threads, &e) == SI_OK ? e : NULL;
}

void re_engine_free(void *e) { si_engine_free(e); }
void re_engine_reset(void *e) { si_engine_reset(e); }
int64_t re_n_pos(const void *e) { return ((const si_engine *)e)->n_pos; }

/* n_layer, n_head, n_head_kv, head_dim, n_ctx, n_vocab, n_embd, n_ff, arch */
void re_dims(const void *ep, int64_t *out) {
    const si_engine *e = ep;
    const si_hparams *h = &e->m->h;
    out[0] = h->n_layer;
    out[1] = h->n_head;
    out[2] = h->n_head_kv;
    out[3] = h->head_dim;
    out[4] = e->n_ctx;
    out[5] = h->n_vocab;
    out[6] = h->n_embd;
    out[7] = (int64_t)h->n_ff;
    out[8] = e->m->arch;
}

const uint16_t *re_k_cache(const void *e) { return ((const si_engine *)e)->k_cache; }
const uint16_t *re_v_cache(const void *e) { return ((const si_engine *)e)->v_cache; }

/* the token loop: one si_engine_forward per token (cmd_run.c:275-283) */
const float *re_forward_loop(void *e, const uint32_t *tokens, int64_t n) {
    const float *lg = NULL;
    for (int64_t i = 0; i < n; i++)
        if (!(lg = si_engine_forward(e, tokens[i]))) return NULL;
    return lg;
}

const float *re_prefill(void *e, const uint32_t *tokens, int64_t n) {
    return si_engine_prefill(e, tokens, n);
}

/* every layer on the reference CPU backend (the loader's choice) */
void re_layers_cpu(void *mp) {
    si_model *m = mp;
    for (uint32_t il = 0; il < m->h.n_layer; il++) m->layer_be[il] = si_backend_cpu();
}

/* every layer on the reference CPU backend with the gemm slot */
void re_layers_cpu_gemm(void *mp) {
    si_model *m = mp;
    for (uint32_t il = 0; il < m->h.n_layer; il++) m->layer_be[il] = &g_cpu_gemm.base;
}

/* every layer on the reference CPU backend with an empty gemm slot */
void re_layers_cpu_nogemm(void *mp) {
    si_model *m = mp;
    for (uint32_t il = 0; il < m->h.n_layer; il++) m->layer_be[il] = &g_cpu_nogemm.base;
}

int re_hip_open(const char *lib, void **be) {
    si_backend *b = NULL;
    const int rc = si_backend_hip_open(lib, 0, &b);
    *be = b;
    return rc;
}

void re_hip_close(void *be) { si_backend_hip_close(be); }

/* Every layer's seven matrices placed on the hip backend (loader hook,
 * si_backend_hip_place) and the layer assigned to it; the head too when
 * `head` is set. With `record`, the layers go through the recorder. */
int re_layers_hip(void *mp, void *be, int head, int record) {
    si_model *m = mp;
    for (uint32_t il = 0; il < m->h.n_layer; il++) {
        si_layer *l = &m->layers[il];
        si_tensor *ts[] = {&l->wq, &l->wk, &l->wv, &l->wo, &l->w_gate, &l->w_up, &l->w_down};
        for (size_t i = 0; i < sizeof ts / sizeof ts[0]; i++) {
            const int rc = si_backend_hip_place(be, ts[i]);
            if (rc) return rc;
        }
        m->layer_be[il] = record ? &g_recorder.base : (si_backend *)be;
    }
    g_rec_inner = be;
    if (head) return si_backend_hip_place(be, &m->output);
    return SI_OK;
}

int re_rec_count(void) { return g_nrec; }

/* call i: weight bytes, type, n_in, n_out, M, X, Y */
void re_rec_get(int i, const void **data, int64_t *meta, const float **X, const float **Y) {
    const rec_call *c = &g_rec[i];
    *data = c->data;
    meta[0] = c->type;
    meta[1] = c->n_in;
    meta[2] = c->n_out;
    meta[3] = c->M;
    *X = c->X;
    *Y = c->Y;
}

void re_rec_clear(void) {
    for (int i = 0; i < g_nrec; i++) {
        free(g_rec[i].X);
        free(g_rec[i].Y);
    }
    g_nrec = 0;
}

/* Sizes and field offsets of the reference's structs, in the order of
 * re_mirror_layout (ref_engine_layout.c). Returns the count. */
#define OFF(T, f) (int64_t) offsetof(T, f)
int re_layout(int64_t *o) {
    int n = 0;
    o[n++] = sizeof(si_tensor);
    o[n++] = sizeof(si_backend);
    o[n++] = OFF(si_backend, row_to_f32);
    o[n++] = sizeof(si_hparams);
    o[n++] = OFF(si_hparams, n_ctx_train);
    o[n++] = OFF(si_hparams, n_ff);
    o[n++] = OFF(si_hparams, rms_eps);
    o[n++] = OFF(si_hparams, head_dim);
    o[n++] = OFF(si_hparams, n_head_gqa);
    o[n++] = sizeof(si_wview);
    o[n++] = sizeof(si_layer);
    o[n++] = OFF(si_layer, w_down);
    o[n++] = OFF(si_layer, attn_norm);
    o[n++] = OFF(si_layer, bv);
    o[n++] = sizeof(si_model);
    o[n++] = OFF(si_model, h);
    o[n++] = OFF(si_model, arch);
    o[n++] = OFF(si_model, tok_embd);
    o[n++] = OFF(si_model, layers);
    o[n++] = OFF(si_model, out_norm);
    o[n++] = OFF(si_model, rope_ffs);
    o[n++] = OFF(si_model, output);
    o[n++] = OFF(si_model, output_tied);
    o[n++] = OFF(si_model, layer_be);
    o[n++] = sizeof(si_engine);
    o[n++] = OFF(si_engine, layer_cb);
    o[n++] = OFF(si_engine, n_ctx);
    o[n++] = OFF(si_engine, n_pos);
    o[n++] = OFF(si_engine, k_cache);
    o[n++] = OFF(si_engine, v_cache);
    o[n++] = OFF(si_engine, xb);
    o[n++] = OFF(si_engine, logits);
    o[n++] = OFF(si_engine, rope_cos);
    o[n++] = OFF(si_engine, rope_sin);
    o[n++] = OFF(si_engine, scores);
    o[n++] = OFF(si_engine, probs);
    o[n++] = OFF(si_engine, q16);
    o[n++] = OFF(si_engine, probs16);
    o[n++] = OFF(si_engine, wscratch);
    o[n++] = OFF(si_engine, rope_ff);
    o[n++] = OFF(si_engine, theta_scale);
    o[n++] = OFF(si_engine, kq_scale);
    o[n++] = sizeof(with_gemm);
    o[n++] = OFF(with_gemm, gemm);
    return n;
}
