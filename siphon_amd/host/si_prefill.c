/* si_prefill: the layer-major prompt pass (see si_prefill.h).
 *
 * Per-row arithmetic follows the reference forward step by step, since the
 * token loop's results are the specification:
 *   rms norm x * scale * w                 engine.c:12-18
 *   norm/bias views (F32 or dequantized)   engine.c:270-282
 *   RoPE angles and rotations              engine.c:26-75
 *   K position-major, V transposed, f16    engine.c:343-357
 *   attention of one query head            engine.c:90-147
 *   SwiGLU                                 engine.c:162-179
 *   residual adds, head                    engine.c:368-398
 * compiled as the reference is (C17, so no contraction of a*b+c; fmaf
 * only where the reference calls it). */
#include "si_prefill.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* host buffers of one pass: `rows` rows of every activation */
typedef struct {
    float *x;      /* residual stream   [rows][n_embd] */
    float *xb;     /* normed input      [rows][n_embd] */
    float *q;      /* queries           [rows][n_embd] */
    float *k, *v;  /* keys, values      [rows][n_kv]   */
    float *att;    /* attention output  [rows][n_embd] */
    float *ff;     /* projection output [rows][n_embd] */
    float *gate;   /* gate, then SwiGLU [rows][n_ff]   */
    float *up;     /*                   [rows][n_ff]   */
} pass_bufs;

/* A norm or bias view as f32: F32 views are read in place; others are
 * dequantized into the engine's scratch, which holds one view at a time
 * (every use below finishes before the next view is materialized). */
static const float *view_f32(si_engine *e, const si_wview *v) {
    if (v->type == SI_T_F32) return (const float *)v->data;
    if (!si_dequant_row(v->type, v->data, e->wscratch, (int)v->n)) {
        si_set_err("norm/bias type %s unsupported", si_quant_name(v->type));
        return NULL;
    }
    return e->wscratch;
}

static int norm_rows(si_engine *e, const si_wview *view, const float *x, float *y,
                     int64_t rows) {
    const int n = (int)e->m->h.n_embd;
    const float *w = view_f32(e, view);
    if (!w) return SI_EFORMAT;
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * n;
        float *yr = y + r * n;
        const float s = si_rms_scale(xr, n, e->m->h.rms_eps);
        for (int i = 0; i < n; i++) yr[i] = xr[i] * s * w[i];
    }
    return SI_OK;
}

static int add_bias(si_engine *e, const si_wview *view, float *y, int64_t rows, int n) {
    if (!view->data) return SI_OK;
    const float *b = view_f32(e, view);
    if (!b) return SI_EFORMAT;
    for (int64_t r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) y[r * n + i] = y[r * n + i] + b[i];
    return SI_OK;
}

/* Y = rows x W^T through the backend's gemm slot, or one gemv per row when
 * it has none. The engine's output widths are the matrices' row counts. */
static int project(si_engine *e, si_backend *be, const si_tensor *w, const float *X, int64_t rows,
                   float *Y, int64_t n_out) {
    if ((int64_t)w->ne[1] != n_out) {
        si_set_err("prefill: a %llu-row matrix where %lld rows are expected",
                   (unsigned long long)w->ne[1], (long long)n_out);
        return SI_EINVAL;
    }
    if (be->gemm) return be->gemm(be, w, X, rows, Y, e->tp);
    const int64_t n_in = (int64_t)w->ne[0];
    for (int64_t r = 0; r < rows; r++) be->gemv(be, w, X + r * n_in, Y + r * n_out, n_out, e->tp);
    return SI_OK;
}

/* cos/sin of every rotated pair at position pos: the angle starts at pos,
 * is divided by the pair's frequency factor when the model has them, and
 * the running angle is multiplied by theta_scale per pair */
static void rope_angles(si_engine *e, int64_t pos) {
    const int pairs = (int)e->m->h.n_rot / 2;
    float theta = (float)pos;
    for (int j = 0; j < pairs; j++) {
        const float a = e->rope_ff ? theta / e->rope_ff[j] : theta;
        e->rope_cos[j] = cosf(a);
        e->rope_sin[j] = sinf(a);
        theta *= e->theta_scale;
    }
}

/* rotate one head in place: adjacent pairs (llama, one fused multiply-add
 * after a rounded product) or pairs half a head apart (qwen2, plain
 * products and sums) */
static void rope_head(const si_engine *e, float *h, int head_dim) {
    const int pairs = (int)e->m->h.n_rot / 2;
    if (e->m->arch == SI_ARCH_LLAMA) {
        for (int j = 0; j < pairs; j++) {
            const float a = h[2 * j], b = h[2 * j + 1];
            const float c = e->rope_cos[j], s = e->rope_sin[j];
            h[2 * j] = fmaf(a, c, -(b * s));
            h[2 * j + 1] = fmaf(a, s, b * c);
        }
        return;
    }
    const int half = head_dim / 2;
    for (int j = 0; j < pairs; j++) {
        const float a = h[j], b = h[j + half];
        const float c = e->rope_cos[j], s = e->rope_sin[j];
        h[j] = a * c - b * s;
        h[j + half] = a * s + b * c;
    }
}

/* one row's attention, query heads split over the lane pool */
typedef struct {
    si_engine *e;
    uint32_t layer;
    int64_t pos;
    const float *q;  /* [n_embd] */
    float *out;      /* [n_embd] */
    si_vec_dot_fn dot;
} row_attn;

static void attend_head(const row_attn *t, int lane, int h) {
    si_engine *e = t->e;
    const si_hparams *hp = &e->m->h;
    const int hd = (int)hp->head_dim;
    const int kvh = h / (int)hp->n_head_gqa;
    const int n = (int)t->pos + 1;
    float *score = e->scores + (size_t)lane * (size_t)e->n_ctx;
    float *prob = e->probs + (size_t)lane * (size_t)e->n_ctx;
    si_f16 *prob16 = e->probs16 + (size_t)lane * (size_t)e->n_ctx;
    const size_t slab = ((size_t)t->layer * hp->n_head_kv + (size_t)kvh) * (size_t)e->n_ctx * hd;
    const si_f16 *keys = e->k_cache + slab;    /* [n_ctx][hd] */
    const si_f16 *vals = e->v_cache + slab;    /* [hd][n_ctx] */
    si_f16 *q16 = e->q16 + (size_t)h * hd;
    for (int d = 0; d < hd; d++) q16[d] = si_f32_to_f16(t->q[(size_t)h * hd + d]);
    for (int j = 0; j < n; j++) t->dot(hd, &score[j], keys + (size_t)j * hd, q16);
    float top = -INFINITY;
    for (int j = 0; j < n; j++) {
        score[j] = score[j] * e->kq_scale;
        if (score[j] > top) top = score[j];
    }
    si_softmax(prob, score, n, top);
    for (int j = 0; j < n; j++) prob16[j] = si_f32_to_f16(prob[j]);
    float *o = t->out + (size_t)h * hd;
    for (int c = 0; c < hd; c++) t->dot(n, &o[c], vals + (size_t)c * e->n_ctx, prob16);
}

static void attend_lane(void *ctx, int lane, int lanes) {
    const row_attn *t = ctx;
    const int heads = (int)t->e->m->h.n_head;
    const int per = (heads + lanes - 1) / lanes;
    const int h1 = (lane + 1) * per < heads ? (lane + 1) * per : heads;
    for (int h = lane * per; h < h1; h++) attend_head(t, lane, h);
}

/* SwiGLU of one row: silu through the polynomial in groups of 8, the
 * remainder through libm's expf, then the product with up */
static void swiglu(float *g, const float *u, int n) {
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = i; k < i + 8; k++) g[k] = si_silu(g[k]) * u[k];
    for (; i < n; i++) g[i] = g[i] / (1.0f + expf(0.0f - g[i])) * u[i];
}

static void add_rows(float *x, const float *d, int64_t count) {
    for (int64_t i = 0; i < count; i++) x[i] = x[i] + d[i];
}

/* One layer-major pass over `rows` tokens at positions pos0.. whose
 * embeddings are in b->x. */
static int run_pass(si_engine *e, pass_bufs *b, int64_t pos0, int64_t rows) {
    si_model *m = e->m;
    const si_hparams *hp = &m->h;
    const int n_embd = (int)hp->n_embd, hd = (int)hp->head_dim;
    const int n_kv = (int)hp->n_head_kv * hd;
    const int64_t n_ff = (int64_t)hp->n_ff;
    const si_vec_dot_fn dot = si_vec_dot_for(SI_T_F16);
    int rc;
    for (uint32_t il = 0; il < hp->n_layer; il++) {
        si_layer *l = &m->layers[il];
        si_backend *be = m->layer_be[il];

        if ((rc = norm_rows(e, &l->attn_norm, b->x, b->xb, rows))) return rc;
        if ((rc = project(e, be, &l->wq, b->xb, rows, b->q, n_embd))) return rc;
        if ((rc = project(e, be, &l->wk, b->xb, rows, b->k, n_kv))) return rc;
        if ((rc = project(e, be, &l->wv, b->xb, rows, b->v, n_kv))) return rc;
        if ((rc = add_bias(e, &l->bq, b->q, rows, n_embd))) return rc;
        if ((rc = add_bias(e, &l->bk, b->k, rows, n_kv))) return rc;
        if ((rc = add_bias(e, &l->bv, b->v, rows, n_kv))) return rc;

        const size_t layer_slab = (size_t)il * hp->n_head_kv * (size_t)e->n_ctx * hd;
        for (int64_t r = 0; r < rows; r++) {
            const int64_t pos = pos0 + r;
            float *q = b->q + r * n_embd, *k = b->k + r * n_kv, *v = b->v + r * n_kv;
            rope_angles(e, pos);
            for (uint32_t h = 0; h < hp->n_head; h++) rope_head(e, q + (size_t)h * hd, hd);
            for (uint32_t h = 0; h < hp->n_head_kv; h++) rope_head(e, k + (size_t)h * hd, hd);
            for (uint32_t h = 0; h < hp->n_head_kv; h++) {
                const size_t head = layer_slab + (size_t)h * (size_t)e->n_ctx * hd;
                si_f16 *kd = e->k_cache + head + (size_t)pos * hd;
                si_f16 *vd = e->v_cache + head + (size_t)pos;
                for (int d = 0; d < hd; d++) {
                    kd[d] = si_f32_to_f16(k[(size_t)h * hd + d]);
                    vd[(size_t)d * e->n_ctx] = si_f32_to_f16(v[(size_t)h * hd + d]);
                }
            }
        }
        for (int64_t r = 0; r < rows; r++) {
            row_attn t = {e, il, pos0 + r, b->q + r * n_embd, b->att + r * n_embd, dot};
            si_tp_run(e->tp, attend_lane, &t);
        }
        if ((rc = project(e, be, &l->wo, b->att, rows, b->ff, n_embd))) return rc;
        add_rows(b->x, b->ff, rows * n_embd);

        if ((rc = norm_rows(e, &l->ffn_norm, b->x, b->xb, rows))) return rc;
        if ((rc = project(e, be, &l->w_gate, b->xb, rows, b->gate, n_ff))) return rc;
        if ((rc = project(e, be, &l->w_up, b->xb, rows, b->up, n_ff))) return rc;
        for (int64_t r = 0; r < rows; r++) swiglu(b->gate + r * n_ff, b->up + r * n_ff, (int)n_ff);
        if ((rc = project(e, be, &l->w_down, b->gate, rows, b->ff, n_embd))) return rc;
        add_rows(b->x, b->ff, rows * n_embd);

        if (e->layer_cb)
            for (int64_t r = 0; r < rows; r++) e->layer_cb(e, (int)il, b->x + r * n_embd);
    }
    return SI_OK;
}

const float *si_engine_prefill(si_engine *e, const uint32_t *tokens, int64_t n) {
    si_model *m = e->m;
    const si_hparams *hp = &m->h;
    if (n < 1 || !tokens) {
        si_set_err("prefill: no tokens");
        return NULL;
    }
    if (e->n_pos + n > e->n_ctx) {
        si_set_err("context full (%lld tokens)", (long long)e->n_ctx);
        return NULL;
    }
    for (int64_t i = 0; i < n; i++)
        if (tokens[i] >= hp->n_vocab) {
            si_set_err("prefill: token %u outside the vocabulary of %u", tokens[i], hp->n_vocab);
            return NULL;
        }
    const int64_t cap = n < SI_PREFILL_ROWS ? n : SI_PREFILL_ROWS;
    const size_t embd = (size_t)cap * hp->n_embd;
    const size_t kv = (size_t)cap * hp->n_head_kv * hp->head_dim;
    const size_t ff = (size_t)cap * hp->n_ff;
    float *mem = si_xmalloc(sizeof(float) * (5 * embd + 2 * kv + 2 * ff));
    pass_bufs b;
    b.x = mem;
    b.xb = b.x + embd;
    b.q = b.xb + embd;
    b.att = b.q + embd;
    b.ff = b.att + embd;
    b.k = b.ff + embd;
    b.v = b.k + kv;
    b.gate = b.v + kv;
    b.up = b.gate + ff;

    si_backend *emb = m->tok_embd.be;
    const float *result = NULL;
    int64_t rows = 0;
    for (int64_t i0 = 0; i0 < n; i0 += rows) {
        rows = n - i0 < cap ? n - i0 : cap;
        for (int64_t r = 0; r < rows; r++)
            emb->row_to_f32(emb, &m->tok_embd, tokens[i0 + r], b.x + r * hp->n_embd);
        if (run_pass(e, &b, e->n_pos, rows)) goto out;
        e->n_pos += rows;
    }
    {
        /* final norm and head of the last row */
        const float *last = b.x + (rows - 1) * hp->n_embd;
        const float *w = view_f32(e, &m->out_norm);
        if (!w) goto out;
        const float s = si_rms_scale(last, (int)hp->n_embd, hp->rms_eps);
        for (uint32_t i = 0; i < hp->n_embd; i++) e->xb[i] = last[i] * s * w[i];
        if (e->layer_cb) e->layer_cb(e, (int)hp->n_layer, e->xb);
        si_backend *head = m->output.be;
        head->gemv(head, &m->output, e->xb, e->logits, (int64_t)hp->n_vocab, e->tp);
        result = e->logits;
    }
out:
    free(mem);
    return result;
}
