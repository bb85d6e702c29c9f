/* Test harness for the "hip" si_backend adapter (siphon_amd/host).
 * TEST INFRASTRUCTURE ONLY. It supplies what a Siphon build would: the
 * error-string functions and a CPU backend whose gemv, gemm (one gemv per
 * row, as the reference CPU backend fills the slot) and row_to_f32 use this
 * repository's CPU oracle (oracle/siq_oracle.c), and exposes the vtable
 * through plain functions for ctypes. */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "si_hip_backend.h"
#include "../../oracle/siq_oracle.h"

static char g_err[512];

const char *si_errstr(void) { return g_err; }

void si_set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

static void cpu_row_to_f32(si_backend *be, const si_tensor *w, uint64_t row, float *out) {
    (void)be;
    uint32_t blk, bytes;
    if (!siq_geometry(w->type, &blk, &bytes)) {
        si_set_err("cpu row_to_f32: unsupported type %u", (unsigned)w->type);
        return;
    }
    const uint64_t row_bytes = w->ne[0] / blk * bytes;
    siq_dequant_row(w->type, (const char *)w->data + row * row_bytes, out, (int64_t)w->ne[0]);
}

/* gemv with the oracle's exact dots (f32 results); y untouched on error */
static void cpu_gemv(si_backend *be, const si_tensor *w, const float *x, float *y, int64_t n_out,
                     si_tp *tp) {
    (void)be;
    (void)tp;
    if (!siq_gemv(w->type, w->data, n_out, (int64_t)w->ne[0], x, y, NULL, 1))
        si_set_err("cpu gemv: unsupported type %u", (unsigned)w->type);
}

/* the gemm slot as the CPU backend fills it: one gemv per activation row */
static int cpu_gemm(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y,
                    si_tp *tp) {
    const int64_t n_in = (int64_t)w->ne[0], n_out = w->ne[1] ? (int64_t)w->ne[1] : 1;
    g_err[0] = 0;
    for (int64_t m = 0; m < M; m++) {
        be->gemv(be, w, X + m * n_in, Y + m * n_out, n_out, tp);
        if (g_err[0]) return SI_EINVAL;
    }
    return SI_OK;
}

static si_backend g_cpu = {"cpu", SI_LOC_HOST, cpu_gemv, cpu_row_to_f32, cpu_gemm};

si_backend *si_backend_cpu(void) { return &g_cpu; }

/* The reference's kernel choice as its SI_SCALAR override sets it
 * (reference kernels.c:80-83); the harness assumes an AVX2 host otherwise. */
si_kern_impl si_kern_impl_get(void) {
    const char *env = getenv("SI_SCALAR");
    return env && env[0] && strcmp(env, "0") != 0 ? SI_KERN_SCALAR : SI_KERN_AVX2;
}

static si_tensor make_tensor(si_backend *be, uint32_t type, uint64_t n_out, uint64_t n_in,
                             const void *data, uint64_t bytes) {
    si_tensor t;
    memset(&t, 0, sizeof t);
    t.type = type;
    t.ne[0] = n_in;
    t.ne[1] = n_out;
    t.n_elems = n_in * n_out;
    t.n_bytes = bytes;
    t.data = data;
    t.loc = SI_LOC_HOST;
    t.be = be;
    return t;
}

const char *th_errstr(void) { return g_err; }

int th_open(const char *path, int device, si_backend **be) {
    g_err[0] = 0;
    return si_backend_hip_open(path, device, be);
}

void th_close(si_backend *be) { si_backend_hip_close(be); }

const char *th_name(si_backend *be) { return be->name; }

/* gemv through the vtable; returns 0, or -1 with th_errstr() set */
int th_gemv(si_backend *be, uint32_t type, uint64_t n_out, uint64_t n_in, const void *data,
            uint64_t bytes, const float *x, float *y, int64_t n) {
    g_err[0] = 0;
    const si_tensor t = make_tensor(be, type, n_out, n_in, data, bytes);
    be->gemv(be, &t, x, y, n, NULL);
    return g_err[0] ? -1 : 0;
}

si_backend *th_cpu(void) { return &g_cpu; }

/* the vtable's gemm slot of be (the hip backend or th_cpu()) */
int th_vtable_gemm(si_backend *be, uint32_t type, uint64_t n_out, uint64_t n_in, const void *data,
                   uint64_t bytes, const float *X, int64_t M, float *Y) {
    g_err[0] = 0;
    const si_tensor t = make_tensor(be, type, n_out, n_in, data, bytes);
    return be->gemm(be, &t, X, M, Y, NULL);
}

int th_gemm(si_backend *be, uint32_t type, uint64_t n_out, uint64_t n_in, const void *data,
            uint64_t bytes, const float *X, int64_t M, float *Y) {
    g_err[0] = 0;
    const si_tensor t = make_tensor(be, type, n_out, n_in, data, bytes);
    return si_backend_hip_gemm(be, &t, X, M, Y);
}

int th_row_to_f32(si_backend *be, uint32_t type, uint64_t n_out, uint64_t n_in, const void *data,
                  uint64_t bytes, uint64_t row, float *out) {
    g_err[0] = 0;
    const si_tensor t = make_tensor(be, type, n_out, n_in, data, bytes);
    be->row_to_f32(be, &t, row, out);
    return g_err[0] ? -1 : 0;
}

int th_weights(si_backend *be, uint64_t *bytes) { return si_backend_hip_weights(be, bytes); }

int th_upload(si_backend *be, uint32_t type, uint64_t n_out, uint64_t n_in, const void *data,
              uint64_t bytes) {
    g_err[0] = 0;
    const si_tensor t = make_tensor(be, type, n_out, n_in, data, bytes);
    return si_backend_hip_upload(be, &t);
}

/* ---- tensor views made by the reference loader (GGUF end-to-end) ---- */

int th_tensor_size(void) { return (int)sizeof(si_tensor); }

int th_place(si_backend *be, si_tensor *t) {
    g_err[0] = 0;
    return si_backend_hip_place(be, t);
}

/* The routed engine's calls: through the backend the tensor is assigned to
 * (t->be), as m->layer_be[il]->gemv, m->output.be->gemv and
 * m->tok_embd.be->row_to_f32 would. Return 0, or -1 with th_errstr() set. */
int th_tensor_gemv(const si_tensor *t, const float *x, float *y, int64_t n) {
    g_err[0] = 0;
    t->be->gemv(t->be, t, x, y, n, NULL);
    return g_err[0] ? -1 : 0;
}

int th_tensor_row(const si_tensor *t, uint64_t row, float *out) {
    g_err[0] = 0;
    t->be->row_to_f32(t->be, t, row, out);
    return g_err[0] ? -1 : 0;
}

int th_tensor_gemm(si_backend *be, const si_tensor *t, const float *X, int64_t M, float *Y) {
    g_err[0] = 0;
    return si_backend_hip_gemm(be, t, X, M, Y);
}
