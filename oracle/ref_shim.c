/* ref_shim: drives the compiled reference (oracle/_ref) from tests and the
 * CPU baseline. TEST INFRASTRUCTURE ONLY. Compiled together with the
 * reference's own sources (src/kernels.c, kernels_avx2.c, backend.c,
 * threadpool.c, util.c, gguf.c) by oracle/Makefile; never shipped in the
 * product.
 *
 * It builds an si_tensor view over caller-owned weight bytes and runs the
 * reference CPU backend's gemv (reference backend.c:85-120) through its
 * lane pool (reference threadpool.c:66-146), timing each call with the
 * monotonic clock as the reference's own timing does (util.c:101-105).
 * For the GGUF end-to-end test it also opens a file with the reference's
 * parser (gguf.c:282-408) and makes the tensor views the model loader
 * would (backend.c:144-176).
 */
#include "siphon/gguf.h"
#include "siphon/kernels.h"
#include "siphon/tensor.h"
#include "siphon/threadpool.h"

#include <time.h>

static double now_sec(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* 1 when the reference dispatches to its AVX2 kernels on this host. */
int ref_shim_impl(void) {
    si_kern_init();
    return si_kern_impl_get() == SI_KERN_AVX2;
}

/* Run the reference gemv `reps` times on `lanes` lanes; secs[i] receives
 * the wall time of call i. Returns 0, or -1 on an unsupported type. */
int ref_shim_gemv(uint32_t type, const void *data, int64_t n_out,
                  int64_t n_in, const float *x, float *y, int lanes,
                  int reps, double *secs) {
    uint32_t blk, tsz;
    si_kern_init();
    if (!si_quant_geometry(type, &blk, &tsz) || n_in % blk) return -1;
    si_tensor w;
    memset(&w, 0, sizeof w);
    w.type = type;
    w.ne[0] = (uint64_t)n_in;
    w.ne[1] = (uint64_t)n_out;
    w.n_elems = (uint64_t)(n_in * n_out);
    w.n_bytes = (uint64_t)(n_in / blk) * tsz * (uint64_t)n_out;
    w.data = data;
    w.loc = SI_LOC_HOST;
    w.be = si_backend_cpu();
    si_tp *tp = si_tp_create(lanes);
    for (int r = 0; r < reps; r++) {
        const double t0 = now_sec();
        w.be->gemv(w.be, &w, x, y, n_out, tp);
        secs[r] = now_sec() - t0;
    }
    si_tp_free(tp);
    return 0;
}

/* ---- GGUF container (the model loader's source of weight bytes) ----- */

/* Open path with the reference parser; NULL on failure (ref_shim_errstr). */
void *ref_shim_gguf_open(const char *path) {
    si_gguf *g = NULL;
    return si_gguf_open(path, &g) == SI_OK ? g : NULL;
}

void ref_shim_gguf_close(void *g) { si_gguf_close(g); }

const char *ref_shim_errstr(void) { return si_errstr(); }

/* The loader's view of tensor `name` (si_tensor_from_gguf), assigned to
 * backend `be` (NULL: the reference CPU backend). SI_OK or its error. */
int ref_shim_gguf_tensor(void *g, const char *name, void *be, si_tensor *out) {
    return si_tensor_from_gguf(g, si_gguf_tensor_find(g, name),
                               be ? (si_backend *)be : si_backend_cpu(), out);
}

/* Where p lies relative to the mapped file: its byte offset from the map
 * base, or -1 when it is outside the mapping. */
int64_t ref_shim_gguf_map_offset(void *g, const void *p) {
    const si_gguf *gg = g;
    const uint8_t *b = gg->map, *q = p;
    return (q >= b && q < b + gg->map_size) ? (int64_t)(q - b) : -1;
}

uint64_t ref_shim_gguf_alignment(void *g) { return ((const si_gguf *)g)->alignment; }

int ref_shim_tensor_size(void) { return (int)sizeof(si_tensor); }

/* The reference CPU backend's gemv and row_to_f32 on tensor view w,
 * whatever backend w is assigned to. */
void ref_shim_tensor_gemv(const si_tensor *w, const float *x, float *y, int64_t n_out,
                          int lanes) {
    si_kern_init();
    si_backend *cpu = si_backend_cpu();
    si_tp *tp = si_tp_create(lanes);
    cpu->gemv(cpu, w, x, y, n_out, tp);
    si_tp_free(tp);
}

void ref_shim_tensor_row(const si_tensor *w, uint64_t row, float *out) {
    si_kern_init();
    si_backend *cpu = si_backend_cpu();
    cpu->row_to_f32(cpu, w, row, out);
}
