/* ref_shim: drives the compiled reference (oracle/_ref) from tests and the
 * CPU baseline. TEST INFRASTRUCTURE ONLY. Compiled together with the
 * reference's own sources (src/kernels.c, kernels_avx2.c, backend.c,
 * threadpool.c, util.c) by oracle/Makefile; never shipped in the product.
 *
 * It builds an si_tensor view over caller-owned weight bytes and runs the
 * reference CPU backend's gemv (reference backend.c:85-120) through its
 * lane pool (reference threadpool.c:66-146), timing each call with the
 * monotonic clock as the reference's own timing does (util.c:101-105).
 */
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
