/* Declarations of the Siphon types and functions the "hip" backend adapter
 * uses, for building it outside a Siphon tree (SI_HIP_STANDALONE: this
 * repository's tests). Inside Siphon the adapter includes
 * "siphon/tensor.h" instead, which declares the same things; the layouts
 * below must therefore stay identical to:
 *   si_loc, si_tensor, si_backend   reference include/siphon/tensor.h:25-55
 *   SI_* error codes                reference include/siphon/common.h:25-34
 *   si_set_err, si_errstr           reference include/siphon/common.h:36-38
 *   si_tp (opaque lane pool)        reference include/siphon/threadpool.h:19
 *   si_backend_cpu                  reference include/siphon/tensor.h:58
 *   si_kern_impl, si_kern_impl_get  reference include/siphon/kernels.h:28-35
 * plus the two lines a Siphon tree adds to support this backend:
 *   SI_LOC_DEVICE = 2               the device location the reference leaves
 *                                   for a later backend (tensor.h:25-29);
 *                                   si_backend_hip_place tags the tensors it
 *                                   made resident with it.
 *   si_backend.gemm                 a trailing vtable slot (after row_to_f32,
 *                                   tensor.h:54) for M activation rows in one
 *                                   call: the batched prefill's matmuls. The
 *                                   CPU backend fills it with M gemv calls.
 * The backend itself stays tagged SI_LOC_HOST: gemv takes and returns host
 * arrays. */
#ifndef SI_MIRROR_H
#define SI_MIRROR_H

#include <stdint.h>

enum {
    SI_OK = 0,
    SI_ENOMEM = -1,
    SI_EIO = -2,
    SI_EFORMAT = -3,
    SI_ENOTSUP = -4,
    SI_EINVAL = -5,
    SI_ENOENT = -6,
    SI_ERANGE = -7,
};

typedef enum {
    SI_LOC_NONE = 0,
    SI_LOC_HOST = 1,
    SI_LOC_DEVICE = 2,
} si_loc;

typedef struct si_tp si_tp;
typedef struct si_backend si_backend;

typedef struct si_tensor {
    uint32_t type;
    uint64_t ne[4];
    uint64_t n_elems;
    uint64_t n_bytes;
    const void *data;
    si_loc loc;
    si_backend *be;
} si_tensor;

struct si_backend {
    const char *name;
    si_loc loc;
    void (*gemv)(si_backend *be, const si_tensor *w, const float *x, float *y, int64_t n_out,
                 si_tp *tp);
    void (*row_to_f32)(si_backend *be, const si_tensor *w, uint64_t row, float *out);
    /* Y[m, i] = <w.row(i), X[m, :]> for m < M, i < ne[1]: X is [M x ne[0]]
     * and Y [M x ne[1]], row-major host arrays, each X row converted to the
     * pair format on its own (the same per-row result as gemv, up to the
     * f32 summation order). SI_OK, or a negative SI_* code with si_set_err
     * called and Y untouched. */
    int (*gemm)(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y,
                si_tp *tp);
};

const char *si_errstr(void);
void si_set_err(const char *fmt, ...);
si_backend *si_backend_cpu(void);

typedef enum {
    SI_KERN_SCALAR = 0,
    SI_KERN_AVX2 = 1,
} si_kern_impl;

si_kern_impl si_kern_impl_get(void);

#endif /* SI_MIRROR_H */
