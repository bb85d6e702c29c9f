/* The "hip" si_backend: C17 adapter from Siphon's backend vtable to the
 * C-ABI of libsiphon_hip.so (include/sihip.h). See si_hip_backend.h. */
#include "si_hip_backend.h"

#include <dlfcn.h>
#include <stdlib.h>
#include <string.h>

#include "sihip.h"
#ifndef SI_HIP_STANDALONE
#include "siphon/kernels.h"
#endif

/* entry points resolved from the library */
typedef struct {
    int (*abi_version)(void);
    int (*init)(int, sihip_ctx **);
    void (*shutdown)(sihip_ctx *);
    const char *(*last_error)(const sihip_ctx *);
    int (*weight_upload)(sihip_ctx *, uint32_t, uint64_t, uint64_t, const void *, uint64_t,
                         sihip_weight **);
    int (*weight_free)(sihip_ctx *, sihip_weight *);
    int (*weight_prepare_gemm)(sihip_ctx *, sihip_weight *);
    uint64_t (*weight_device_bytes)(const sihip_weight *);
    int (*gemv)(sihip_ctx *, const sihip_weight *, const float *, float *, int64_t);
    int (*gemm)(sihip_ctx *, const sihip_weight *, const float *, int64_t, float *);
    int (*set_option)(sihip_ctx *, const char *, int64_t);
} hip_fns;

/* one uploaded tensor, keyed by its mmap data pointer; type and shape are
 * kept to detect a pointer that now belongs to a different tensor */
typedef struct {
    const void *data;
    uint32_t type;
    uint64_t n_out, n_in, bytes;
    uint64_t print;   /* content fingerprint (fingerprint()) */
    sihip_weight *w;
} slot;

/* A hash of 16 spans of 64 bytes of a tensor: the first, the last and 14
 * evenly spaced between them (all of a tensor of 1 KiB or less), mixed 8
 * bytes at a time, so a lookup costs about 0.1 us. A tensor of the same
 * type and shape mapped at a reused address (a model closed and another
 * opened while the backend stays open) almost surely differs in one of
 * them, so it gets a fresh upload; two tensors that agree at both edges
 * (zero padding, edge blocks a fine-tune left alone) still differ inside. */
static uint64_t fingerprint(const void *data, uint64_t bytes) {
    enum { SPAN = 64, SPANS = 16 };
    const unsigned char *p = data;
    uint64_t h = 0xcbf29ce484222325ULL ^ bytes;
    const uint64_t whole = bytes <= (uint64_t)SPAN * SPANS;
    const uint64_t step = whole ? SPAN : (bytes - SPAN) / (SPANS - 1);
    for (uint64_t s = 0; s < SPANS; s++) {
        const uint64_t off = whole ? s * SPAN : (s + 1 < SPANS ? s * step : bytes - SPAN);
        if (off >= bytes) break;
        const uint64_t len = bytes - off < SPAN ? bytes - off : SPAN;
        for (uint64_t i = 0; i < len; i += 8) {
            uint64_t v = 0;
            memcpy(&v, p + off + i, len - i < 8 ? len - i : 8);
            h = (h ^ v) * 0x100000001b3ULL;
            h ^= h >> 29;
        }
    }
    return h;
}

typedef struct {
    si_backend base;  /* first member: the engine sees a plain si_backend */
    void *dl;
    hip_fns f;
    sihip_ctx *ctx;
    slot *slots;      /* open addressing, capacity a power of two */
    size_t cap, n;
} hip_backend;

static hip_backend *as_hip(si_backend *be) { return (hip_backend *)be; }

static size_t slot_hash(const void *p, size_t cap) {
    uint64_t v = (uint64_t)(uintptr_t)p;
    v ^= v >> 33;
    v *= 0xff51afd7ed558ccdULL;
    v ^= v >> 33;
    return (size_t)v & (cap - 1);
}

static slot *slot_find(hip_backend *hb, const void *data) {
    if (!hb->cap) return NULL;
    for (size_t i = slot_hash(data, hb->cap);; i = (i + 1) & (hb->cap - 1)) {
        if (hb->slots[i].data == data) return &hb->slots[i];
        if (!hb->slots[i].data) return NULL;
    }
}

static int slot_insert(hip_backend *hb, const slot *ins) {
    if ((hb->n + 1) * 2 > hb->cap) {
        const size_t ncap = hb->cap ? hb->cap * 2 : 64;
        slot *ns = calloc(ncap, sizeof *ns);
        if (!ns) return SI_ENOMEM;
        for (size_t i = 0; i < hb->cap; i++) {
            if (!hb->slots[i].data) continue;
            size_t j = slot_hash(hb->slots[i].data, ncap);
            while (ns[j].data) j = (j + 1) & (ncap - 1);
            ns[j] = hb->slots[i];
        }
        free(hb->slots);
        hb->slots = ns;
        hb->cap = ncap;
    }
    size_t j = slot_hash(ins->data, hb->cap);
    while (hb->slots[j].data) j = (j + 1) & (hb->cap - 1);
    hb->slots[j] = *ins;
    hb->n++;
    return SI_OK;
}

/* Map an SIHIP_* code (same values as SI_*; SIHIP_EDEVICE is extra) to SI_*. */
static int si_code(int rc) { return rc == SIHIP_EDEVICE ? SI_EIO : rc; }

/* The device copy of w, uploaded on first use. A cached copy whose key
 * pointer now belongs to a tensor of another type, shape or content (its
 * memory was reused) is stale: it is replaced. */
static int device_weight(hip_backend *hb, const si_tensor *w, sihip_weight **out) {
    const uint64_t n_in = w->ne[0], n_out = w->ne[1] ? w->ne[1] : 1;
    const uint64_t print = fingerprint(w->data, w->n_bytes);
    slot *s = slot_find(hb, w->data);
    if (s) {
        if (s->type == w->type && s->n_out == n_out && s->n_in == n_in && s->bytes == w->n_bytes &&
            s->print == print) {
            *out = s->w;
            return SI_OK;
        }
        sihip_weight *dw = NULL;
        const int rc = hb->f.weight_upload(hb->ctx, w->type, n_out, n_in, w->data, w->n_bytes, &dw);
        if (rc) {
            si_set_err("hip: upload of a %llu x %llu tensor (type %u): %s",
                       (unsigned long long)n_out, (unsigned long long)n_in, (unsigned)w->type,
                       hb->f.last_error(hb->ctx));
            return si_code(rc);
        }
        hb->f.weight_free(hb->ctx, s->w);
        s->type = w->type;
        s->n_out = n_out;
        s->n_in = n_in;
        s->bytes = w->n_bytes;
        s->print = print;
        s->w = dw;
        *out = dw;
        return SI_OK;
    }
    sihip_weight *dw = NULL;
    const int rc = hb->f.weight_upload(hb->ctx, w->type, n_out, n_in, w->data, w->n_bytes, &dw);
    if (rc) {
        si_set_err("hip: upload of a %llu x %llu tensor (type %u): %s",
                   (unsigned long long)n_out, (unsigned long long)n_in, (unsigned)w->type,
                   hb->f.last_error(hb->ctx));
        return si_code(rc);
    }
    const slot ins = {w->data, w->type, n_out, n_in, w->n_bytes, print, dw};
    const int irc = slot_insert(hb, &ins);
    if (irc) {
        hb->f.weight_free(hb->ctx, dw);
        si_set_err("hip: out of host memory for the weight table");
        return irc;
    }
    *out = dw;
    return SI_OK;
}

static void hip_gemv(si_backend *be, const si_tensor *w, const float *x, float *y, int64_t n_out,
                     si_tp *tp) {
    (void)tp;
    hip_backend *hb = as_hip(be);
    sihip_weight *dw;
    if (device_weight(hb, w, &dw)) return;
    if (hb->f.gemv(hb->ctx, dw, x, y, n_out))
        si_set_err("hip gemv: %s", hb->f.last_error(hb->ctx));
}

static void hip_row_to_f32(si_backend *be, const si_tensor *w, uint64_t row, float *out) {
    (void)be;
    si_backend *cpu = si_backend_cpu();
    cpu->row_to_f32(cpu, w, row, out);
}

int si_backend_hip_gemm(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y) {
    if (!be || !w || !X || !Y || M <= 0) {
        si_set_err("hip gemm: bad arguments");
        return SI_EINVAL;
    }
    hip_backend *hb = as_hip(be);
    sihip_weight *dw;
    const int rc = device_weight(hb, w, &dw);
    if (rc) return rc;
    const int grc = hb->f.gemm(hb->ctx, dw, X, M, Y);
    if (grc) {
        si_set_err("hip gemm: %s", hb->f.last_error(hb->ctx));
        return si_code(grc);
    }
    return SI_OK;
}

/* the vtable's gemm slot */
static int hip_gemm(si_backend *be, const si_tensor *w, const float *X, int64_t M, float *Y,
                    si_tp *tp) {
    (void)tp;
    return si_backend_hip_gemm(be, w, X, M, Y);
}

int si_backend_hip_upload(si_backend *be, const si_tensor *w) {
    if (!be || !w || !w->data) {
        si_set_err("hip upload: bad arguments");
        return SI_EINVAL;
    }
    hip_backend *hb = as_hip(be);
    sihip_weight *dw;
    const int rc = device_weight(hb, w, &dw);
    if (rc) return rc;
    const int grc = hb->f.weight_prepare_gemm(hb->ctx, dw);
    if (grc) {
        si_set_err("hip: gemm copy of a %llu x %llu tensor: %s",
                   (unsigned long long)w->ne[1], (unsigned long long)w->ne[0],
                   hb->f.last_error(hb->ctx));
        return si_code(grc);
    }
    return SI_OK;
}

int si_backend_hip_place(si_backend *be, si_tensor *w) {
    const int rc = si_backend_hip_upload(be, w);
    if (rc) return rc;
    w->loc = SI_LOC_DEVICE;
    w->be = be;
    return SI_OK;
}

int si_backend_hip_weights(const si_backend *be, uint64_t *device_bytes) {
    const hip_backend *hb = (const hip_backend *)be;
    uint64_t total = 0;
    for (size_t i = 0; i < hb->cap; i++)
        if (hb->slots[i].data) total += hb->f.weight_device_bytes(hb->slots[i].w);
    if (device_bytes) *device_bytes = total;
    return (int)hb->n;
}

#define RESOLVE(field, name)                                                        \
    do {                                                                            \
        *(void **)(&hb->f.field) = dlsym(hb->dl, name);                             \
        if (!hb->f.field) {                                                         \
            si_set_err("hip: %s has no symbol %s", path, name);                     \
            dlclose(hb->dl);                                                        \
            free(hb);                                                               \
            return SI_ENOENT;                                                       \
        }                                                                           \
    } while (0)

int si_backend_hip_open(const char *lib_path, int device, si_backend **out) {
    if (!out) {
        si_set_err("hip: NULL output");
        return SI_EINVAL;
    }
    const char *path = lib_path ? lib_path : getenv("SIPHON_HIP_LIB");
    if (!path) path = "libsiphon_hip.so";
    hip_backend *hb = calloc(1, sizeof *hb);
    if (!hb) {
        si_set_err("hip: out of host memory");
        return SI_ENOMEM;
    }
    hb->dl = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!hb->dl) {
        si_set_err("hip: cannot load %s: %s", path, dlerror());
        free(hb);
        return SI_ENOENT;
    }
    RESOLVE(abi_version, "sihip_abi_version");
    RESOLVE(init, "sihip_init");
    RESOLVE(shutdown, "sihip_shutdown");
    RESOLVE(last_error, "sihip_last_error");
    RESOLVE(weight_upload, "sihip_weight_upload");
    RESOLVE(weight_free, "sihip_weight_free");
    RESOLVE(weight_prepare_gemm, "sihip_weight_prepare_gemm");
    RESOLVE(weight_device_bytes, "sihip_weight_device_bytes");
    RESOLVE(gemv, "sihip_gemv");
    RESOLVE(gemm, "sihip_gemm");
    RESOLVE(set_option, "sihip_set_option");
    if (hb->f.abi_version() != SIHIP_ABI_VERSION) {
        si_set_err("hip: %s has ABI version %d, this build expects %d", path,
                   hb->f.abi_version(), SIHIP_ABI_VERSION);
        dlclose(hb->dl);
        free(hb);
        return SI_ENOTSUP;
    }
    if (hb->f.init(device, &hb->ctx)) {
        si_set_err("hip: device %d: %s", device, hb->f.last_error(NULL));
        dlclose(hb->dl);
        free(hb);
        return SI_EIO;
    }
    /* Q8_0 activations as the reference's CPU path makes them: its scalar
     * quantizer (kernels.c:542-558) when it runs the scalar kernels (no
     * AVX2, or SI_SCALAR set; kernels.c:56-85), else the SIMD one */
    if (si_kern_impl_get() == SI_KERN_SCALAR &&
        hb->f.set_option(hb->ctx, "Q80_SCALAR", 1)) {
        si_set_err("hip: %s", hb->f.last_error(hb->ctx));
        hb->f.shutdown(hb->ctx);
        dlclose(hb->dl);
        free(hb);
        return SI_EIO;
    }
    hb->base.name = "hip";
    hb->base.loc = SI_LOC_HOST;  /* inputs and outputs are host arrays */
    hb->base.gemv = hip_gemv;
    hb->base.row_to_f32 = hip_row_to_f32;
    hb->base.gemm = hip_gemm;
    *out = &hb->base;
    return SI_OK;
}

void si_backend_hip_close(si_backend *be) {
    if (!be) return;
    hip_backend *hb = as_hip(be);
    for (size_t i = 0; i < hb->cap; i++)
        if (hb->slots[i].data) hb->f.weight_free(hb->ctx, hb->slots[i].w);
    free(hb->slots);
    hb->f.shutdown(hb->ctx);
    dlclose(hb->dl);
    free(hb);
}
