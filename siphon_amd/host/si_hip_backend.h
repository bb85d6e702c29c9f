/* si_hip_backend: a Siphon si_backend whose gemv runs on an MI355X.
 *
 * The reference routes every weight x activation product of a layer
 * through the backend vtable (reference include/siphon/tensor.h:43-55;
 * engine.c:317-378 picks m->layer_be[il]). This adapter is a second
 * instance of that vtable, named "hip", written in C17 like the reference
 * host: it dlopens libsiphon_hip.so (the C-ABI of include/sihip.h), so the
 * engine links no HIP code and starts without a GPU when the backend is
 * not requested.
 *
 *   gemv        y = W x through sihip_gemv. Each weight tensor is uploaded
 *               once, on its first use, keyed by its mmap data pointer;
 *               the device keeps its own repacked copy, the mmap stays
 *               borrowed. Same contract as cpu_gemv (reference
 *               backend.c:85-120): on failure si_set_err is called and y
 *               is left untouched. The lane pool argument is unused.
 *   row_to_f32  the embedding row lookup (once per token, reference
 *               engine.c:303): delegated to the CPU backend's dequantizer
 *               on the mmap'd row, which is where the weight bytes live.
 *   gemm        the prefill slot the vtable gains (si_backend_hip_gemm):
 *               Y[m, :] = W X[m, :] for M rows in one call.
 *
 * There is no silent CPU fallback: if the library or the device is
 * missing, si_backend_hip_open fails with a message and the caller keeps
 * its CPU backend (that choice is the engine's, as for any backend).
 */
#ifndef SI_HIP_BACKEND_H
#define SI_HIP_BACKEND_H

#ifdef SI_HIP_STANDALONE
#include "si_mirror.h"
#else
#include "siphon/tensor.h"
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* dlopen lib_path (NULL: $SIPHON_HIP_LIB, else "libsiphon_hip.so" on the
 * loader path), check its ABI version and open device `device`.
 * Returns SI_OK and the backend, or a negative SI_* code with si_errstr()
 * set: SI_ENOENT (library not found or symbol missing), SI_ENOTSUP (ABI
 * version mismatch), SI_EIO (no usable device). */
int si_backend_hip_open(const char *lib_path, int device, si_backend **out);

/* Free every uploaded weight, the device context and the library handle. */
void si_backend_hip_close(si_backend *be);

/* Prefill: Y[m, :] = <W rows, X[m, :]> for m < M; X is [M x ne0] and Y is
 * [M x ne1], row-major host arrays. SI_OK or a negative SI_* code (Y
 * untouched on failure). */
int si_backend_hip_gemm(si_backend *be, const si_tensor *w, const float *X, int64_t M,
                        float *Y);

/* Upload w now rather than on its first gemv or gemm: the model loader's
 * hook for device-resident weights (after si_tensor_from_gguf, reference
 * backend.c:144-176, model.c:13), so neither the first token nor the first
 * prompt pays an upload. Builds the matrix-core GEMM copy too where the type
 * has one. Idempotent: a tensor already on the device (same data pointer,
 * type and shape) is not uploaded again. SI_OK or a negative SI_* code with
 * si_errstr() set. */
int si_backend_hip_upload(si_backend *be, const si_tensor *w);

/* Make w resident on the device and assign it to this backend: uploads it
 * as si_backend_hip_upload does, then sets w->loc = SI_LOC_DEVICE and
 * w->be = be. w->data keeps the mmap pointer: it stays the key of the
 * device copy and the source row_to_f32 reads (the model must keep its
 * si_gguf open, as for the CPU backend). The model loader's hook for the
 * tensors of layers assigned to this backend and for the output head
 * (reference model.c:171; the engine then reaches them through
 * m->layer_be[il] and m->output.be). On failure w is left untouched. SI_OK
 * or a negative SI_* code with si_errstr() set. */
int si_backend_hip_place(si_backend *be, si_tensor *w);

/* Number of weight tensors uploaded so far and their device bytes. */
int si_backend_hip_weights(const si_backend *be, uint64_t *device_bytes);

#ifdef __cplusplus
}
#endif

#endif /* SI_HIP_BACKEND_H */
