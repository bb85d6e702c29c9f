/* sihip: C-ABI of libsiphon_hip.so, the MI355X (gfx950) backend for
 * Siphon's quantized matvec / matmul path.
 *
 * The reference routes every weight x activation product through one
 * vtable slot, si_backend.gemv (reference include/siphon/tensor.h:43-55),
 * whose CPU implementation is cpu_gemv (reference src/backend.c:85-120):
 * convert the f32 activation row once into the weight type's "dot pair"
 * format (Q8_K for K-quants, Q8_0 for Q4_0/Q5_0/Q8_0, F16 for F16), then
 * one full dot product per output row. This library is the device side of
 * a second si_backend instance: the host (C17) dlopens it, uploads each
 * weight tensor once, and forwards gemv calls here. Plain C types only;
 * no HIP or torch types cross this boundary (streams are opaque void*).
 *
 * Graph capture: the *_dev entry points may be captured into a HIP graph
 * once their workspaces exist. A call that would have to allocate during
 * capture (a context workspace growing, a weight's GEMM copy not yet built)
 * returns SIHIP_EINVAL instead. A workspace that grows is replaced, not
 * freed: graphs captured earlier keep using the old buffer, which stays
 * allocated until sihip_shutdown.
 *
 * Conventions (mirroring the reference):
 *  - return 0 (SI_OK) or a negative SI_* code (reference
 *    include/siphon/common.h:25-34); SIHIP_EDEVICE is added for HIP
 *    runtime failures. A human-readable message for the last failure on a
 *    context is available from sihip_last_error (like si_errstr,
 *    reference src/util.c:7-17, but per context).
 *  - on failure, outputs are left untouched (reference backend.c:90-98).
 *  - weight shapes follow the reference: W is [n_out x n_in] row-major,
 *    ne[0] = n_in, each row n_in / block_elems consecutive GGUF blocks
 *    (reference backend.c:88, 112; tensor.h:66-70).
 *  - results are deterministic run to run: no split-K atomics, every
 *    output is reduced in a fixed order.
 */
#ifndef SIHIP_H
#define SIHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIHIP_ABI_VERSION 3

/* error codes: the reference's SI_* values plus one for the device */
#define SIHIP_OK        0
#define SIHIP_ENOMEM   (-1)
#define SIHIP_ENOTSUP  (-4)
#define SIHIP_EINVAL   (-5)
#define SIHIP_ERANGE   (-7)
#define SIHIP_EDEVICE  (-8)

typedef struct sihip_ctx sihip_ctx;
typedef struct sihip_weight sihip_weight;

/* ---- lifecycle ------------------------------------------------------- */

/* Returns SIHIP_ABI_VERSION; the loader refuses a library whose value
 * differs from the header it was compiled against. */
int sihip_abi_version(void);

/* Open a context on HIP device `device` (0-based). */
int sihip_init(int device, sihip_ctx **out);
/* Release the context and its staging buffers. Weights must be freed
 * first. */
void sihip_shutdown(sihip_ctx *ctx);
/* Message of the most recent failure on ctx ("" if none). With ctx NULL,
 * the most recent failure of sihip_init. */
const char *sihip_last_error(const sihip_ctx *ctx);
/* Tuning knob of a context (no reference counterpart: layout and launch
 * choices of this backend, for tests and tuning). Each is read once from
 * the environment variable SIHIP_<name> at sihip_init; a negative value
 * restores the built-in rule. Names: WG_PER_CU, WAVE_TARGET, SPLIT_ELEMS,
 * TILE_COLS (these four apply to later uploads and launches), GEMM_MIN_M,
 * GEMM_MT, GEMM_SBK, GEMM2_MIN_M, GEMM2_WAVES, GEMM6_MIN_M, GEMMH_MIN_M,
 * GEMMQ_MIN_M, GEMMQ_XMODE, GEMM2S_MAX_M, GEMMKS_MAX_M (the largest M on
 * the small-M K-quant GEMMs, 0: none), GEMMKS_Q4K, GEMMS_WAVES, and
 * Q80_SCALAR: 1 quantizes Q8_0-pair
 * activations with the reference's portable scalar routine (reference
 * kernels.c:542-558), as the reference does when SI_SCALAR is set or the
 * host lacks AVX2 (kernels.c:56-85); the rule is the SIMD routine
 * (kernels_avx2.c:594-645). Unknown names: SIHIP_EINVAL. */
int sihip_set_option(sihip_ctx *ctx, const char *name, int64_t value);

/* ---- weights --------------------------------------------------------- */

/* Upload one weight matrix given as GGUF blocks (the bytes of an mmap'd
 * tensor, reference si_tensor.data, tensor.h:30-38). ggml_type is the
 * on-disk type id (reference quant.h:103-119): F16, Q4_0, Q5_0, Q8_0,
 * Q2_K, Q3_K, Q4_K, Q5_K, Q6_K. `bytes` must equal
 * n_out * (n_in / block_elems) * block_bytes, and n_in must be a multiple
 * of the block size (reference backend.c:158-164 rejects the same). The
 * device keeps its own copy, repacked for the kernels; the host bytes
 * stay owned by the caller. */
int sihip_weight_upload(sihip_ctx *ctx, uint32_t ggml_type, uint64_t n_out,
                        uint64_t n_in, const void *host_blocks,
                        uint64_t bytes, sihip_weight **out);
int sihip_weight_free(sihip_ctx *ctx, sihip_weight *w);
/* Build now the weight's second device copy in the order of the
 * matrix-core GEMMs (the K-quants, F16, Q4_0, Q5_0, Q8_0), which sihip_gemm
 * otherwise builds on its first call with M >= 3. No reference
 * counterpart: it belongs to the batched prefill slot, which the reference
 * lacks (its prompt runs token by token, cmd_run.c:275-283). For loaders
 * that put everything on the device before the first token. Idempotent. */
int sihip_weight_prepare_gemm(sihip_ctx *ctx, sihip_weight *w);
/* Device bytes the weight occupies: the repacked copy (>= the GGUF bytes),
 * the column-slice partial sums, and the GEMM copy once built. */
uint64_t sihip_weight_device_bytes(const sihip_weight *w);
/* Layout introspection: row columns (256-element super-blocks for the
 * K-quants, 32-element blocks otherwise) handled side by side by one
 * wavefront, 1..64 (a power of two). Chosen at upload from the shape; the
 * option TILE_COLS (sihip_set_option) forces it (tests, tuning). */
int sihip_weight_tile_cols(const sihip_weight *w);
/* Layout introspection: rounds of a wave tile (tile_cols columns each) per
 * column slice of the matvec. Rows of 8192 elements or more are cut into
 * slices of about 4096 elements computed by separate workgroups and added
 * in slice order; equal to the tile's round count when the rows are not
 * sliced. The option SPLIT_ELEMS (sihip_set_option) sets the slice length
 * in elements at upload (0: no slices). */
int sihip_weight_slice_rounds(const sihip_weight *w);

/* ---- matvec / matmul: host pointers, synchronous ---------------------
 * Same semantics as the reference cpu_gemv (backend.c:85-120):
 * y[i] = <W.row(i), pair(x)> for i < n_out, with pair(x) the activation
 * converted by the bit-exact quantizer of the weight type's pair format.
 * n_out may be smaller than the uploaded row count (reference gemv takes
 * n_out from the caller, engine.c:317-378). */
int sihip_gemv(sihip_ctx *ctx, const sihip_weight *w, const float *x,
               float *y, int64_t n_out);
/* Prefill: Y[m, :] = gemv(W, X[m, :]) for m < M; X is [M x n_in] and Y is
 * [M x n_out], row-major. The reference has no GEMM (prompt tokens run one
 * si_engine_forward each, reference cmd_run.c:275-283); this is its
 * batched equivalent, with X quantized per row. */
int sihip_gemm(sihip_ctx *ctx, const sihip_weight *w, const float *X,
               int64_t M, float *Y);
/* Weight values of one row, out[0..n_in): the si_backend row_to_f32 slot
 * (reference backend.c:122-131, which calls si_dequant_row_* of
 * kernels.c:599-817), from the device copy, bit-identical to the reference
 * dequantizer. */
int sihip_dequant_row(sihip_ctx *ctx, const sihip_weight *w, uint64_t row,
                      float *out);

/* ---- device pointers, stream-ordered (no host synchronisation) -------
 * x, y, X, Y point to device memory; stream is a hipStream_t (NULL for
 * the default stream). */
int sihip_gemv_dev(sihip_ctx *ctx, const sihip_weight *w, const float *x,
                   float *y, int64_t n_out, void *stream);
int sihip_gemm_dev(sihip_ctx *ctx, const sihip_weight *w, const float *X,
                   int64_t M, float *Y, void *stream);
/* sihip_gemm_dev that allocates nothing. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc). Same
 * kernels and results as sihip_gemm_dev; the quantized activation planes,
 * K-slice partial sums and arrival counters live in a static scratch of
 * 16 MiB + 256 KiB per device instead of the context's workspaces. Limits:
 * the activation planes must fit the scratch (about M * n_in <= 14.7e6;
 * larger calls return SIHIP_ERANGE); where the K-slice partial sums do not
 * fit as well, the call runs without K slices. The weight's GEMM copy must
 * exist (sihip_weight_prepare_gemm), else SIHIP_EINVAL. All calls on one
 * device share the scratch: calls that overlap on a device race. */
int sihip_gemm_dev_noalloc(sihip_ctx *ctx, const sihip_weight *w, const float *X,
                           int64_t M, float *Y, void *stream);
/* Rows [row0, row0 + nrows) dequantized as sihip_dequant_row, row r at
 * out + (r - row0) * ldo (out 16-byte aligned, ldo >= n_in, a multiple of
 * 4): an embedding lookup for a host that keeps activations on the device. */
int sihip_dequant_rows_dev(sihip_ctx *ctx, const sihip_weight *w,
                           uint64_t row0, uint64_t nrows, float *out,
                           int64_t ldo, void *stream);
/* Several matrices that share one input x (q/k/v at reference
 * engine.c:317-319, gate/up at 375-376) in one launch: y[i] receives
 * gemv(w[i], x). All w[i] must have the same n_in; at most 4. */
int sihip_gemv_multi_dev(sihip_ctx *ctx, int count,
                         const sihip_weight *const *w, const float *x,
                         float *const *y, void *stream);
/* The M-row counterpart: Y[i] (M x n_out[i], row-major) receives
 * sihip_gemm_dev(w[i], X), the weights sharing one X (M x n_in, 16-byte
 * aligned): the q/k/v and gate/up matrices of the batched forward that
 * replaces the reference's prompt loop (cmd_run.c:275-283; engine.c:317-319,
 * 375-376, whose gemv calls each re-quantize x, backend.c:100-108). The
 * activation is quantized once per record layout; weights of one kernel
 * family run with one m-tile count, so their K slicing, and with it the f32
 * summation order, may differ from a single sihip_gemm_dev call (same
 * tolerance). All w[i] must have the same n_in; at most 4. */
int sihip_gemm_multi_dev(sihip_ctx *ctx, int count,
                         const sihip_weight *const *w, const float *X,
                         int64_t M, float *const *Y, void *stream);

/* Decode attention of one layer at position pos over an f16 KV cache, for
 * every query head h (reference attn_head, engine.c:90-147): the query
 * narrowed to f16; score j = f16 dot(key j, query) * kq_scale for
 * j <= pos; softmax; probabilities narrowed to f16; out[h * head_dim + c] =
 * f16 dot(value row c, probabilities). KV head of h: h / (n_head /
 * n_head_kv). Device pointers, the layer's slice of the reference's cache
 * layouts (engine.c:200-203, 345-357):
 *   q        f32 [n_head * head_dim]
 *   k_cache  f16 bits [n_head_kv][n_ctx][head_dim]
 *   v_cache  f16 bits [n_head_kv][head_dim][n_ctx]  (transposed)
 *   out      f32 [n_head * head_dim]
 *   scores   f32 [n_head][n_ctx] scaled scores, optional (NULL: the
 *            context's workspace)
 *   probs16  f16 bits [n_head][n_ctx] probabilities, optional (NULL: not
 *            written)
 *   the first pos + 1 entries of each row are written.
 * Bit-identical to the reference's x86 path (its AVX2 f16 dot, softmax and
 * exp polynomial), up to the order of the softmax's double total and the
 * rounding of libm's expf on the last n % 8 positions, which change a
 * result only in rare cases. head_dim <= 512. Calls sharing a context's
 * workspace must not overlap. */
int sihip_attn_decode_dev(sihip_ctx *ctx, const float *q, const uint16_t *k_cache,
                          const uint16_t *v_cache, int64_t n_head, int64_t n_head_kv,
                          int64_t head_dim, int64_t n_ctx, int64_t pos, float kq_scale,
                          float *out, float *scores, uint16_t *probs16, void *stream);

/* ---- device memory for hosts without a HIP runtime of their own -------
 * The reference host is plain C17 and never links HIP; these let it (and
 * tests) hold activations and outputs on the device for the *_dev entry
 * points. Copies are synchronous and ordered after all work on the
 * device's default stream. */
int sihip_dev_alloc(sihip_ctx *ctx, uint64_t bytes, void **dptr);
int sihip_dev_free(sihip_ctx *ctx, void *dptr);
int sihip_memcpy_htod(sihip_ctx *ctx, void *dst, const void *src, uint64_t bytes);
int sihip_memcpy_dtoh(sihip_ctx *ctx, void *dst, const void *src, uint64_t bytes);
/* Wait for all work on the context's device. */
int sihip_synchronize(sihip_ctx *ctx);

/* ---- building blocks exposed for parity tests ------------------------ */

/* Activation quantizers on the device, host pointers. n must be a multiple
 * of the block size. Output bytes are the reference block layouts:
 *  Q8_K (reference kernels.c:561-595): f32 d, int8 qs[256], int16
 *    bsums[16] per 256 (292 B); bsums of an all-zero block are written as 0.
 *  Q8_0 (reference kernels_avx2.c:594-645, the SIMD path production
 *    dispatches to on x86): f16 d, int8 qs[32] per 32 (34 B).
 *  F16 pair conversion (reference backend.c:19-27): RNE binary16. */
int sihip_quantize_q8_K(sihip_ctx *ctx, const float *x, void *out, int64_t n);
/* X [M x n_in] (host, row-major) through the GEMMs' activation quantizer
 * (the records of the matrix-core kernels, m blocks of bm = 16, 32, 64 or
 * 128 rows), read back into out as each row's Q8_K blocks in the layout of
 * si_quant_row_q8_K (kernels.h:67; 292 bytes per block, rows in order), so
 * they can be compared with it bit for bit. */
int sihip_quantize_q8_K_rows(sihip_ctx *ctx, const float *X, int64_t M, int64_t n_in,
                             int bm, void *out);
int sihip_quantize_q8_0(sihip_ctx *ctx, const float *x, void *out, int64_t n);
int sihip_convert_f16(sihip_ctx *ctx, const float *x, void *out, int64_t n);

/* One dot product on the device with the per-row kernel ABI of the
 * reference (si_vec_dot_fn, reference kernels.h:45): *s = <x, y> where x
 * is one row of `wtype` blocks and y is already in the pair format. */
int sihip_vec_dot(sihip_ctx *ctx, uint32_t wtype, int n, float *s,
                  const void *x, const void *y);

/* Calibration, with no counterpart in the reference: one streaming read
 * of `bytes` bytes at p (device memory, 16-byte aligned, bytes a multiple
 * of 16) in one launch, nothing written unless a folded checksum of the
 * data hits a fixed 32-bit value (then one word per workgroup goes to
 * sink, which must hold 4096 words). It measures the HBM rate a launch
 * that only reads that many bytes reaches, the ceiling the matvec
 * launches are compared with. */
int sihip_probe_read_dev(sihip_ctx *ctx, const void *p, uint64_t bytes, uint32_t *sink,
                         void *stream);

/* Matvec over n_rows consecutive weight rows (host bytes) against a
 * pair-format activation (host bytes): the per-row dot of many rows in one
 * launch, used by parity tests with the reference's own quantized input. */
int sihip_gemv_pair(sihip_ctx *ctx, uint32_t wtype, int64_t n_rows,
                    int64_t n_in, const void *rows, const void *xq,
                    float *y);

#ifdef __cplusplus
}
#endif

#endif /* SIHIP_H */
