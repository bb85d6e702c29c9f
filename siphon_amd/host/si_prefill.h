/* si_prefill: Siphon's prompt processed layer by layer, M tokens at a time.
 *
 * The reference runs a prompt one token at a time: cmd_run.c:275-283 calls
 * si_engine_forward (engine.c:288-398) once per prompt token, so every
 * weight matrix is streamed once per token through the backend's gemv.
 * si_engine_prefill runs the same graph layer-major instead: per layer,
 * one call of the layer backend's gemm slot per weight matrix for all M
 * rows (the hip backend: the MI355X's int8 and f16 matrix cores), with the
 * per-row steps in between (norms, biases, RoPE, KV-cache writes, attention
 * over the cache, SwiGLU, residuals) computed as si_engine_forward
 * computes them, rows in token order. Attention of row r reads the cache
 * at positions up to its own, all written by then, so each row sees what
 * it sees in the token loop.
 *
 * Inside Siphon this is one more engine source file; here it is built
 * against the mirror of Siphon's declarations (SI_HIP_STANDALONE).
 */
#ifndef SI_PREFILL_H
#define SI_PREFILL_H

#ifdef SI_HIP_STANDALONE
#include "si_engine_mirror.h"
#else
#include "siphon/engine.h"
#include "siphon/kernels.h"
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Rows per layer-major pass: a longer prompt runs in passes of this many
 * tokens (each pass sees the cache the earlier ones wrote), which bounds
 * the host buffers at about 10 * SI_PREFILL_ROWS * n_embd floats. */
#define SI_PREFILL_ROWS 512

/* Run tokens[0..n) at positions e->n_pos .. e->n_pos + n - 1, writing their
 * K and V into the cache, and advance e->n_pos by n. Returns the logits row
 * of the last token (engine-owned, valid until the next call), or NULL with
 * si_errstr() set: n < 1, a token outside the vocabulary, a context too
 * short for all n tokens (nothing is run then), an unsupported norm or bias
 * type, or a failed gemm (positions and cache contents are then
 * unspecified, as after a failed si_engine_forward).
 *
 * The result is that of n calls of si_engine_forward (the last one's
 * logits, the same KV cache) when each layer backend's gemm gives the rows
 * of its gemv, as the CPU backend's (one gemv per row) does bit for bit; a
 * gemm that sums in another f32 order (the hip backend's matrix-core GEMMs)
 * differs from its gemv by that order's rounding, within the tolerance of
 * the reference dot. A backend with no gemm slot (NULL) gets one gemv call
 * per row. The head and embedding go through m->output.be and
 * m->tok_embd.be (the loader sets both to the CPU backend; the reference
 * forward calls si_backend_cpu() there, engine.c:302-303, 393-394).
 * e->layer_cb, if set, is called for every row after every layer, rows in
 * token order, and once with the last row after the final norm. */
const float *si_engine_prefill(si_engine *e, const uint32_t *tokens, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* SI_PREFILL_H */
