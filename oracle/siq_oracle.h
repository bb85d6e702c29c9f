/* siq_oracle: CPU oracle for Siphon's quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (siphon_amd/) links,
 * loads or calls this library; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker.
 *
 * It is an independent C17 restatement of the reference's block formats,
 * activation quantizers and dot products:
 *   block layouts            include/siphon/quant.h:31-100
 *   f16 <-> f32              src/kernels.c:98-176
 *   nearest_int, Q8_K quant  src/kernels.c:528-533, 561-595
 *   Q8_0 quant (SIMD form)   src/kernels_avx2.c:594-645
 *   Q8_0 quant (scalar form) src/kernels.c:542-558
 *   dequantization           src/kernels.c:599-817
 *   dot products             src/kernels.c:180-523 (value semantics)
 *   activation pairing       src/kernels.c:946-960
 *   gemv driver              src/backend.c:17-120
 *
 * Dot products are evaluated EXACTLY: the integer parts as int64 sums and
 * the block scales in double, so the result is the true value of the
 * quantized dot. The reference's float accumulation differs from it by
 * about 1e-7 of the L1 norm of the terms; every output is also returned
 * with that L1 norm so tests can apply |gpu - ref| <= 1e-5*L1 + 1e-6.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   f16 conversion: exhaustive 65536 round trip + numpy float16 over
 *     random and edge floats; golden vectors from the compiled reference.
 *   quantizers: bit-exact against golden vectors (quants, d, bsums) and
 *     the compiled reference on seeded inputs, plus invariants.
 *   dequant: bit-exact against golden vectors and the compiled reference.
 *   dots: exact-integer formulation checked against an element-wise
 *     dequant formulation (independent) and the reference's outputs.
 */
#ifndef SIQ_ORACLE_H
#define SIQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (on-disk enum values). */
enum {
    SIQ_F32 = 0,
    SIQ_F16 = 1,
    SIQ_Q4_0 = 2,
    SIQ_Q5_0 = 6,
    SIQ_Q8_0 = 8,
    SIQ_Q2_K = 10,
    SIQ_Q3_K = 11,
    SIQ_Q4_K = 12,
    SIQ_Q5_K = 13,
    SIQ_Q6_K = 14,
    SIQ_Q8_K = 15,
};

/* Elements and bytes per block; 0 for unsupported types. */
int siq_geometry(uint32_t type, uint32_t *blk_elems, uint32_t *blk_bytes);
/* Activation format a weight type pairs with; 0 if unsupported. */
int siq_pair(uint32_t wtype, uint32_t *pair);

float siq_f16_to_f32(uint16_t h);
uint16_t siq_f32_to_f16(float f);

/* Activation quantizers. n must be a multiple of the block size. */
void siq_quantize_q8_K(const float *x, void *out, int64_t n);
/* SIMD-path semantics (the one production dispatches on x86). */
void siq_quantize_q8_0(const float *x, void *out, int64_t n);
/* Portable scalar-path semantics (SI_SCALAR=1). */
void siq_quantize_q8_0_scalar(const float *x, void *out, int64_t n);
void siq_convert_f16(const float *x, uint16_t *out, int64_t n);
/* Convert x into the given pair format (F16, Q8_0 SIMD semantics, Q8_K). */
int siq_quantize_pair(uint32_t pair, const float *x, void *out, int64_t n);

/* Weight values of one row, as the reference dequantizer produces them. */
int siq_dequant_row(uint32_t type, const void *w, float *out, int64_t n);

/* Exact dot of one weight row against pair-format activations. */
int siq_vec_dot(uint32_t wtype, int64_t n, const void *w, const void *a,
                double *dot, double *l1);
/* Same value computed element-wise from dequantized weights and
 * activations (independent formulation, used to cross-check). */
int siq_vec_dot_dequant(uint32_t wtype, int64_t n, const void *w,
                        const void *a, double *dot, double *l1);

/* y[r] = <W.row(r), pair(x)> for r < n_out, rows n_in long. Converts x
 * once, then one exact dot per row, rows split across `lanes` threads in
 * contiguous chunks. l1 (optional) receives each row's term L1 norm. */
int siq_gemv(uint32_t wtype, const void *W, int64_t n_out, int64_t n_in,
             const float *x, float *y, double *l1, int lanes);
/* M independent gemvs: Y[m, :] = gemv(W, X[m, :]). */
int siq_gemm(uint32_t wtype, const void *W, int64_t n_out, int64_t n_in,
             const float *X, int64_t M, float *Y, double *L1, int lanes);

/* ---- decode attention over an f16 KV cache (reference engine.c:90-147) --
 * Evaluated in the reference's x86 operation order, bit for bit:
 *   siq_expf_poly     the exp polynomial of softmax groups, kernels.c:820-850
 *   siq_softmax       groups of 8 with the 8-lane sum order, a double total,
 *                     libm expf on the tail, kernels.c:855-885
 *   siq_dot_f16_simd  32 f32 FMA accumulators, the register/lane reduction
 *                     tree, the tail in double, kernels_avx2.c:118-148
 * Pinned (tests/test_oracle_attn.py) against the compiled reference's own
 * functions and an attention golden fixture from it, bit-exact, and against
 * double-precision mathematics (exp error, softmax sum, dot value). */
float siq_expf_poly(float x);
void siq_softmax(float *y, const float *x, int64_t n, float max);
float siq_dot_f16_simd(int64_t n, const uint16_t *a, const uint16_t *b);
/* Every head h of one layer at position pos: q f32 [n_head * hd]; the
 * layer's caches k f16 [n_head_kv][n_ctx][hd] and v f16 [n_head_kv][hd][n_ctx]
 * (reference engine.c:200-203, 345-357); KV head h / (n_head / n_head_kv).
 * out f32 [n_head * hd]; scores (scaled, f32) and probs16 (f16 bits), each
 * [n_head][n_ctx] with the first pos + 1 entries of a row written, are
 * optional. Returns 1, or 0 on bad arguments. */
int siq_attn_decode(const float *q, const uint16_t *k, const uint16_t *v, int64_t n_head,
                    int64_t n_head_kv, int64_t hd, int64_t n_ctx, int64_t pos, float kq_scale,
                    float *out, float *scores, uint16_t *probs16);

#ifdef __cplusplus
}
#endif

#endif /* SIQ_ORACLE_H */
