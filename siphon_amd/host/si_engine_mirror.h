/* Declarations of the Siphon engine and model types, and of the kernel,
 * thread-pool and allocation functions, that the batched prefill
 * (si_prefill.c) uses, for building it outside a Siphon tree
 * (SI_HIP_STANDALONE: this repository's tests). Inside Siphon the prefill
 * includes "siphon/engine.h" and "siphon/kernels.h" instead, which declare
 * the same things. The layouts below must stay identical to:
 *   si_arch, si_hparams, si_wview,
 *   si_layer, si_model              reference include/siphon/model.h:17-76
 *   si_engine                       reference include/siphon/engine.h:29-68
 * (tests/test_prefill.py compares every field offset with the reference's
 * own build), and the functions to:
 *   si_tp_nlanes, si_tp_run         reference include/siphon/threadpool.h:27-33
 *   si_f32_to_f16, si_vec_dot_for,
 *   si_dequant_row, si_silu,
 *   si_softmax, si_rms_scale        reference include/siphon/kernels.h:24-93
 *   si_quant_name                   reference include/siphon/quant.h:127
 *   si_xmalloc                      reference include/siphon/common.h:47
 */
#ifndef SI_ENGINE_MIRROR_H
#define SI_ENGINE_MIRROR_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "si_mirror.h"

typedef uint16_t si_f16;
typedef struct si_gguf si_gguf;

enum { SI_T_F32 = 0, SI_T_F16 = 1 };

typedef enum {
    SI_ARCH_LLAMA = 0,
    SI_ARCH_QWEN2 = 1,
} si_arch;

typedef struct {
    si_arch arch;
    uint32_t n_vocab;
    uint64_t n_ctx_train;
    uint32_t n_embd;
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t n_layer;
    uint32_t n_rot;
    uint64_t n_ff;
    float rms_eps;
    float rope_freq_base;
    float attn_scale;
    uint32_t head_dim;
    uint32_t n_head_gqa;
} si_hparams;

typedef struct {
    const void *data;
    uint32_t type;
    uint64_t n;
} si_wview;

typedef struct {
    si_tensor wq, wk, wv, wo;
    si_tensor w_gate, w_up, w_down;
    si_wview attn_norm;
    si_wview ffn_norm;
    si_wview bq, bk, bv;
} si_layer;

typedef struct {
    si_gguf *g;
    si_hparams h;
    si_arch arch;
    si_tensor tok_embd;
    si_layer *layers;
    si_wview out_norm;
    si_wview rope_ffs;
    si_tensor output;
    bool output_tied;
    si_backend **layer_be;
} si_model;

typedef struct si_engine {
    si_model *m;
    si_tp *tp;
    void (*layer_cb)(struct si_engine *e, int layer, const float *x);
    void *layer_cb_ctx;
    int64_t n_ctx;
    int64_t n_pos;
    si_f16 *k_cache;
    si_f16 *v_cache;
    float *x, *xb;
    float *q, *k, *v;
    float *attn_out;
    float *gate, *up;
    float *ffbuf;
    float *logits;
    float *rope_cos, *rope_sin;
    float *scores;
    float *probs;
    si_f16 *q16;
    si_f16 *probs16;
    float *wscratch;
    const float *rope_ff;
    float *rope_ff_buf;
    float theta_scale;
    float kq_scale;
} si_engine;

typedef void (*si_task_fn)(void *ctx, int lane, int n_lanes);
int si_tp_nlanes(const si_tp *tp);
void si_tp_run(si_tp *tp, si_task_fn fn, void *ctx);

typedef void (*si_vec_dot_fn)(int n, float *s, const void *x, const void *y);
si_f16 si_f32_to_f16(float f);
si_vec_dot_fn si_vec_dot_for(uint32_t wtype);
bool si_dequant_row(uint32_t type, const void *x, float *y, int n);
float si_silu(float x);
void si_softmax(float *y, const float *x, int n, float max);
float si_rms_scale(const float *x, int n, float eps);
const char *si_quant_name(uint32_t type);
void *si_xmalloc(size_t n);

#endif /* SI_ENGINE_MIRROR_H */
