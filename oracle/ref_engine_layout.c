/* Sizes and field offsets of the mirrored Siphon structs (si_mirror.h,
 * si_engine_mirror.h) as the prefill and the adapter see them, in the order
 * of re_layout (ref_engine_shim.c, the reference's own headers): the tests
 * require both lists to be equal. TEST INFRASTRUCTURE ONLY. */
#include <stddef.h>

#include "si_engine_mirror.h"

#define OFF(T, f) (int64_t) offsetof(T, f)
int re_mirror_layout(int64_t *o) {
    int n = 0;
    o[n++] = sizeof(si_tensor);
    o[n++] = offsetof(si_backend, gemm);  /* the reference struct ends where gemm starts */
    o[n++] = OFF(si_backend, row_to_f32);
    o[n++] = sizeof(si_hparams);
    o[n++] = OFF(si_hparams, n_ctx_train);
    o[n++] = OFF(si_hparams, n_ff);
    o[n++] = OFF(si_hparams, rms_eps);
    o[n++] = OFF(si_hparams, head_dim);
    o[n++] = OFF(si_hparams, n_head_gqa);
    o[n++] = sizeof(si_wview);
    o[n++] = sizeof(si_layer);
    o[n++] = OFF(si_layer, w_down);
    o[n++] = OFF(si_layer, attn_norm);
    o[n++] = OFF(si_layer, bv);
    o[n++] = sizeof(si_model);
    o[n++] = OFF(si_model, h);
    o[n++] = OFF(si_model, arch);
    o[n++] = OFF(si_model, tok_embd);
    o[n++] = OFF(si_model, layers);
    o[n++] = OFF(si_model, out_norm);
    o[n++] = OFF(si_model, rope_ffs);
    o[n++] = OFF(si_model, output);
    o[n++] = OFF(si_model, output_tied);
    o[n++] = OFF(si_model, layer_be);
    o[n++] = sizeof(si_engine);
    o[n++] = OFF(si_engine, layer_cb);
    o[n++] = OFF(si_engine, n_ctx);
    o[n++] = OFF(si_engine, n_pos);
    o[n++] = OFF(si_engine, k_cache);
    o[n++] = OFF(si_engine, v_cache);
    o[n++] = OFF(si_engine, xb);
    o[n++] = OFF(si_engine, logits);
    o[n++] = OFF(si_engine, rope_cos);
    o[n++] = OFF(si_engine, rope_sin);
    o[n++] = OFF(si_engine, scores);
    o[n++] = OFF(si_engine, probs);
    o[n++] = OFF(si_engine, q16);
    o[n++] = OFF(si_engine, probs16);
    o[n++] = OFF(si_engine, wscratch);
    o[n++] = OFF(si_engine, rope_ff);
    o[n++] = OFF(si_engine, theta_scale);
    o[n++] = OFF(si_engine, kq_scale);
    o[n++] = sizeof(si_backend);
    o[n++] = OFF(si_backend, gemm);
    return n;
}
