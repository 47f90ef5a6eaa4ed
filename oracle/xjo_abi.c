/*
 * Oracle-side layout dump of include/xj_abi.h (test infrastructure only).
 * Lists sizeof/offsetof of every boundary field in the order
 * oracle/ref/ref_shim.c lists them for the reference headers
 * (src/xiaoju-pipe/core/xj_model.h:13-61, xj_stage.h:13-39); tests/test_abi.py
 * compares the two lists.
 */
#include "xjo.h"

#include <stddef.h>

#define OFF(T, f) (long)offsetof(T, f)

int xjo_abi_offsets(long *o, int max) {
    long v[] = {
        (long)sizeof(xj_w), OFF(xj_w, data), OFF(xj_w, file_off), OFF(xj_w, nbytes), OFF(xj_w, type), OFF(xj_w, ne0), OFF(xj_w, ne1),
        (long)sizeof(xj_layer), OFF(xj_layer, recurrent), OFF(xj_layer, attn_norm), OFF(xj_layer, post_norm), OFF(xj_layer, wqkv),
        OFF(xj_layer, wq), OFF(xj_layer, wk), OFF(xj_layer, wv), OFF(xj_layer, wo), OFF(xj_layer, q_norm), OFF(xj_layer, k_norm),
        OFF(xj_layer, ssm_qkv), OFF(xj_layer, ssm_gate), OFF(xj_layer, ssm_conv1d), OFF(xj_layer, ssm_dt), OFF(xj_layer, ssm_a),
        OFF(xj_layer, ssm_beta), OFF(xj_layer, ssm_alpha), OFF(xj_layer, ssm_norm), OFF(xj_layer, ssm_out),
        OFF(xj_layer, ffn_gate), OFF(xj_layer, ffn_up), OFF(xj_layer, ffn_down),
        (long)sizeof(xj_hparams), OFF(xj_hparams, n_layer), OFF(xj_hparams, n_embd), OFF(xj_hparams, n_ff), OFF(xj_hparams, n_vocab),
        OFF(xj_hparams, n_head), OFF(xj_hparams, n_head_kv), OFF(xj_hparams, head_dim), OFF(xj_hparams, n_rot),
        OFF(xj_hparams, rope_base), OFF(xj_hparams, eps), OFF(xj_hparams, conv_k), OFF(xj_hparams, d_inner), OFF(xj_hparams, s_k),
        OFF(xj_hparams, h_k), OFF(xj_hparams, h_v), OFF(xj_hparams, s_v), OFF(xj_hparams, key_dim), OFF(xj_hparams, conv_dim),
        OFF(xj_hparams, full_attn_interval), OFF(xj_hparams, eos), OFF(xj_hparams, eot),
        (long)sizeof(xj_model), OFF(xj_model, gguf), OFF(xj_model, hp), OFF(xj_model, tok_embd), OFF(xj_model, output_norm),
        OFF(xj_model, output), OFF(xj_model, layers), OFF(xj_model, fingerprint), OFF(xj_model, has_mtp), OFF(xj_model, mtp_eh),
        OFF(xj_model, mtp_enorm), OFF(xj_model, mtp_hnorm), OFF(xj_model, mtp_head_norm), OFF(xj_model, mtp_gguf),
        (long)sizeof(struct xj_stage), OFF(struct xj_stage, m), OFF(struct xj_stage, l0), OFF(struct xj_stage, l1),
        OFF(struct xj_stage, n_ctx), OFF(struct xj_stage, max_batch), OFF(struct xj_stage, n_past), OFF(struct xj_stage, has_head),
        OFF(struct xj_stage, mtp), OFF(struct xj_stage, backend), OFF(struct xj_stage, keep), OFF(struct xj_stage, ck_start),
        OFF(struct xj_stage, ck_T), OFF(struct xj_stage, forward), OFF(struct xj_stage, logits), OFF(struct xj_stage, rollback),
        OFF(struct xj_stage, reset), OFF(struct xj_stage, destroy), OFF(struct xj_stage, impl),
    };
    int n = (int)(sizeof v / sizeof v[0]);
    for (int i = 0; i < n && i < max; i++) o[i] = v[i];
    return n;
}
