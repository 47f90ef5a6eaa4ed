/*
 * xj_abi.h - the data types the xiaoju-pipe token loop passes across its
 * backend boundary, restated field for field so that a stage built by this
 * library can be handed to the reference's pipeline and speculative driver
 * unchanged.
 *
 * Every struct below must keep the field order, types and padding of the
 * reference declaration it mirrors; tests/test_abi.py compares offsetof() of
 * every field against the reference headers when they are available.
 *
 *   xj_type          <- src/xiaoju-pipe/core/gguf.h:13-17   (ggml type ids)
 *   xj_w             <- src/xiaoju-pipe/core/xj_model.h:13-19
 *   xj_layer         <- src/xiaoju-pipe/core/xj_model.h:21-31
 *   xj_hparams       <- src/xiaoju-pipe/core/xj_model.h:33-46
 *   xj_model         <- src/xiaoju-pipe/core/xj_model.h:48-61
 *   struct xj_stage  <- src/xiaoju-pipe/core/xj_stage.h:13-39
 *
 * gguf_file is only ever used through a pointer here, so it stays an
 * incomplete type (the reference's loader owns its definition).
 */
#ifndef XJ_ABI_H
#define XJ_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (gguf.h:13-17). */
enum xj_type {
    XJ_F32 = 0, XJ_F16 = 1, XJ_Q4_0 = 2, XJ_Q4_1 = 3, XJ_Q5_0 = 6, XJ_Q5_1 = 7,
    XJ_Q8_0 = 8, XJ_Q2_K = 10, XJ_Q3_K = 11, XJ_Q4_K = 12, XJ_Q5_K = 13, XJ_Q6_K = 14,
    XJ_BF16 = 30,
};

#define XJ_MAX_LAYERS 128

typedef struct xj_gguf_file gguf_file;

/* One weight: `data` points into the host mapping of the GGUF file.
 * ne0 = input length of a row, ne1 = number of rows. */
typedef struct {
    const void *data;
    uint64_t    file_off;
    uint64_t    nbytes;
    uint32_t    type;
    int64_t     ne0, ne1;
} xj_w;

typedef struct {
    bool recurrent;          /* true: Gated DeltaNet, false: gated GQA */
    xj_w attn_norm, post_norm;
    xj_w wqkv;               /* optional fused q|k|v */
    xj_w wq, wk, wv, wo, q_norm, k_norm;
    xj_w ssm_qkv, ssm_gate, ssm_conv1d, ssm_dt, ssm_a, ssm_beta, ssm_alpha, ssm_norm, ssm_out;
    xj_w ffn_gate, ffn_up, ffn_down;
} xj_layer;

typedef struct {
    int   n_layer, n_embd, n_ff, n_vocab;
    int   n_head, n_head_kv, head_dim;
    int   n_rot;
    float rope_base, eps;
    int   conv_k;
    int   d_inner;
    int   s_k;
    int   h_k, h_v;
    int   s_v;
    int   key_dim, conv_dim;
    int   full_attn_interval;
    uint32_t eos, eot;
} xj_hparams;

typedef struct {
    gguf_file *gguf;
    xj_hparams hp;
    xj_w tok_embd, output_norm, output;
    xj_layer layers[XJ_MAX_LAYERS];
    uint64_t fingerprint;
    bool has_mtp;
    xj_w mtp_eh, mtp_enorm, mtp_hnorm, mtp_head_norm;
    gguf_file *mtp_gguf;
} xj_model;

typedef struct xj_stage xj_stage;

/* A contiguous range of layers [l0, l1) behind a five-entry vtable.
 * forward: x is caller-owned host memory [T][n_embd], overwritten in place.
 * logits : x [T][n_embd] -> logits [T][n_vocab], host memory.
 * All calls are synchronous and return 0 or -1 with a message in err. */
struct xj_stage {
    const xj_model *m;
    int l0, l1;
    int n_ctx;
    int max_batch;
    int n_past;
    bool has_head;
    bool mtp;
    const char *backend;
    int keep;
    int ck_start, ck_T;
    int  (*forward)(xj_stage *s, float *x, int T, char *err, size_t errlen);
    int  (*logits)(xj_stage *s, const float *x, int T, float *logits, char *err, size_t errlen);
    int  (*rollback)(xj_stage *s, int n_past, char *err, size_t errlen);
    void (*reset)(xj_stage *s);
    void (*destroy)(xj_stage *s);
    void *impl;
};

#ifdef __cplusplus
}
#endif
#endif /* XJ_ABI_H */
