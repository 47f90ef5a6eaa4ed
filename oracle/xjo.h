/*
 * xjo.h - the oracle: a CPU restatement of the reference's token loop, used
 * ONLY as the checker by tests/, __graft_entry__.smoke() and the CPU-baseline
 * leg of bench.py. Nothing in the product links or calls it.
 *
 *   xjo_f16 / xjo_to_f16 / xjo_dequant_row  <- src/xiaoju-pipe/core/xj_quant.h:9-122
 *   xjo_matmul, xjo_rmsnorm, xjo_rope,       <- src/xiaoju-pipe/core/xj_cpu.c:36-77
 *   xjo_attn_decode                          <- src/xiaoju-pipe/core/xj_cpu.c:106-147 (attention
 *                                               after the projections; the oracle stage uses it)
 *   xjo_stage_new (forward/logits/rollback/  <- src/xiaoju-pipe/core/xj_cpu.c:83-418
 *     reset/destroy, embed)
 *   xjo_greedy                               <- src/xiaoju-pipe/core/xj_net.c:532-559 (no-remote
 *                                               eval) + src/xiaoju-pipe/tools/xjpipe-host.c:17-18,131-144
 *   xjo_delta_recurrent                      <- the delta rule of src/xiaoju-pipe/core/xj_cpu.c:196-213
 *                                               with decay and beta passed in directly
 *
 * kv_f16 != 0 rounds every K/V value through fp16 (round to nearest even) when
 * it is stored, as the Metal backend's cache does (xj_kernels.metal:440-452);
 * kv_f16 == 0 is the reference CPU path's own fp32 cache (xj_cpu.c:411-412).
 *
 * How each part is pinned: see the module header of each .c file and the
 * tests that compare it with the reference compiled from source (oracle/_ref)
 * and with the committed golden vectors in tests/golden/.
 */
#ifndef XJO_H
#define XJO_H

#include "../include/xj_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

float    xjo_f16(uint16_t h);
uint16_t xjo_to_f16(float f);
uint64_t xjo_row_bytes(uint32_t type, int64_t n);
void     xjo_dequant_row(uint32_t type, const void *src, float *y, int64_t n);
/* y[t][r] = dot(dequant(W[r]), x[t]); OpenMP over rows. */
void     xjo_matmul(uint32_t type, const void *w, int64_t K, int64_t N, const float *x, float *y, int T);
void     xjo_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void     xjo_l2norm(float *x, int n, float eps);
void     xjo_rope(float *v, int n_rot, int pos, float base);
void     xjo_embed(const xj_model *m, int32_t token, float *out);

xj_stage *xjo_stage_new(const xj_model *m, int l0, int l1, int n_ctx, int max_batch, bool has_head,
                        int kv_f16, char *err, size_t errlen);

/* Greedy decoding through stages[0..n_stages) (the last has the head):
 * prefill `prompt` in chunks of the smallest max_batch, then produce n_gen
 * tokens: out[0] = argmax of the prompt's last logits, out[i] = argmax after
 * feeding out[i-1]. margins[i] (optional) = top-1 minus top-2 logit. */
int xjo_greedy(xj_stage **stages, int n_stages, const int32_t *prompt, int n_prompt, int n_gen,
               int32_t *out, float *margins, char *err, size_t errlen);

/* First index of the maximum (strict >), xj_spec.c:12-16. */
int xjo_argmax(const float *x, int n);

/* The app's top-k 40 / top-p 0.95 sampler (ios/App/XJGlue.c:251-282), the
 * uniform number rand30 / 2^30 passed in. */
int xjo_sample(const float *lg, int n, float temp, uint32_t rand30);
/* The app's sample_cb over a stream of numbers (rand30[used++] per draw at
 * temp > 0), for the reference's own driver (xj_sample_fn). */
typedef struct {
    float temp;
    const uint32_t *rand30;
    int n, used;
} xjo_sampler;
int xjo_sampler_cb(void *ctx, const float *lg, int n);
/* The app's UTF-8 piece streaming (ios/App/XJGlue.c:285-305): piece (its first
 * 256 bytes) after the held-back bytes; the bytes up to an incomplete trailing
 * character go to *out (returned count), that character is held back. */
typedef struct { char pending[8]; int npending; } xjo_utf8;
int xjo_utf8_emit(xjo_utf8 *h, const char *s, int n, char *out);
/* One token of the causal depthwise conv + SiLU (xj_cpu.c:172-182), x and
 * state [C][KC-1] updated in place. */
void xjo_conv_silu(int C, int KC, float *x, const float *w, float *state);
/* One token of L2 norms + the gated delta rule over all value heads
 * (xj_cpu.c:183-213); q, k normalised in place, ck may be NULL. */
void xjo_delta_step(int Hk, int Hv, int S, float eps, float qscale, float *q, float *k, const float *v,
                    const float *beta_raw, const float *alpha_raw, const float *dt, const float *A, float *state,
                    float *out, float *ck);
/* g = silu(g) * u (xj_cpu.c:273). */
void xjo_swiglu(size_t n, float *g, const float *u);
/* Gated GQA attention after the projections (xj_cpu.c:106-147); see attn_core. */
void xjo_attn_decode(int T, int H, int Hkv, int D, int n_rot, float base, float eps, int n_past, int kv_f16,
                     const float *qg, float *k, const float *v, const float *qnw, const float *knw,
                     float *kc, float *vc, float *att);

void xjo_delta_recurrent(int H, int S, int T, const float *q, const float *k, const float *v,
                         const float *decay, const float *beta, float qscale, float *state, float *out);

#ifdef __cplusplus
}
#endif
#endif
