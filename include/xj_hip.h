/*
 * xj_hip.h - the MI355X (gfx950) backend for the xiaoju-pipe token loop.
 *
 * Three layers, all C ABI (plain pointers and sizes):
 *
 *  1. The drop-in stage. xj_hip_stage_new returns a `struct xj_stage` whose
 *     vtable behaves like the Metal stage it replaces, so the reference's
 *     pipeline (xj_pipeline_eval/verify/rollback) and speculative driver run
 *     on it unchanged.
 *       xj_hip_stage_new    <- xj_metal_stage_new  src/xiaoju-pipe/core/xj_stage.h:46-47
 *       xj_hip_device_name  <- xj_metal_device_name src/xiaoju-pipe/core/xj_stage.h:48
 *       xj_hip_tune_note    <- xj_metal_tune_note  src/xiaoju-pipe/core/xj_stage.h:50
 *
 *  2. Host-side counterparts of the reference loader, needed because the
 *     reference sources do not ship with this library. They carry the xjh_
 *     prefix so that a program linking the reference's own core objects next to
 *     this library sees no duplicate symbols; a model built by either loader
 *     can be passed to xj_hip_stage_new (the struct layout is the same):
 *       xjh_model_load / xjh_model_free <- xj_model_load / xj_model_free
 *                                          src/xiaoju-pipe/core/xj_model.h:64,69
 *       xjh_model_load_layers           <- xj_model_load_layers  xj_model.h:66
 *       xjh_model_attach_mtp            <- xj_model_attach_mtp   xj_model.h:72
 *       xjh_model_mtp_range             <- xj_model_mtp_range    xj_model.h:74
 *                                          (takes a path instead of a gguf_file)
 *       xjh_model_ranges                <- xj_model_ranges       xj_model.h:78
 *       xjh_model_layer_bytes           <- xj_model_layer_bytes  xj_model.h:80
 *       xjh_row_bytes / xjh_type_block  <- xj_row_bytes / xj_type_block
 *       / xjh_type_name                    / xj_type_name  src/xiaoju-pipe/core/gguf.h:81-83
 *     plus a writer for synthetic qwen35 GGUF files and the Q4_K / Q6_K /
 *     Q8_0 quantizers it uses (the reference has none for K-quants).
 *
 *  3. Device-resident extensions with no Metal counterpart: a chain of HIP
 *     stages that keeps the hidden state in HBM between stages, embeds token
 *     ids and takes the greedy argmax on the device, and replays one decode
 *     step as a HIP graph; a speculative driver with a separate draft model;
 *     and one C entry point per kernel (dequant, GEMV, norms, RoPE, attention,
 *     DeltaNet, argmax) used by the parity tests and the benchmark.
 *
 * Errors: every function that can fail returns -1 (or NULL) and writes a
 * message into err[errlen], as the reference does.
 */
#ifndef XJ_HIP_H
#define XJ_HIP_H

#include "xj_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- stage -- */

/* Same contract as xj_metal_stage_new (xj_stage.h:46-47, semantics
 * xj_metal.m:554-663): validates the layer range and weight mapping, copies
 * the weights of [l0,l1) (and the head when has_head) into HBM, allocates the
 * fp16 KV cache of every attention layer ([n_ctx][n_head_kv*head_dim]) and the
 * fp32 conv/recurrent state of every DeltaNet layer. backend = "hip".
 * With a model that has an MTP layer, [n_layer, n_layer + 1) builds the MTP
 * stage (mtp = true, xj_cpu.c:378-379): forward takes T rows of
 * [embedding | hidden] (2 n_embd floats each; the result, n_embd per row, is
 * written to the first T * n_embd floats), each half RMS-normalised with
 * nextn.enorm / nextn.hnorm and mapped back by nextn.eh_proj before the layer
 * (xj_cpu.c:253-261); its head normalises with nextn.shared_head_norm
 * (xj_cpu.c:287). */
xj_stage   *xj_hip_stage_new(const xj_model *m, int l0, int l1, int n_ctx, int max_batch,
                             bool has_head, char *err, size_t errlen);
const char *xj_hip_device_name(void);
const char *xj_hip_tune_note(void);

/* Bytes of HBM a stage holds besides the repacked weights
 * (counterpart of xj_stage_state_bytes, xj_stage.h:57). A single-stage
 * chain (xjh_chain_new) adds up to XJ_STAGE_SPLIT - 1 further sets of the
 * stage's scratch for prompts of several chunks: when it is built if
 * max_batch >= 16, else on the first such prompt. */
uint64_t    xj_hip_stage_state_bytes(const xj_model *m, int l0, int l1, int n_ctx, int max_batch);

/* Copy the whole recurrent state (conv + DeltaNet state of every layer) of a
 * HIP stage into snapshot slot `slot` (0 <= slot < 8), and restore it while
 * setting n_past. Lets a draft model roll back across separate T=1 calls,
 * which the reference's keep/rollback (one forward call only) cannot. */
int xj_hip_stage_snapshot(xj_stage *s, int slot, char *err, size_t errlen);
int xj_hip_stage_restore(xj_stage *s, int slot, int n_past, char *err, size_t errlen);
/* Test hook, no counterpart in the reference: fill every attention layer's K
 * and V cache from position pos0 to n_ctx with the fp16 pattern `bits`
 * (e.g. 0x7E00, a NaN), standing for stale memory that a decode step must
 * never read before writing it. */
int xj_hip_stage_fill_kv(xj_stage *s, int pos0, uint16_t bits, char *err, size_t errlen);

/* -------------------------------------------------------- host loader -- */

int         xjh_type_block(uint32_t type, int *block_bytes);
uint64_t    xjh_row_bytes(uint32_t type, int64_t n);
const char *xjh_type_name(uint32_t type);
/* The whole file mapped; the model table as xj_model_load builds it
 * (xj_model.c:129-209): hparams, layer pattern, tensors, tied head, eos/eot,
 * fingerprint, and the MTP layer in layers[n_layer] when the file has one. */
xj_model   *xjh_model_load(const char *path, char *err, size_t errlen);
void        xjh_model_free(xj_model *m);
/* Partial load for a stage of layers [l0, l1) (xj_model.c:214-233):
 * only the GGUF header is read, then one mapping spans the merged byte ranges
 * of those layers (with_io: also token_embd, output_norm, output). Tensors
 * outside the mapping keep data = NULL, so a stage over other layers fails
 * ("weights are not mapped"); the file may be a partial download as long as
 * it reaches the end of that span. Error for an empty or out-of-range [l0, l1). */
xj_model   *xjh_model_load_layers(const char *path, int l0, int l1, bool with_io, char *err, size_t errlen);
/* Attach the MTP layer of another GGUF of the same model (xj_model.c:275-300):
 * only its header and the MTP layer's byte span need to be present in that
 * file. No-op when m already has one; error when the shapes differ or the
 * file has no MTP layer. The mapping is released by xjh_model_free(m). */
int         xjh_model_attach_mtp(xj_model *m, const char *path, char *err, size_t errlen);
/* Byte span [lo, hi) of the MTP layer (layer tensors and nextn.*) of the
 * GGUF at path, from its header alone (xj_model.c:262-273). */
int         xjh_model_mtp_range(const char *path, uint64_t *lo, uint64_t *hi, char *err, size_t errlen);
/* Byte ranges [lo, hi) of the file that layers [l0, l1) (and with include_embd
 * the embedding, output norm and untied head) occupy, sorted, ranges at most
 * 4096 bytes apart merged; returns their count, at most max (xj_model.c:315-328). */
int         xjh_model_ranges(const xj_model *m, int l0, int l1, bool include_embd, uint64_t (*ranges)[2], int max);
/* Total tensor bytes of layers [l0, l1) (xj_model.c:330-338). */
uint64_t    xjh_model_layer_bytes(const xj_model *m, int l0, int l1);

/* --------------------------------------------------- synthetic models -- */

/* Shape and quantization recipe of a random-weight qwen35 model. Matrices are
 * N(0, w_std); norm weights 1 + 0.1 N; ssm_a = -exp(0.5 N); ssm_dt = 0.5 N;
 * conv1d 0.5 N. Every value is a pure function of (seed, tensor name, row). */
typedef struct {
    int n_layer, n_embd, n_ff, n_vocab;
    int n_head, n_head_kv, head_dim, n_rot;
    float rope_base, eps;
    int conv_k, s_k, h_k, h_v;          /* d_inner = h_v * s_k */
    int full_attn_interval;
    uint32_t type_default;              /* every matrix not named below */
    uint32_t type_embd, type_out, type_v, type_down;
    float w_std;
    uint64_t seed;
    int nextn;                          /* 1: one MTP layer (blk.{n_layer}, nextn.*) */
    int32_t eos_id;                     /* >= 0: tokenizer.ggml.eos_token_id */
    int32_t eot_id;                     /* >= 0: a token list with "<|im_end|>" at this id */
} xjs_config;

/* Fill out[n] with N(0, std) from the build's generator: splitmix64 feeding
 * Box-Muller in double, rounded to float. */
void xjs_fill_normal(float *out, int64_t n, uint64_t seed, float std);
/* Per-tensor seed = seed ^ FNV-1a(name). */
uint64_t xjs_tensor_seed(uint64_t seed, const char *name);
/* Quantize n_rows rows of k floats into `out` (row_bytes(type, k) each). */
int  xjs_quantize(uint32_t type, const float *x, int64_t n_rows, int64_t k, void *out,
                  char *err, size_t errlen);
/* Write a qwen35 GGUF v3 file for cfg; returns total bytes or -1. */
int64_t xjs_write_model(const char *path, const xjs_config *cfg, char *err, size_t errlen);

/* ------------------------------------------ device chain (fast path) -- */

typedef struct xjh_chain xjh_chain;

/* A chain runs HIP stages in sequence on one stream with the hidden state
 * kept in HBM; the last stage must have the head. Mirrors the no-remote branch
 * of eval_once (xj_net.c:541-559) with embedding and argmax on the device. */
xjh_chain *xjh_chain_new(xj_stage **stages, int n_stages, char *err, size_t errlen);
void       xjh_chain_free(xjh_chain *c);
/* Feed n tokens in chunks of max_batch. When nlog > 0 the logits of the last
 * min(nlog, rows) rows of the final chunk are computed: copied to `logits`
 * [nlog][n_vocab] when it is not NULL, and their greedy argmax (first maximum)
 * written to `argmax`. keep != 0 turns this call into a verify (xj_net.c:668):
 * all n tokens in one chunk, recurrent checkpoints kept for rollback. The
 * token the next decode step feeds is the last row's argmax or, with the
 * sampler on (xjh_chain_set_sampler), its draw (one number consumed). */
int  xjh_chain_eval(xjh_chain *c, const int32_t *tokens, int n, int nlog, int keep,
                    float *logits, int32_t *argmax, char *err, size_t errlen);
/* Up to n_steps steps entirely on the device. The first input token is the
 * one left by the previous eval/decode; out[i] receives the token chosen after
 * step i (so out[0] is the first step's argmax or, with the sampler on, its
 * draw with the next number). One step is one HIP graph launch. Generation stops at the model's end token
 * (hp.eos / hp.eot, xj_spec.c:29,139): it is the last token written and it is
 * not fed, so the state is that of the tokens before it. Returns the number of
 * tokens written (0 when the previous token already was an end token), or -1. */
int  xjh_chain_decode(xjh_chain *c, int n_steps, int32_t *out, char *err, size_t errlen);
/* The token that the next decode step would feed (the last argmax or draw). */
int  xjh_chain_last_token(xjh_chain *c);
/* The app's sampler on the device-resident path: with temperature > 0 every
 * token the chain produces - after xjh_chain_eval's last row, at each
 * xjh_chain_decode step, and the target's tokens in both speculative drivers -
 * is the draw of the app's top-k 40 / top-p 0.95 sampler from its logits row,
 * with the next of the n numbers rand30[] (each < 2^30) standing in for its
 * arc4random_uniform(1 << 30); numbers are consumed in order, one per token
 * produced, and a call that would need more than are left fails.
 * temperature <= 0 is greedy decoding (no number consumed, the app's rule).
 * Drafts stay greedy, as the reference's MTP drafts are. A chain reset keeps
 * the numbers and the count; this call restarts the count.
 * Replaces: the app's sample_cb passed to xj_spec_next
 * (src/xiaoju-pipe/ios/App/XJGlue.c:248-282, core/xj_spec.c:135,185). */
int  xjh_chain_set_sampler(xjh_chain *c, float temperature, const uint32_t *rand30, int n,
                           char *err, size_t errlen);
/* Numbers consumed since the last xjh_chain_set_sampler. */
int  xjh_chain_sampler_used(xjh_chain *c);
int  xjh_chain_rollback(xjh_chain *c, int n_past, char *err, size_t errlen);
void xjh_chain_reset(xjh_chain *c);
int  xjh_chain_n_past(xjh_chain *c);
/* Average GPU time of the last xjh_chain_decode, in ms per step, from HIP
 * events recorded on the chain's stream around the replayed graphs. */
double xjh_chain_last_decode_ms(xjh_chain *c);

/* Run only the GEMV launches of one T=1 decode step (same shapes and weights,
 * epilogues redirected to scratch so no state changes) `iters` times between
 * HIP events on the chain's stream. Reports the mean GPU ms per step, the
 * algorithmic HBM bytes of those launches per step, and the launch count. */
int  xjh_chain_time_gemv(xjh_chain *c, int iters, double *ms_per_step, double *bytes_per_step,
                         int *launches_per_step, char *err, size_t errlen);

/* Speculative decoding with a separate draft model (no reference
 * counterpart: the reference drafts with an MTP layer, xj_spec.c:131-209, and
 * the accept/rollback rule below is that function's). Each step feeds the
 * pending token t to the draft and lets it propose up to k tokens by greedy
 * T=1 steps, verifies [t, d1..dk] on the target in one batch, accepts the
 * longest prefix the target's token agrees with (its argmax, or with the
 * target's sampler on its draw, row i with the next number + i, so the output
 * is that of plain sampled decoding with the same numbers) and rolls both
 * models back. Greedy with k = 4, after rounds whose drafts were all
 * accepted, the draft makes the next round's drafts while the target
 * verifies (from the round's last draft: one step for the target's next
 * token, then k); they are used when the target accepts every draft and its
 * next token is the guessed one, so the tokens are those of the sequential
 * rounds (XJ_SPEC_PIPE=0: always sequential).
 * oracle (optional, n_oracle ids) replaces the drafts, with every
 * (g*7+j) % oracle_miss == 0 draft made wrong, as xj_spec.c:173-177; the
 * guess of the target's next token is then the oracle's. */
typedef struct {
    long n_steps, n_drafted, n_accepted;
    long acc_at[4];
    double t_total_ms, t_draft_ms;
    long n_overlap, n_overlap_held;   /* rounds drafted ahead during a verification; of them used */
} xjh_spec_stats;
/* Returns the number of tokens written to out (at most n_gen): generation
 * stops after an end token (hp.eos / hp.eot), which is written but not fed,
 * and an accepted end token cuts the accepted drafts there (xj_spec.c:139,
 * :193-194). -1 on error. */
int xjh_spec_generate(xjh_chain *target, xjh_chain *draft, int k, int n_gen,
                      const int32_t *oracle, int n_oracle, int oracle_miss,
                      int32_t *out, xjh_spec_stats *stats, char *err, size_t errlen);

/* Speculative decoding with the model's own MTP stage as the drafter, the
 * reference's algorithm (xj_spec.c:97-209, greedy or the chain's sampler: the MTP stage
 * takes every fed position with the token after it, drafts k <= 4 tokens, the
 * first from the pending positions and each further one from
 * [embedding(previous draft) | shared_head_norm(previous MTP output)]; the
 * target verifies [t, d1..dk] in one batch and keeps the agreeing prefix).
 * The target's hidden rows pass its output_norm before the MTP stage takes
 * them, and an MTP output passes shared_head_norm before it is fed back, both
 * as x * (sc * w) (the driver's defaults, XJ_MTP_MAIN_POST / XJ_MTP_CHAIN_POST
 * = 0 turn them off as in the reference).
 * Feeds the prompt itself (both models are reset first); out receives the
 * tokens of plain greedy decoding (with the target's sampler on: of plain
 * sampled decoding with the same numbers), end tokens handled as in xjh_spec_generate;
 * returns their count or -1. draft_log (optional) receives the first
 * draft_cap drafted tokens in order, before any oracle replacement. oracle /
 * oracle_miss as for xjh_spec_generate. mtp: xj_hip_stage_new(m, n_layer,
 * n_layer + 1, ..., has_head = true) of the target's model.
 * Replaces: xj_spec_feed / xj_spec_next with an MTP stage
 * (src/xiaoju-pipe/core/xj_spec.c:117-209) over the device chain. */
int xjh_spec_generate_mtp(xjh_chain *target, xj_stage *mtp, int k, const int32_t *prompt, int n_prompt,
                          int n_gen, const int32_t *oracle, int n_oracle, int oracle_miss,
                          int32_t *out, xjh_spec_stats *stats, int32_t *draft_log, int draft_cap,
                          char *err, size_t errlen);

/* ----------------------------------------------------- per-op kernels -- */

/* Device memory and stream helpers for tests and benchmarks. All per-op
 * entry points run on the library's own stream and return after the GPU
 * finished unless stated otherwise. */
void *xjh_malloc(size_t bytes);
void  xjh_free(void *p);
int   xjh_h2d(void *dst, const void *src, size_t bytes);
int   xjh_d2h(void *dst, const void *src, size_t bytes);
/* Device-to-device copy (the runtime's copy kernel): the known-size transfer
 * that calibrates the HBM byte counters of a profiler run. */
int   xjh_d2d(void *dst, const void *src, size_t bytes);
int   xjh_sync(void);
const char *xjh_last_error(void);

/* Repack a GGUF tensor (n_rows rows of k elements, GGUF block layout) into the
 * device layout the kernels read; returns the device pointer, NULL on error.
 * Q4_K and F32 keep the GGUF layout; Q6_K and Q8_0 are split into planes
 * (quants, high bits, scales, d) so every load is 16-byte aligned. */
void *xjh_upload_weight(uint32_t type, const void *host, int64_t n_rows, int64_t k,
                        char *err, size_t errlen);
/* Bit-exact dequantization of rows [r0, r0+n) of an uploaded weight into y. */
int xjh_dequant(uint32_t type, const void *dw, int64_t n_rows, int64_t k, int64_t r0, int64_t n,
                float *y, char *err, size_t errlen);
/* y[t][r] = W[r] . x[t] (add != 0: y += ...), T in 1..max, fp32 accumulate. */
int xjh_gemv(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T,
             float *y, int add, char *err, size_t errlen);
/* xjh_gemv without any allocation: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The same kernels and
 * results as xjh_gemv, bit for bit; the prepared activations go to a static
 * 1 MiB scratch array that each GPU holds from the library's load to the end
 * of the process, so T * (7.625 * k rounded up to 256 bytes) must fit in
 * 1 MiB (k = 9216: T <= 14), or the call fails with a message. Nothing in the
 * scratch needs to start at zero; every call on a GPU reuses that GPU's copy,
 * so calls that overlap on one GPU (other threads) race. The first call in a
 * process creates the library's stream, as every per-op entry does. */
int xjh_gemv_noalloc(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T,
                     float *y, int add, char *err, size_t errlen);
/* The same product for a prefill chunk on the matrix cores: Q4_K or Q6_K
 * rows, k % 256 == 0, T in 1..64. The activations enter as two f16 planes per
 * 256-element block (v * 2^-e = hi + lo) and the weights as integers exact in
 * f16, so every product is exact and only the fp32 accumulation rounds
 * (~1e-7 of the float64 product; xjh_gemv, with 21-bit activations, agrees
 * to ~1e-6). Counterpart of the Metal batched kernel mvb
 * (src/xiaoju-pipe/metal/xj_kernels.metal:84-388) for long batches. */
int xjh_gemm(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T,
             float *y, int add, char *err, size_t errlen);
/* Mean ms of xjh_gemm (prep launch included) over rotating copies, like xjh_gemv_time. */
double xjh_gemm_time(uint32_t type, void *const *dws, int n_copies, int64_t n_rows, int64_t k,
                     const float *x, int T, float *y, int iters, char *err, size_t errlen);
/* Time `iters` back-to-back launches of xjh_gemv over n_copies weights
 * (rotating, to defeat the caches), with HIP events on the library stream.
 * Returns the mean ms per launch, or -1. */
double xjh_gemv_time(uint32_t type, void *const *dws, int n_copies, int64_t n_rows, int64_t k,
                     const float *x, int T, float *y, int iters, char *err, size_t errlen);
/* out[t] = rmsnorm(x[t]) * w  (mode 0: x * sc * w, xj_cpu.c:56-61), x[t]/sqrt(sum x^2 + eps)
 * (mode 1, xj_cpu.c:185-193) or x * (sc * w) (mode 2, the speculative driver's norm_inplace,
 * xj_spec.c:19-25); sc = 1/sqrt(sum x^2 / n + eps) with the sum in double. */
int xjh_norm(int mode, const float *x, const float *w, int n, int rows, float eps, float *out,
             char *err, size_t errlen);
/* g[i] = silu(g[i]) * u[i] over n floats, in place.
 * Replaces: src/xiaoju-pipe/metal/xj_kernels.metal:591-600 (xj_swiglu);
 * CPU form xj_cpu.c:273. */
int xjh_swiglu(float *g, const float *u, int64_t n, char *err, size_t errlen);
/* NeoX RoPE in place: for token t < T and head h < n_heads, the pairs
 * (i, i + n_rot/2) of x + t*tok_stride + h*head_stride are rotated by
 * theta = (pos0 + t) * base^(-2i/n_rot) (cos and sin evaluated in float on the
 * host, as xj_cpu.c:68-77 does).
 * Replaces: src/xiaoju-pipe/metal/xj_kernels.metal:422-437 (xj_rope). */
int xjh_rope(float *x, int T, int n_heads, int64_t tok_stride, int64_t head_stride, int n_rot,
             int pos0, float base, char *err, size_t errlen);
/* Depthwise causal conv + SiLU in place over x [T][C] (kernel K in 2..8,
 * weights w [C][K], state [C][K-1] = the last K-1 inputs, oldest first,
 * carried across calls); ck (may be NULL when ck_n == 0) receives the state
 * after each of the first ck_n tokens, [ck_n][C][K-1]. The code is the qkv
 * GEMV's conv epilogue.
 * Replaces: src/xiaoju-pipe/metal/xj_kernels.metal:525-549 (xj_conv_silu);
 * CPU form xj_cpu.c:172-182. */
int xjh_conv_silu(float *x, float *state, const float *w, int C, int K, int T, float *ck, int ck_n,
                  char *err, size_t errlen);
/* Gated GQA attention of T new tokens at positions n_past .. n_past+T-1, after
 * the projections, through the token loop's own kernels: qg [T][H][2D]
 * (q | gate per head), k, v [T][Hkv*D] (raw projections); the new keys get
 * RMSNorm(k_norm) + RoPE and are stored with the values into the fp16 caches
 * kc, vc [n_ctx][Hkv*D] (IEEE half bits); out [T][H*D] = softmax(q'.K^T /
 * sqrt(D)) V * sigmoid(gate) with q' = RoPE(RMSNorm(q) * q_norm). D in
 * {64, 128, 256}, H/Hkv in {1, 2, 4, 8}.
 * Replaces: src/xiaoju-pipe/metal/xj_kernels.metal:439-523 (xj_kv_store,
 * xj_attn_scores, xj_softmax, xj_attn_out); CPU form xj_cpu.c:106-147. */
int xjh_attn_decode(int T, int H, int Hkv, int D, int n_rot, float rope_base, float eps, int n_past,
                    int n_ctx, const float *qg, const float *k, const float *v, const float *q_norm,
                    const float *k_norm, uint16_t *kc, uint16_t *vc, float *out,
                    char *err, size_t errlen);
/* T tokens of the DeltaNet recurrence after the conv, through the token
 * loop's own kernel: per token, q and k of each of the Hk key heads (at
 * qkv[t*qkv_stride + hk*S] and + k_off) are L2-normalised (double sum,
 * x / sqrt(sum + eps)), then value head hv (key head hv % Hk, values at
 * + v_off + hv*S) takes the gated delta rule with b = sigmoid(beta_raw[t][hv]),
 * decay exp(softplus(alpha_raw[t][hv] + dt[hv]) * A[hv]); out [T][Hv*S] =
 * (S_j . q) * qscale (before the gated norm). state [Hv][S][S] ([value j][key
 * i]) is updated; ck [ck_n][Hv][S][S] receives the state after each of the
 * first ck_n tokens (ck_n <= T). S in {64, 128}; state and ck 16-byte aligned.
 * Replaces: src/xiaoju-pipe/metal/xj_kernels.metal:552-589 (xj_delta_net,
 * with the L2 norms of xj_norm mode 1 applied inside); CPU form
 * xj_cpu.c:183-213, :218. */
int xjh_delta_step(const float *qkv, int qkv_stride, int k_off, int v_off, const float *beta_raw,
                   const float *alpha_raw, const float *dt, const float *A, int Hk, int Hv, int S, int T,
                   float eps, float qscale, float *state, float *out, float *ck, int ck_n,
                   char *err, size_t errlen);
/* One token per row of the device logits [T][n]: the app's sampler, top-k 40
 * then top-p 0.95 at `temperature` (p_i = exp((v_i - v_0) / temperature) in
 * double over the 40 largest, sorted descending), the pick made with
 * rand30[t] / 2^30 (host array, each below 2^30) in place of
 * arc4random_uniform(1 << 30); temperature <= 0: the first maximum.
 * Replaces: the app's `sample`, src/xiaoju-pipe/ios/App/XJGlue.c:251-282
 * (ties among the 40 values ordered by index). */
int xjh_sample(const float *logits, int n, int T, float temperature, const uint32_t *rand30,
               int32_t *out_host, char *err, size_t errlen);
/* UTF-8 piece streaming (host only): pieces of generated text go to cb only
 * as whole UTF-8 characters. xjh_utf8_emit appends piece (its first 256
 * bytes) to the bytes held back from earlier pieces, passes everything up to
 * an incomplete trailing character (judged from the last 4 bytes) to cb,
 * holds that character back and returns cb's result (0 when nothing is
 * passed). Replaces: the app's `emit`, src/xiaoju-pipe/ios/App/XJGlue.c:285-305,
 * with the state the app keeps in host_box (XJGlue.c:161) as its own struct;
 * xjh_piece_fn is xjg_piece_fn (XJGlue.h:12). */
typedef int (*xjh_piece_fn)(void *ctx, const char *utf8, int len);
typedef struct {
    char pending[8];
    int32_t npending;
} xjh_utf8_state;
void xjh_utf8_reset(xjh_utf8_state *st);
int xjh_utf8_emit(xjh_utf8_state *st, const char *piece, int n, xjh_piece_fn cb, void *ctx);
/* First index of the maximum of each of T rows of n floats. */
int xjh_argmax(const float *x, int n, int T, int32_t *out_host, char *err, size_t errlen);
/* Gated delta rule (standalone, decay and beta given per token and head):
 * state [H][S][S] ([head][value j][key i], as xj_cpu.c:203), q,k,v [T][H][S],
 * decay,beta [T][H], out [T][H][S]. o = S^T q * qscale after the update. */
int xjh_delta_recurrent(int H, int S, int T, const float *q, const float *k, const float *v,
                        const float *decay, const float *beta, float qscale,
                        float *state, float *out, char *err, size_t errlen);
/* The same recurrence evaluated chunk-wise (chunk tokens per chunk) with the
 * chunk-level products on MFMA; must agree with xjh_delta_recurrent. */
int xjh_delta_chunked(int H, int S, int T, int chunk, const float *q, const float *k,
                      const float *v, const float *decay, const float *beta, float qscale,
                      float *state, float *out, char *err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif /* XJ_HIP_H */
