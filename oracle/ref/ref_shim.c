/*
 * Checker-side shim around the reference's CPU path, compiled together with
 * the reference sources from /root/reference (never copied) into
 * oracle/_ref/libxjref.so by oracle/Makefile. It exposes the reference's own
 * static helpers (matmul, rmsnorm, rope from src/xiaoju-pipe/core/xj_cpu.c,
 * the decoders of xj_quant.h) and its greedy driver so the tests can compare
 * the oracle with the reference bit for bit. Test infrastructure only.
 */
#include "xj_cpu.c"   /* the reference translation unit itself, so its statics are reachable */
#include "xj_spec.h"

#include <stddef.h>

#define OFF(T, f) (long)offsetof(T, f)

void ref_dequant_row(uint32_t type, const void *src, float *y, int64_t n) { xj_dequant_row(type, src, y, n); }
uint16_t ref_to_f16(float f) { return xj_to_f16(f); }
float ref_f16(uint16_t h) { return xj_f16(h); }
uint64_t ref_row_bytes(uint32_t type, int64_t n) { return xj_row_bytes(type, n); }

void ref_matmul(uint32_t type, const void *w, int64_t K, int64_t N, const float *x, float *y, int T) {
    cpu_impl im;
    memset(&im, 0, sizeof im);
    int nt = 1;
#ifdef _OPENMP
    nt = omp_get_max_threads();
#endif
    im.rowbuf = malloc(sizeof(float) * (size_t)K * nt);
    xj_w ww;
    memset(&ww, 0, sizeof ww);
    ww.data = w; ww.type = type; ww.ne0 = K; ww.ne1 = N; ww.nbytes = xj_row_bytes(type, K) * (uint64_t)N;
    matmul(&im, &ww, x, y, T);
    free(im.rowbuf);
}

void ref_rmsnorm(float *out, const float *x, const float *w, int n, float eps) { rmsnorm(out, x, w, n, eps); }
void ref_rope(float *v, int n_rot, int pos, float base) { rope(v, n_rot, pos, base); }

xj_model *ref_model_load(const char *path, char *err, size_t errlen) { return xj_model_load(path, err, errlen); }
void ref_model_free(xj_model *m) { xj_model_free(m); }
xj_model *ref_model_load_layers(const char *path, int l0, int l1, bool with_io, char *err, size_t errlen) {
    return xj_model_load_layers(path, l0, l1, with_io, err, errlen);
}
int ref_model_ranges(const xj_model *m, int l0, int l1, bool io, uint64_t (*r)[2], int max) { return xj_model_ranges(m, l0, l1, io, r, max); }
int ref_model_attach_mtp(xj_model *m, const char *path, char *err, size_t errlen) { return xj_model_attach_mtp(m, path, err, errlen); }
int ref_model_mtp_range(const char *path, uint64_t *lo, uint64_t *hi, char *err, size_t errlen) {
    gguf_file *g = gguf_open_header(path, err, errlen);
    if (!g) return -1;
    const int rc = xj_model_mtp_range(g, lo, hi, err, errlen);
    gguf_close(g);
    return rc;
}
xj_stage *ref_stage_new(const xj_model *m, int l0, int l1, int n_ctx, int max_batch, bool has_head, char *err, size_t errlen) {
    return xj_cpu_stage_new(m, l0, l1, n_ctx, max_batch, has_head, err, errlen);
}
void ref_embed(const xj_model *m, int32_t tok, float *out) { xj_embed(m, tok, out); }

static int greedy_pick(void *ctx, const float *x, int n) {
    (void)ctx;
    int b = 0;
    for (int i = 1; i < n; i++) if (x[i] > x[b]) b = i;
    return b;
}

/* The reference's own driver (xj_pipeline + xj_spec with k = 0, as
 * xjpipe-host runs it) over CPU stages [0,split) and [split,L)+head. */
int ref_greedy(const xj_model *m, int split, int n_ctx, int max_batch, const int32_t *prompt, int n_prompt,
               int n_gen, int32_t *out, float *margins, char *err, size_t errlen) {
    const int L = m->hp.n_layer, V = m->hp.n_vocab;
    if (split <= 0 || split > L) split = L;
    xj_stage *a = xj_cpu_stage_new(m, 0, split, n_ctx, max_batch, split == L, err, errlen);
    xj_stage *b = split < L ? xj_cpu_stage_new(m, split, L, n_ctx, max_batch, true, err, errlen) : NULL;
    if (!a || (split < L && !b)) return -1;
    xj_pipeline p;
    xj_spec sp;
    int rc = xj_pipeline_init(&p, m, a, NULL, b) || xj_spec_init(&sp, &p, NULL, 0);
    if (!rc) rc = xj_spec_feed(&sp, prompt, n_prompt, err, errlen);
    for (int g = 0; g < n_gen && !rc; g++) {
        const float *lg = sp.last_logits;
        int top = greedy_pick(NULL, lg, V);
        float second = -INFINITY;
        for (int i = 0; i < V; i++) if (i != top && lg[i] > second) second = lg[i];
        if (margins) margins[g] = lg[top] - second;
        int32_t o[XJ_SPEC_MAXK + 1];
        int k = xj_spec_next(&sp, greedy_pick, NULL, o, n_gen - g, err, errlen);
        if (k != 1) { rc = -1; break; }
        out[g] = o[0];
    }
    xj_spec_free(&sp);
    xj_pipeline_free(&p);
    a->destroy(a);
    if (b) b->destroy(b);
    return rc ? -1 : 0;
}

/* A stage that forwards every call to `inner` and records the greedy token
 * of every logits row it returns: wrapped around the MTP stage, that is the
 * sequence of drafts the driver proposes (one logits call per draft,
 * xj_spec.c:157,170). */
typedef struct {
    struct xj_stage s;
    xj_stage *inner;
    int32_t *log;
    int cap, n;
} rec_stage;

static int rec_forward(xj_stage *s, float *x, int T, char *err, size_t errlen) {
    rec_stage *r = (rec_stage *)s;
    r->inner->keep = s->keep;
    const int rc = r->inner->forward(r->inner, x, T, err, errlen);
    s->n_past = r->inner->n_past; s->keep = r->inner->keep; s->ck_start = r->inner->ck_start; s->ck_T = r->inner->ck_T;
    return rc;
}
static int rec_logits(xj_stage *s, const float *x, int T, float *logits, char *err, size_t errlen) {
    rec_stage *r = (rec_stage *)s;
    const int rc = r->inner->logits(r->inner, x, T, logits, err, errlen);
    const int V = s->m->hp.n_vocab;
    for (int t = 0; !rc && t < T; t++)
        if (r->n < r->cap) r->log[r->n++] = greedy_pick(NULL, logits + (size_t)t * V, V);
    return rc;
}
static int rec_rollback(xj_stage *s, int n_past, char *err, size_t errlen) {
    rec_stage *r = (rec_stage *)s;
    const int rc = r->inner->rollback(r->inner, n_past, err, errlen);
    s->n_past = r->inner->n_past; s->ck_T = r->inner->ck_T;
    return rc;
}
static void rec_reset(xj_stage *s) {
    rec_stage *r = (rec_stage *)s;
    r->inner->reset(r->inner);
    s->n_past = r->inner->n_past;
}

static int is_end_tok(const xj_model *m, int32_t t) { return (uint32_t)t == m->hp.eot || (uint32_t)t == m->hp.eos; }

/* The reference's own speculative driver (xj_pipeline over stages a | b, the
 * MTP stage mtp drafting k tokens per step; mtp = NULL or k = 0: plain
 * greedy) over whatever stages it is given - the reference's CPU stages, the
 * oracle's, or the HIP library's through the same vtable. oracle/n_oracle
 * replace the drafts (the driver's test mode, xj_spec.h:37-38). Tokens into
 * out, ending after an end token as xjpipe-host's loop does
 * (tools/xjpipe-host.c:129-136; the end token is kept here); returns their
 * count. stats = {verify steps, drafted, accepted}; drafts (optional) gets the
 * MTP stage's proposals in order. */
int ref_spec_run_s(const xj_model *m, xj_stage *a, xj_stage *b, xj_stage *mtp, int k, const int32_t *prompt,
                   int n_prompt, int n_gen, const int32_t *oracle, int n_oracle, int oracle_miss, xj_sample_fn sample,
                   void *sctx, int32_t *out, long *stats, int32_t *drafts, int draft_cap, int *n_drafts, char *err,
                   size_t errlen);

int ref_spec_run(const xj_model *m, xj_stage *a, xj_stage *b, xj_stage *mtp, int k, const int32_t *prompt, int n_prompt,
                 int n_gen, const int32_t *oracle, int n_oracle, int oracle_miss, int32_t *out, long *stats,
                 int32_t *drafts, int draft_cap, int *n_drafts, char *err, size_t errlen) {
    return ref_spec_run_s(m, a, b, mtp, k, prompt, n_prompt, n_gen, oracle, n_oracle, oracle_miss, greedy_pick, NULL,
                          out, stats, drafts, draft_cap, n_drafts, err, errlen);
}

/* The same with the caller's sampler in place of the greedy pick (the app
 * passes its sample_cb here, ios/App/XJGlue.c:333). */
int ref_spec_run_s(const xj_model *m, xj_stage *a, xj_stage *b, xj_stage *mtp, int k, const int32_t *prompt,
                   int n_prompt, int n_gen, const int32_t *oracle, int n_oracle, int oracle_miss, xj_sample_fn sample,
                   void *sctx, int32_t *out, long *stats, int32_t *drafts, int draft_cap, int *n_drafts, char *err,
                   size_t errlen) {
    xj_pipeline p;
    xj_spec sp;
    rec_stage rec;
    memset(&rec, 0, sizeof rec);
    if (mtp) {
        rec.s = *mtp;
        rec.s.forward = rec_forward; rec.s.logits = rec_logits; rec.s.rollback = rec_rollback; rec.s.reset = rec_reset;
        rec.inner = mtp; rec.log = drafts; rec.cap = drafts ? draft_cap : 0;
    }
    int rc = xj_pipeline_init(&p, m, a, NULL, b) || xj_spec_init(&sp, &p, mtp ? &rec.s : NULL, k);
    if (rc) { snprintf(err, errlen, "pipeline / spec init failed"); return -1; }
    sp.oracle = oracle; sp.n_oracle = n_oracle; sp.oracle_miss = oracle_miss;
    rc = xj_spec_feed(&sp, prompt, n_prompt, err, errlen);
    int produced = 0, ended = 0;
    while (!rc && produced < n_gen && !ended) {
        int32_t o[XJ_SPEC_MAXK + 1];
        const int n = xj_spec_next(&sp, sample, sctx, o, n_gen - produced, err, errlen);
        if (n < 1) { rc = -1; break; }
        for (int i = 0; i < n && produced < n_gen && !ended; i++) {
            out[produced++] = o[i];
            ended = is_end_tok(m, o[i]);
        }
    }
    if (stats) { stats[0] = sp.n_steps; stats[1] = sp.n_drafted; stats[2] = sp.n_accepted; }
    if (n_drafts) *n_drafts = rec.n;
    xj_spec_free(&sp);
    xj_pipeline_free(&p);
    return rc ? -1 : produced;
}

/* offsetof every field of the boundary types, in a fixed order shared with
 * xjo_abi_offsets (oracle/xjo_abi.c, built from include/xj_abi.h) */
int ref_abi_offsets(long *o, int max) {
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
