/*
 * Oracle (test infrastructure only): the reference CPU stage restated.
 *
 *   xjo_matmul        <- src/xiaoju-pipe/core/xj_cpu.c:36-54  row dequant + sequential fp32 dot
 *   xjo_rmsnorm       <- xj_cpu.c:56-61    double sum, x*sc*w
 *   xjo_rope          <- xj_cpu.c:68-77    NeoX pairs (i, i+n_rot/2), theta in fp32
 *   attn_full         <- xj_cpu.c:83-151   gated GQA: q|gate interleaved per head
 *   xjo_attn_decode   <- xj_cpu.c:106-147  its part after the projections (attn_core)
 *   xjo_conv_silu     <- xj_cpu.c:172-182  one token of the causal conv + SiLU
 *   xjo_swiglu        <- xj_cpu.c:273
 *   xjo_delta_step    <- xj_cpu.c:183-213  one token of L2 norms + the gated delta rule
 *   attn_linear       <- xj_cpu.c:155-223  conv+SiLU, L2(q,k), gated delta rule, gated RMSNorm
 *   ensure_ck         <- xj_cpu.c:228-242
 *   stage_forward     <- xj_cpu.c:244-280
 *   stage_logits      <- xj_cpu.c:282-291
 *   stage_rollback    <- xj_cpu.c:293-319
 *   stage_reset       <- xj_cpu.c:321-330
 *   xjo_embed         <- xj_cpu.c:369-373
 *   xjo_stage_new     <- xj_cpu.c:375-418  (the MTP stage included: prologue xj_cpu.c:253-261,
 *                                           head norm xj_cpu.c:287)
 *
 * Every floating-point expression keeps the reference's shape and order so
 * that, built with the reference's flags (-O3 -fopenmp, GNU C, fp-contract
 * fast), it rounds exactly as the reference does. Pinned bit-for-bit against
 * oracle/_ref (the reference compiled from source) by tests/test_oracle.py and
 * by the committed end-to-end vectors in tests/golden/.
 */
#include "xjo.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    float *kc, *vc;         /* attention: [n_ctx][n_head_kv*head_dim] */
    float *conv, *ssm;      /* DeltaNet: [conv_dim][conv_k-1], [h_v][s_v][s_k] */
    float *ck_conv, *ck_ssm;
} olayer;

typedef struct {
    olayer *ls;
    float *h, *a, *b, *c, *d, *g, *u;   /* scratch, max_batch * scratch_floats each */
    float *rowbuf;                       /* one dequantized row per thread */
    int nthreads, n_ck, kv_f16;
} ostage;

static int max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int thread_id(void) {
#ifdef _OPENMP
    return omp_get_thread_num();
#else
    return 0;
#endif
}

static void matmul_buf(float *rowbuf, uint32_t type, const void *w, int64_t K, int64_t N,
                       const float *x, float *y, int T) {
    const uint64_t rb = xjo_row_bytes(type, K);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < N; r++) {
        float *buf = rowbuf + (size_t)thread_id() * K;
        xjo_dequant_row(type, (const uint8_t *)w + r * rb, buf, K);
        for (int t = 0; t < T; t++) {
            const float *xt = x + (size_t)t * K;
            float s = 0;
            for (int64_t k = 0; k < K; k++) s += buf[k] * xt[k];
            y[(size_t)t * N + r] = s;
        }
    }
}

void xjo_matmul(uint32_t type, const void *w, int64_t K, int64_t N, const float *x, float *y, int T) {
    float *rowbuf = malloc(sizeof(float) * (size_t)K * max_threads());
    matmul_buf(rowbuf, type, w, K, N, x, y, T);
    free(rowbuf);
}

static void mm(ostage *o, const xj_w *w, const float *x, float *y, int T) {
    matmul_buf(o->rowbuf, w->type, w->data, w->ne0, w->ne1, x, y, T);
}

void xjo_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float sc = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * sc * (w ? w[i] : 1.0f);
}

void xjo_l2norm(float *x, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float sc = 1.0f / sqrtf((float)ss + eps);
    for (int i = 0; i < n; i++) x[i] *= sc;
}

static inline float silu(float v) { return v / (1.0f + expf(-v)); }
static inline float sigm(float v) { return 1.0f / (1.0f + expf(-v)); }
static inline float softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

void xjo_rope(float *v, int n_rot, int pos, float base) {
    const int half = n_rot / 2;
    for (int i = 0; i < half; i++) {
        const float theta = pos * powf(base, -2.0f * i / n_rot);
        const float c = cosf(theta), s = sinf(theta);
        const float x0 = v[i], x1 = v[i + half];
        v[i] = x0 * c - x1 * s;
        v[i + half] = x0 * s + x1 * c;
    }
}

static const float *F32(const xj_w *w) { return (const float *)w->data; }


/* The part of attn_full after the projections (xj_cpu.c:106-147): key
 * norm + RoPE + store of each new key/value at n_past + t (rounded through
 * fp16 when kv_f16), then for every token and query head the query norm +
 * RoPE, softmax(q.K^T * scale) V over positions 0..n_past+t, times
 * sigmoid(gate). qg [T][H][2D] (q | gate per head), k, v [T][Hkv][D] (k is
 * normalised and rotated in place), caches [n_ctx][Hkv*D], att [T][H][D]. */
static void attn_core(int T, int H, int Hkv, int D, int n_rot, float base, float eps, int n_past, int kv_f16,
                      const float *qg, float *k, const float *v, const float *qnw, const float *knw,
                      float *kc, float *vc, float *att) {
    const int nq = 2 * H * D, nk = Hkv * D;
    const float scale = 1.0f / sqrtf((float)D);
    /* normalise + rotate the new keys and append the batch to the cache first,
     * so token t of the batch sees tokens 0..t of it */
    for (int t = 0; t < T; t++) {
        const int pos = n_past + t;
        float *kt = k + (size_t)t * nk;
        const float *vt = v + (size_t)t * nk;
        for (int g = 0; g < Hkv; g++) {
            xjo_rmsnorm(kt + g * D, kt + g * D, knw, D, eps);
            xjo_rope(kt + g * D, n_rot, pos, base);
        }
        float *kd = kc + (size_t)pos * nk, *vd = vc + (size_t)pos * nk;
        for (int e = 0; e < nk; e++) {
            kd[e] = kv_f16 ? xjo_f16(xjo_to_f16(kt[e])) : kt[e];
            vd[e] = kv_f16 ? xjo_f16(xjo_to_f16(vt[e])) : vt[e];
        }
    }

#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; t++) {
        for (int hh = 0; hh < H; hh++) {
            const int pos = n_past + t, kvh = hh / (H / Hkv);
            float q[1024];
            const float *qr = qg + (size_t)t * nq + (size_t)hh * 2 * D;
            xjo_rmsnorm(q, qr, qnw, D, eps);
            xjo_rope(q, n_rot, pos, base);
            float *sc = malloc(sizeof(float) * (size_t)(pos + 1));
            float mx = -INFINITY;
            for (int j = 0; j <= pos; j++) {
                const float *kj = kc + (size_t)j * nk + (size_t)kvh * D;
                float dsum = 0;
                for (int i = 0; i < D; i++) dsum += q[i] * kj[i];
                sc[j] = dsum * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double sum = 0;
            for (int j = 0; j <= pos; j++) { sc[j] = expf(sc[j] - mx); sum += sc[j]; }
            float *oh = att + (size_t)t * H * D + (size_t)hh * D;
            for (int i = 0; i < D; i++) oh[i] = 0;
            for (int j = 0; j <= pos; j++) {
                const float *vj = vc + (size_t)j * nk + (size_t)kvh * D;
                const float p = (float)(sc[j] / sum);
                for (int i = 0; i < D; i++) oh[i] += p * vj[i];
            }
            free(sc);
            const float *gate = qr + D;
            for (int i = 0; i < D; i++) oh[i] *= sigm(gate[i]);
        }
    }
}

void xjo_attn_decode(int T, int H, int Hkv, int D, int n_rot, float base, float eps, int n_past, int kv_f16,
                     const float *qg, float *k, const float *v, const float *qnw, const float *knw,
                     float *kc, float *vc, float *att) {
    attn_core(T, H, Hkv, D, n_rot, base, eps, n_past, kv_f16, qg, k, v, qnw, knw, kc, vc, att);
}

static void attn_full(xj_stage *s, ostage *o, int il, const float *h, float *out, int T) {
    const xj_hparams *hp = &s->m->hp;
    const xj_layer *L = &s->m->layers[il];
    olayer *st = &o->ls[il - s->l0];
    const int D = hp->head_dim, H = hp->n_head, Hkv = hp->n_head_kv;
    const int nq = 2 * H * D, nk = Hkv * D;
    float *qg = o->a, *k = o->b, *v = o->c, *att = o->d;

    if (L->wqkv.nbytes) {
        float *qkv = o->g;
        mm(o, &L->wqkv, h, qkv, T);
        for (int t = 0; t < T; t++) {
            const float *r = qkv + (size_t)t * (nq + 2 * nk);
            memcpy(qg + (size_t)t * nq, r, sizeof(float) * nq);
            memcpy(k + (size_t)t * nk, r + nq, sizeof(float) * nk);
            memcpy(v + (size_t)t * nk, r + nq + nk, sizeof(float) * nk);
        }
    } else {
        mm(o, &L->wq, h, qg, T);
        mm(o, &L->wk, h, k, T);
        mm(o, &L->wv, h, v, T);
    }

    attn_core(T, H, Hkv, D, hp->n_rot, hp->rope_base, hp->eps, s->n_past, o->kv_f16, qg, k, v, F32(&L->q_norm),
              F32(&L->k_norm), st->kc, st->vc, att);
    mm(o, &L->wo, att, out, T);
}

/* Causal depthwise conv of one token + SiLU (xj_cpu.c:172-182): for each of
 * the C channels the window is the KC-1 stored inputs (state [C][KC-1],
 * oldest first) followed by x[c]; the state shifts by one and keeps x[c];
 * x[c] becomes silu(window . w[c][0..KC-1]). */
void xjo_conv_silu(int C, int KC, float *x, const float *w, float *state) {
    for (int c = 0; c < C; c++) {
        float *cs = state + (size_t)c * (KC - 1);
        const float *wc = w + (size_t)c * KC;
        float acc = 0;
        for (int kk = 0; kk < KC - 1; kk++) acc += cs[kk] * wc[kk];
        acc += x[c] * wc[KC - 1];
        for (int kk = 0; kk < KC - 2; kk++) cs[kk] = cs[kk + 1];
        cs[KC - 2] = x[c];
        x[c] = silu(acc);
    }
}

/* One token of the gated delta rule over all value heads (xj_cpu.c:183-213,
 * after the conv): q and k of every key head L2-normalised in place
 * (xj_cpu.c:185-193), then value head hv (key head hv % Hk) with
 * b = sigmoid(beta_raw[hv]), eg = exp(softplus(alpha_raw[hv] + dt[hv]) * A[hv]):
 *   row_j <- row_j * eg; delta_j = (v_j - row_j . k) * b;
 *   row_j <- row_j + k * delta_j; out_j = (row_j . q) * qscale
 * over the state [Hv][S (value j)][S (key i)]. ck (may be NULL) receives the
 * state after the token. */
void xjo_delta_step(int Hk, int Hv, int S, float eps, float qscale, float *q, float *k, const float *v,
                    const float *beta_raw, const float *alpha_raw, const float *dt, const float *A, float *state,
                    float *out, float *ck) {
    for (int g = 0; g < Hk; g++) {
        xjo_l2norm(q + g * S, S, eps);
        xjo_l2norm(k + g * S, S, eps);
    }
#pragma omp parallel for schedule(static)
    for (int hv = 0; hv < Hv; hv++) {
        const int hk = hv % Hk;
        const float *qh = q + hk * S, *kh = k + hk * S, *vh = v + hv * S;
        const float b = sigm(beta_raw[hv]);
        const float g = softplus(alpha_raw[hv] + dt[hv]) * A[hv];
        const float eg = expf(g);
        float *M = state + (size_t)hv * S * S;
        float *oh = out + hv * S;
        for (int j = 0; j < S; j++) {
            float *row = M + (size_t)j * S;
            float sk = 0;
            for (int i = 0; i < S; i++) { row[i] *= eg; sk += row[i] * kh[i]; }
            const float delta = (vh[j] - sk) * b;
            float acc = 0;
            for (int i = 0; i < S; i++) { row[i] += kh[i] * delta; acc += row[i] * qh[i]; }
            oh[j] = acc * qscale;
        }
        if (ck) memcpy(ck + (size_t)hv * S * S, M, sizeof(float) * S * S);
    }
}

/* g[i] = silu(g[i]) * u[i] (xj_cpu.c:273). */
void xjo_swiglu(size_t n, float *g, const float *u) {
    for (size_t i = 0; i < n; i++) g[i] = silu(g[i]) * u[i];
}

static void attn_linear(xj_stage *s, ostage *o, int il, const float *h, float *out, int T) {
    const xj_hparams *hp = &s->m->hp;
    const xj_layer *L = &s->m->layers[il];
    olayer *st = &o->ls[il - s->l0];
    const int CD = hp->conv_dim, KC = hp->conv_k, Hv = hp->h_v, Hk = hp->h_k, S = hp->s_k;
    float *qkv = o->a, *z = o->b, *beta = o->c, *alpha = o->d, *ob = o->g;

    mm(o, &L->ssm_qkv, h, qkv, T);
    mm(o, &L->ssm_gate, h, z, T);
    mm(o, &L->ssm_beta, h, beta, T);
    mm(o, &L->ssm_alpha, h, alpha, T);

    const float *cw = F32(&L->ssm_conv1d), *dt = F32(&L->ssm_dt), *A = F32(&L->ssm_a), *nw = F32(&L->ssm_norm);
    const float qscale = 1.0f / sqrtf((float)S);

    for (int t = 0; t < T; t++) {
        float *x = qkv + (size_t)t * CD;
        xjo_conv_silu(CD, KC, x, cw, st->conv);
        float *ot = ob + (size_t)t * hp->d_inner;
        const int ck = s->keep && t < T - 1;
        xjo_delta_step(Hk, Hv, S, hp->eps, qscale, x, x + hp->key_dim, x + 2 * hp->key_dim, beta + (size_t)t * Hv,
                       alpha + (size_t)t * Hv, dt, A, st->ssm, ot, ck ? st->ck_ssm + (size_t)t * Hv * S * S : NULL);
#pragma omp parallel for schedule(static)
        for (int hv = 0; hv < Hv; hv++) {
            float *oh = ot + hv * S;
            const float *zh = z + (size_t)t * hp->d_inner + hv * S;
            xjo_rmsnorm(oh, oh, nw, S, hp->eps);
            for (int j = 0; j < S; j++) oh[j] *= silu(zh[j]);
        }
        if (ck) memcpy(st->ck_conv + (size_t)t * CD * (KC - 1), st->conv, sizeof(float) * CD * (KC - 1));
    }
    mm(o, &L->ssm_out, ob, out, T);
}

static int ensure_ck(xj_stage *s, int n, char *err, size_t errlen) {
    ostage *o = s->impl;
    const xj_hparams *hp = &s->m->hp;
    if (n <= o->n_ck) return 0;
    for (int il = s->l0; il < s->l1; il++) {
        olayer *st = &o->ls[il - s->l0];
        if (!st->ssm) continue;
        free(st->ck_conv);
        free(st->ck_ssm);
        st->ck_conv = malloc(sizeof(float) * n * hp->conv_dim * (hp->conv_k - 1));
        st->ck_ssm = malloc(sizeof(float) * n * hp->h_v * hp->s_v * hp->s_k);
        if (!st->ck_conv || !st->ck_ssm) { snprintf(err, errlen, "out of memory for checkpoints"); o->n_ck = 0; return -1; }
    }
    o->n_ck = n;
    return 0;
}

static int stage_forward(xj_stage *s, float *x, int T, char *err, size_t errlen) {
    ostage *o = s->impl;
    const xj_hparams *hp = &s->m->hp;
    const int E = hp->n_embd;
    if (T <= 0 || T > s->max_batch) { snprintf(err, errlen, "%d tokens exceed max_batch %d", T, s->max_batch); s->keep = 0; return -1; }
    if (s->n_past + T > s->n_ctx) { snprintf(err, errlen, "context full (%d)", s->n_ctx); s->keep = 0; return -1; }
    if (s->keep && ensure_ck(s, T - 1, err, errlen)) { s->keep = 0; return -1; }
    s->ck_start = s->n_past;
    s->ck_T = s->keep ? T : 0;
    if (s->mtp) {
        /* x holds [embedding | hidden] per token: each half RMS-normalised with its
         * own weights, then eh_proj back to n_embd (xj_cpu.c:253-261) */
        const xj_model *m = s->m;
        for (int t = 0; t < T; t++) {
            xjo_rmsnorm(o->h + (size_t)t * 2 * E, x + (size_t)t * 2 * E, F32(&m->mtp_enorm), E, hp->eps);
            xjo_rmsnorm(o->h + (size_t)t * 2 * E + E, x + (size_t)t * 2 * E + E, F32(&m->mtp_hnorm), E, hp->eps);
        }
        mm(o, &m->mtp_eh, o->h, x, T);
    }
    for (int il = s->l0; il < s->l1; il++) {
        const xj_layer *L = &s->m->layers[il];
        for (int t = 0; t < T; t++) xjo_rmsnorm(o->h + (size_t)t * E, x + (size_t)t * E, F32(&L->attn_norm), E, hp->eps);
        if (L->recurrent) attn_linear(s, o, il, o->h, o->u, T);
        else attn_full(s, o, il, o->h, o->u, T);
        for (size_t i = 0; i < (size_t)T * E; i++) x[i] += o->u[i];
        for (int t = 0; t < T; t++) xjo_rmsnorm(o->h + (size_t)t * E, x + (size_t)t * E, F32(&L->post_norm), E, hp->eps);
        mm(o, &L->ffn_gate, o->h, o->g, T);
        mm(o, &L->ffn_up, o->h, o->a, T);
        xjo_swiglu((size_t)T * hp->n_ff, o->g, o->a);
        mm(o, &L->ffn_down, o->g, o->u, T);
        for (size_t i = 0; i < (size_t)T * E; i++) x[i] += o->u[i];
    }
    s->n_past += T;
    s->keep = 0;
    return 0;
}

static int stage_logits(xj_stage *s, const float *x, int T, float *logits, char *err, size_t errlen) {
    ostage *o = s->impl;
    const int E = s->m->hp.n_embd;
    if (!s->has_head) { snprintf(err, errlen, "this stage has no output head"); return -1; }
    if (T < 1 || T > s->max_batch) { snprintf(err, errlen, "head called with %d tokens", T); return -1; }
    const xj_w *nw = s->mtp ? &s->m->mtp_head_norm : &s->m->output_norm;   /* xj_cpu.c:287 */
    for (int t = 0; t < T; t++) xjo_rmsnorm(o->h + (size_t)t * E, x + (size_t)t * E, F32(nw), E, s->m->hp.eps);
    mm(o, &s->m->output, o->h, logits, T);
    return 0;
}

static int stage_rollback(xj_stage *s, int n_past, char *err, size_t errlen) {
    ostage *o = s->impl;
    const xj_hparams *hp = &s->m->hp;
    if (n_past == s->n_past) { s->ck_T = 0; return 0; }
    int recurrent = 0;
    for (int il = s->l0; il < s->l1; il++) recurrent |= o->ls[il - s->l0].ssm != NULL;
    if (!recurrent) {
        if (n_past < 0 || n_past > s->n_past) { snprintf(err, errlen, "cannot roll back to %d", n_past); return -1; }
        s->n_past = n_past;
        return 0;
    }
    const int j = n_past - s->ck_start - 1;
    if (!s->ck_T || s->n_past != s->ck_start + s->ck_T || j < 0 || j >= s->ck_T - 1) {
        snprintf(err, errlen, "cannot roll back to %d (checkpoints %d+%d, now %d)", n_past, s->ck_start, s->ck_T, s->n_past);
        return -1;
    }
    const size_t nc = (size_t)hp->conv_dim * (hp->conv_k - 1), ns = (size_t)hp->h_v * hp->s_v * hp->s_k;
    for (int il = s->l0; il < s->l1; il++) {
        olayer *st = &o->ls[il - s->l0];
        if (!st->ssm) continue;
        memcpy(st->conv, st->ck_conv + (size_t)j * nc, nc * 4);
        memcpy(st->ssm, st->ck_ssm + (size_t)j * ns, ns * 4);
    }
    s->n_past = n_past;
    s->ck_T = 0;
    return 0;
}

static void stage_reset(xj_stage *s) {
    ostage *o = s->impl;
    const xj_hparams *hp = &s->m->hp;
    for (int il = s->l0; il < s->l1; il++) {
        olayer *st = &o->ls[il - s->l0];
        if (st->conv) memset(st->conv, 0, sizeof(float) * hp->conv_dim * (hp->conv_k - 1));
        if (st->ssm) memset(st->ssm, 0, sizeof(float) * hp->h_v * hp->s_v * hp->s_k);
    }
    s->n_past = 0;
}

static void stage_destroy(xj_stage *s) {
    if (!s) return;
    ostage *o = s->impl;
    if (o) {
        if (o->ls)
            for (int i = 0; i < s->l1 - s->l0; i++) {
                free(o->ls[i].kc); free(o->ls[i].vc); free(o->ls[i].conv); free(o->ls[i].ssm);
                free(o->ls[i].ck_conv); free(o->ls[i].ck_ssm);
            }
        free(o->ls);
        free(o->h); free(o->a); free(o->b); free(o->c); free(o->d); free(o->g); free(o->u);
        free(o->rowbuf);
        free(o);
    }
    free(s);
}

static size_t scratch_floats(const xj_hparams *hp) {
    size_t n = (size_t)hp->n_ff;
    const size_t qkv = 2 * (size_t)hp->n_head * hp->head_dim + 2 * (size_t)hp->n_head_kv * hp->head_dim;
    if (qkv > n) n = qkv;
    if ((size_t)hp->conv_dim > n) n = (size_t)hp->conv_dim;
    if ((size_t)hp->n_embd * 2 > n) n = 2 * (size_t)hp->n_embd;
    return n;
}

void xjo_embed(const xj_model *m, int32_t token, float *out) {
    const xj_w *w = &m->tok_embd;
    if (token < 0 || token >= w->ne1) { memset(out, 0, sizeof(float) * w->ne0); return; }
    xjo_dequant_row(w->type, (const uint8_t *)w->data + (uint64_t)token * xjo_row_bytes(w->type, w->ne0), out, w->ne0);
}

xj_stage *xjo_stage_new(const xj_model *m, int l0, int l1, int n_ctx, int max_batch, bool has_head,
                        int kv_f16, char *err, size_t errlen) {
    const xj_hparams *hp = &m->hp;
    const bool mtp = m->has_mtp && l0 == hp->n_layer && l1 == hp->n_layer + 1;   /* xj_cpu.c:378-379 */
    if (l0 < 0 || (l1 > hp->n_layer && !mtp) || l0 > l1) { snprintf(err, errlen, "bad layer range [%d,%d)", l0, l1); return NULL; }
    if (hp->head_dim > 1024) { snprintf(err, errlen, "head_dim too large"); return NULL; }
    for (int il = l0; il < l1; il++)
        if (!m->layers[il].ffn_down.data) { snprintf(err, errlen, "layer %d weights are not mapped", il); return NULL; }
    if (has_head && !m->output.data) { snprintf(err, errlen, "output head is not mapped"); return NULL; }
    xj_stage *s = calloc(1, sizeof(*s));
    ostage *o = calloc(1, sizeof(*o));
    s->m = m; s->l0 = l0; s->l1 = l1; s->n_ctx = n_ctx; s->max_batch = max_batch; s->has_head = has_head;
    s->mtp = mtp;
    s->backend = kv_f16 ? "cpu-oracle-kvf16" : "cpu-oracle";
    s->forward = stage_forward; s->logits = stage_logits; s->rollback = stage_rollback;
    s->reset = stage_reset; s->destroy = stage_destroy;
    s->impl = o;
    o->kv_f16 = kv_f16;
    o->nthreads = max_threads();
    const size_t sf = scratch_floats(hp) * (size_t)max_batch;
    o->h = malloc(sf * 4); o->a = malloc(sf * 4); o->b = malloc(sf * 4); o->c = malloc(sf * 4);
    o->d = malloc(sf * 4); o->g = malloc(sf * 4); o->u = malloc(sf * 4);
    int64_t maxk = 2 * (int64_t)hp->n_embd;
    if (hp->n_ff > maxk) maxk = hp->n_ff;
    if (hp->d_inner > maxk) maxk = hp->d_inner;
    if ((int64_t)hp->n_head * hp->head_dim > maxk) maxk = (int64_t)hp->n_head * hp->head_dim;
    o->rowbuf = malloc(sizeof(float) * maxk * o->nthreads);
    o->ls = calloc(l1 - l0 ? l1 - l0 : 1, sizeof(olayer));
    for (int il = l0; il < l1; il++) {
        olayer *st = &o->ls[il - l0];
        if (m->layers[il].recurrent) {
            st->conv = calloc((size_t)hp->conv_dim * (hp->conv_k - 1), 4);
            st->ssm = calloc((size_t)hp->h_v * hp->s_v * hp->s_k, 4);
        } else {
            st->kc = malloc((size_t)n_ctx * hp->n_head_kv * hp->head_dim * 4);
            st->vc = malloc((size_t)n_ctx * hp->n_head_kv * hp->head_dim * 4);
            if (!st->kc || !st->vc) { snprintf(err, errlen, "KV cache allocation failed"); stage_destroy(s); return NULL; }
        }
    }
    if (!o->h || !o->rowbuf) { snprintf(err, errlen, "out of memory"); stage_destroy(s); return NULL; }
    return s;
}
