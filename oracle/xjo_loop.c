/*
 * Oracle (test infrastructure only): the host token loop and the standalone
 * delta rule.
 *
 *   xjo_argmax          <- src/xiaoju-pipe/core/xj_spec.c:12-16 (strict >: first maximum wins)
 *   xjo_greedy          <- eval_once, no-remote branch, src/xiaoju-pipe/core/xj_net.c:532-559
 *                          (chunks of the smallest max_batch, logits of the last row only)
 *                          driven by the greedy loop of src/xiaoju-pipe/tools/xjpipe-host.c:131-144
 *   xjo_sample          <- the app's sampler, src/xiaoju-pipe/ios/App/XJGlue.c:251-282
 *                          (the uniform number passed in)
 *   xjo_utf8_emit       <- the app's emit, src/xiaoju-pipe/ios/App/XJGlue.c:285-305
 *                          (the callback replaced by an output buffer)
 *   xjo_delta_recurrent <- the per-head update of src/xiaoju-pipe/core/xj_cpu.c:203-213
 *                          (decay and beta are inputs instead of being derived from alpha/dt/A)
 *
 * Pinned by: token sequences of the reference pipeline compiled from source
 * (oracle/_ref, tests/golden/greedy_*.json) and, for the delta rule, by the
 * invariants of tests/test_oracle.py (decay=1,beta=0 keeps the state; beta=1
 * with orthonormal keys writes v exactly; linearity in v for a zero state).
 */
#include "xjo.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* The app's sampler (ios/App/XJGlue.c:251-282) with the uniform number
 * given as rand30 (< 2^30) in place of arc4random_uniform(1 << 30): greedy at
 * temp <= 0; otherwise the 40 largest values (the first of equal values kept),
 * sorted descending, p_i = exp((v_i - v_0) / temp) in double, cut where the
 * running share first reaches 0.95, pick with r = rand30 / 2^30 * kept mass. */
int xjo_sample(const float *lg, int n, float temp, uint32_t rand30) {
    int best = 0;
    for (int i = 1; i < n; i++) if (lg[i] > lg[best]) best = i;
    if (temp <= 0) return best;
    enum { K = 40 };
    int idx[K], k = 0, mi = 0;
    float val[K];
    for (int i = 0; i < n; i++) {
        const float v = lg[i];
        if (k < K) {
            idx[k] = i; val[k] = v;
            if (v < val[mi]) mi = k;
            k++;
        } else if (v > val[mi]) {
            idx[mi] = i; val[mi] = v;
            mi = 0;
            for (int j = 1; j < K; j++) if (val[j] < val[mi]) mi = j;
        }
    }
    for (int i = 0; i < k; i++)
        for (int j = i + 1; j < k; j++)
            if (val[j] > val[i]) { float tv = val[i]; val[i] = val[j]; val[j] = tv; int ti = idx[i]; idx[i] = idx[j]; idx[j] = ti; }
    double p[K], sum = 0;
    for (int i = 0; i < k; i++) { p[i] = exp((val[i] - val[0]) / temp); sum += p[i]; }
    double acc = 0;
    int cut = k;
    for (int i = 0; i < k; i++) { acc += p[i] / sum; if (acc >= 0.95) { cut = i + 1; break; } }
    double s2 = 0;
    for (int i = 0; i < cut; i++) s2 += p[i];
    double r = (double)rand30 / (double)(1u << 30) * s2;
    for (int i = 0; i < cut; i++) { r -= p[i]; if (r <= 0) return idx[i]; }
    return idx[0];
}

/* The app's sample_cb (ios/App/XJGlue.c:248) over a given stream of numbers:
 * each call with temp > 0 takes the next one (arc4random_uniform's place);
 * temp <= 0 takes none. Past the end of the stream the draw uses 0. */
int xjo_sampler_cb(void *ctx, const float *lg, int n) {
    xjo_sampler *s = (xjo_sampler *)ctx;
    uint32_t r = 0;
    if (s->temp > 0) {
        if (s->used < s->n) r = s->rand30[s->used];
        s->used++;
    }
    return xjo_sample(lg, n, s->temp, r);
}

/* The app's emit (ios/App/XJGlue.c:285-305): the held-back bytes, then at most
 * 256 bytes of the piece; from the end, skip up to 4 bytes of continuation
 * (10xxxxxx) to the last lead byte, whose sequence length (4 from 0xF0, 3 from
 * 0xE0, 2 from 0xC0, else 1) says whether its character is complete; an
 * incomplete one is held back for the next piece. */
int xjo_utf8_emit(xjo_utf8 *h, const char *s, int n, char *out) {
    int o = h->npending;
    memcpy(out, h->pending, (size_t)o);
    if (n > 256) n = 256;
    memcpy(out + o, s, (size_t)n);
    o += n;
    int ok = o;
    for (int back = 1; back <= 4 && back <= o; back++) {
        const unsigned char c = (unsigned char)out[o - back];
        if ((c & 0xC0) == 0x80) continue;
        const int need = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1;
        if (need > back) ok = o - back;
        break;
    }
    h->npending = o - ok;
    memcpy(h->pending, out + ok, (size_t)h->npending);
    return ok;
}

int xjo_argmax(const float *x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

static float second_best(const float *x, int n, int top) {
    float v = -INFINITY;
    for (int i = 0; i < n; i++)
        if (i != top && x[i] > v) v = x[i];
    return v;
}

/* embed -> every stage's forward -> head of the last stage, for n tokens */
static int eval_tokens(xj_stage **st, int ns, const int32_t *tok, int n, float *x, float *logits,
                       char *err, size_t errlen) {
    const xj_model *m = st[0]->m;
    const int E = m->hp.n_embd;
    int B = st[0]->max_batch;
    for (int i = 1; i < ns; i++) if (st[i]->max_batch < B) B = st[i]->max_batch;
    for (int i = 0; i < n; i += B) {
        const int T = n - i < B ? n - i : B;
        for (int t = 0; t < T; t++) xjo_embed(m, tok[i + t], x + (size_t)t * E);
        for (int k = 0; k < ns; k++)
            if (st[k]->forward(st[k], x, T, err, errlen)) return -1;
        if (i + T == n && st[ns - 1]->logits(st[ns - 1], x + (size_t)(T - 1) * E, 1, logits, err, errlen)) return -1;
    }
    return 0;
}

int xjo_greedy(xj_stage **st, int ns, const int32_t *prompt, int n_prompt, int n_gen, int32_t *out,
               float *margins, char *err, size_t errlen) {
    const xj_model *m = st[0]->m;
    const int V = m->hp.n_vocab;
    int B = st[0]->max_batch;
    for (int i = 1; i < ns; i++) if (st[i]->max_batch < B) B = st[i]->max_batch;
    float *x = malloc(sizeof(float) * (size_t)m->hp.n_embd * B);
    float *logits = malloc(sizeof(float) * (size_t)V);
    int rc = eval_tokens(st, ns, prompt, n_prompt, x, logits, err, errlen);
    for (int g = 0; g < n_gen && rc == 0; g++) {
        const int id = xjo_argmax(logits, V);
        out[g] = id;
        if (margins) margins[g] = logits[id] - second_best(logits, V, id);
        if (g + 1 < n_gen) rc = eval_tokens(st, ns, &out[g], 1, x, logits, err, errlen);
    }
    free(x);
    free(logits);
    return rc;
}

void xjo_delta_recurrent(int H, int S, int T, const float *q, const float *k, const float *v,
                         const float *decay, const float *beta, float qscale, float *state, float *out) {
#pragma omp parallel for schedule(static)
    for (int hh = 0; hh < H; hh++) {
        float *M = state + (size_t)hh * S * S;
        for (int t = 0; t < T; t++) {
            const size_t base = ((size_t)t * H + hh) * S;
            const float *qh = q + base, *kh = k + base, *vh = v + base;
            const float eg = decay[(size_t)t * H + hh], b = beta[(size_t)t * H + hh];
            for (int j = 0; j < S; j++) {
                float *row = M + (size_t)j * S;
                float sk = 0;
                for (int i = 0; i < S; i++) { row[i] *= eg; sk += row[i] * kh[i]; }
                const float delta = (vh[j] - sk) * b;
                float acc = 0;
                for (int i = 0; i < S; i++) { row[i] += kh[i] * delta; acc += row[i] * qh[i]; }
                out[base + j] = acc * qscale;
            }
        }
    }
}
