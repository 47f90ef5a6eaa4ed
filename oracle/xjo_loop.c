/*
 * Oracle (test infrastructure only): the host token loop and the standalone
 * delta rule.
 *
 *   xjo_argmax          <- src/xiaoju-pipe/core/xj_spec.c:12-16 (strict >: first maximum wins)
 *   xjo_greedy          <- eval_once, no-remote branch, src/xiaoju-pipe/core/xj_net.c:532-559
 *                          (chunks of the smallest max_batch, logits of the last row only)
 *                          driven by the greedy loop of src/xiaoju-pipe/tools/xjpipe-host.c:131-144
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
