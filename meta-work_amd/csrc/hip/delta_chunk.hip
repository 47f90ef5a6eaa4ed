// Chunk-wise gated delta rule (gfx950) - the prefill form of the recurrence
// S_t = a_t S_{t-1} + beta_t (v_t - a_t S_{t-1} k_t) k_t^T, o_t = S_t q_t * qscale
// (per head; state [value j][key i] as src/xiaoju-pipe/core/xj_cpu.c:203-213).
// The reference evaluates it token by token; this is the published chunk form
// (Yang, Kautz, Hatamizadeh, "Gated Delta Networks", ICLR 2025; Yang et al.,
// "Parallelizing Linear Transformers with the Delta Rule over Sequence Length",
// NeurIPS 2024), derived for this state orientation:
//   within a chunk of C tokens with start state M0 and lg_t = sum_{s<=t} log a_s,
//   delta = X (V - diag(e^lg) K M0^T),  X = (I + A)^-1 diag(beta),
//   A[s][r] = beta_s e^(lg_s - lg_r) k_s.k_r  (r < s)
//   O     = diag(e^lg) Q M0^T + P delta,  P[t][r] = e^(lg_t - lg_r) q_t.k_r (r <= t)
//   M_C   = e^lg_C M0 + delta^T diag(e^(lg_C - lg)) K
// Decay ratios are formed as exp of differences of cumulative logs, so 64
// steps of small decays never underflow a product.
//
// Phase 1 (all chunks and heads in parallel) builds W = X diag(e^lg) K,
// U = X V, P and the decay vectors; phase 2 walks the chunks in order, one
// work-group per (head, 16 value rows), since the value rows of the state are
// independent: delta = U - W M0^T, O, M_C.
#include "common.h"
#include "kernels.h"

namespace xjk {

constexpr int kC = 64;

template <int S>
struct WorkLayout {
    static constexpr int W = 0, U = kC * S, P = 2 * kC * S, GAM = 2 * kC * S + kC * kC, GEND = GAM + kC, GC = GEND + kC;
    static constexpr int SIZE = GC + 4;
};

template <int S>
__global__ __launch_bounds__(256) void dc_prep(int H, int T, const float *__restrict__ q, const float *__restrict__ k,
                                               const float *__restrict__ v, const float *__restrict__ decay,
                                               const float *__restrict__ beta, float *__restrict__ work) {
    using WL = WorkLayout<S>;
    const int n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    __shared__ float Ks[kC][S];
    __shared__ float AX[kC][kC + 1];
    __shared__ float lg[kC], bb[kC], gam[kC];
    __shared__ float rowtmp[kC];
    float *wk = work + ((int64_t)n * H + h) * WL::SIZE;
    for (int idx = tid; idx < kC * S; idx += 256) {
        const int t = idx / S, i = idx % S, tok = n * kC + t;
        Ks[t][i] = tok < T ? k[((int64_t)tok * H + h) * S + i] : 0.f;
    }
    if (tid < kC) {
        const int tok = n * kC + tid;
        lg[tid] = tok < T ? logf(decay[(int64_t)tok * H + h]) : 0.f;
        bb[tid] = tok < T ? beta[(int64_t)tok * H + h] : 0.f;
    }
    __syncthreads();
    if (tid == 0) {
        double acc = 0;
        for (int t = 0; t < kC; t++) { acc += lg[t]; lg[t] = (float)acc; }
    }
    __syncthreads();
    if (tid < kC) gam[tid] = expf(lg[tid]);
    // A (strictly lower) = beta_s e^(lg_s-lg_r) k_s.k_r
    for (int idx = tid; idx < kC * kC; idx += 256) {
        const int s = idx / kC, r = idx % kC;
        float a = 0.f;
        if (r < s) {
            float dsum = 0.f;
            for (int i = 0; i < S; i++) dsum = fmaf(Ks[s][i], Ks[r][i], dsum);
            a = bb[s] * expf(lg[s] - lg[r]) * dsum;
        }
        AX[s][r] = a;
    }
    __syncthreads();
    // X = (I + A)^-1 diag(beta), in place, row by row (unit lower triangular solve)
    for (int s = 0; s < kC; s++) {
        if (tid < kC) {
            const int r = tid;
            float x = 0.f;
            if (r < s) {
                for (int m = r; m < s; m++) x = fmaf(-AX[s][m], AX[m][r], x);
            } else if (r == s) {
                x = bb[s];
            }
            rowtmp[r] = x;
        }
        __syncthreads();
        if (tid < kC) AX[s][tid] = rowtmp[tid];
        __syncthreads();
    }
    // W = X diag(gam) K and U = X V
    for (int idx = tid; idx < kC * S; idx += 256) {
        const int s = idx / S, i = idx % S;
        float w = 0.f, u = 0.f;
        for (int r = 0; r <= s; r++) {
            const int tok = n * kC + r;
            const float vr = tok < T ? v[((int64_t)tok * H + h) * S + i] : 0.f;
            w = fmaf(AX[s][r] * gam[r], Ks[r][i], w);
            u = fmaf(AX[s][r], vr, u);
        }
        wk[WL::W + idx] = w;
        wk[WL::U + idx] = u;
    }
    // P[t][r] = e^(lg_t - lg_r) q_t . k_r for r <= t
    for (int idx = tid; idx < kC * kC; idx += 256) {
        const int t = idx / kC, r = idx % kC, tok = n * kC + t;
        float p = 0.f;
        if (r <= t && tok < T) {
            const float *qt = q + ((int64_t)tok * H + h) * S;
            float dsum = 0.f;
            for (int i = 0; i < S; i++) dsum = fmaf(qt[i], Ks[r][i], dsum);
            p = expf(lg[t] - lg[r]) * dsum;
        }
        wk[WL::P + idx] = p;
    }
    if (tid < kC) {
        wk[WL::GAM + tid] = gam[tid];
        wk[WL::GEND + tid] = expf(lg[kC - 1] - lg[tid]);
    }
    if (tid == 0) wk[WL::GC] = gam[kC - 1];
}

template <int S>
__global__ __launch_bounds__(256) void dc_scan(int H, int T, const float *__restrict__ q, const float *__restrict__ k,
                                               const float *__restrict__ work, float qscale, float *__restrict__ state,
                                               float *__restrict__ out) {
    using WL = WorkLayout<S>;
    constexpr int JB = 16;
    const int h = blockIdx.x, j0 = blockIdx.y * JB, tid = threadIdx.x;
    __shared__ float Mb[JB][S + 4];
    __shared__ float dl[kC][JB + 1];
    for (int idx = tid; idx < JB * S; idx += 256) Mb[idx / S][idx % S] = state[((int64_t)h * S + j0 + idx / S) * S + idx % S];
    __syncthreads();
    const int nch = (T + kC - 1) / kC;
    const int jj = tid % JB, sg = tid / JB;   // (row group, value row) for delta and O
    for (int n = 0; n < nch; n++) {
        const float *wk = work + ((int64_t)n * H + h) * WL::SIZE;
        for (int s = sg; s < kC; s += 256 / JB) {
            const float *Wr = wk + WL::W + s * S;
            float d = 0.f;
            for (int i = 0; i < S; i++) d = fmaf(Wr[i], Mb[jj][i], d);
            dl[s][jj] = wk[WL::U + s * S + j0 + jj] - d;
        }
        __syncthreads();
        for (int t = sg; t < kC; t += 256 / JB) {
            const int tok = n * kC + t;
            if (tok >= T) continue;
            const float *qt = q + ((int64_t)tok * H + h) * S;
            float a = 0.f;
            for (int i = 0; i < S; i++) a = fmaf(qt[i], Mb[jj][i], a);
            float o = wk[WL::GAM + t] * a;
            const float *Pr = wk + WL::P + t * kC;
            for (int r = 0; r <= t; r++) o = fmaf(Pr[r], dl[r][jj], o);
            out[((int64_t)tok * H + h) * S + j0 + jj] = o * qscale;
        }
        __syncthreads();
        const float gC = wk[WL::GC];
        for (int idx = tid; idx < JB * S; idx += 256) {
            const int r0 = idx / S, i = idx % S;
            float m = gC * Mb[r0][i];
            for (int r = 0; r < kC; r++) {
                const int tok = n * kC + r;
                const float kr = tok < T ? k[((int64_t)tok * H + h) * S + i] : 0.f;
                m = fmaf(wk[WL::GEND + r] * dl[r][r0], kr, m);
            }
            Mb[r0][i] = m;
        }
        __syncthreads();
    }
    for (int idx = tid; idx < JB * S; idx += 256) state[((int64_t)h * S + j0 + idx / S) * S + idx % S] = Mb[idx / S][idx % S];
}

size_t delta_chunked_work_bytes(int H, int S, int T, int chunk) {
    if (chunk != kC || T < 1 || H < 1) return 0;
    const int64_t nch = (T + kC - 1) / kC;
    if (S == 128) return (size_t)nch * H * WorkLayout<128>::SIZE * 4;
    if (S == 64) return (size_t)nch * H * WorkLayout<64>::SIZE * 4;
    return 0;
}

int delta_chunked_launch(int H, int S, int T, int chunk, const float *q, const float *k, const float *v,
                         const float *decay, const float *beta, float qscale, float *state, float *out, float *work,
                         hipStream_t st) {
    if (chunk != kC) return -1;
    const int nch = (T + kC - 1) / kC;
    if (S == 128) {
        hipLaunchKernelGGL(dc_prep<128>, dim3(nch, H), dim3(256), 0, st, H, T, q, k, v, decay, beta, work);
        hipLaunchKernelGGL(dc_scan<128>, dim3(H, 128 / 16), dim3(256), 0, st, H, T, q, k, work, qscale, state, out);
    } else if (S == 64) {
        hipLaunchKernelGGL(dc_prep<64>, dim3(nch, H), dim3(256), 0, st, H, T, q, k, v, decay, beta, work);
        hipLaunchKernelGGL(dc_scan<64>, dim3(H, 64 / 16), dim3(256), 0, st, H, T, q, k, work, qscale, state, out);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
