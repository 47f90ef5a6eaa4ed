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
// Every chunk-level dense product runs on the matrix cores in fp32
// (v_mfma_f32_16x16x4f32: fp32 products, fp32 sums). Phase 1 (all chunks and
// heads in parallel) forms K K^T and Q K^T, solves for X (one wavefront, row
// by row with its column of X in registers, while the others finish P from
// the chunk's q, k and v staged in LDS), then W = X diag(e^lg) K and U = X V.
// Phase 2 walks the chunks in order, one work-group per (head, 16 value rows)
// since the value rows of the state are independent: delta = U - W M0^T, O,
// M_C.
#include "common.h"
#include "kernels.h"

namespace xjk {

constexpr int kC = 64;
typedef float v4f __attribute__((ext_vector_type(4)));

// D (16x16) += A (16x4) B (4x16) on the matrix cores. Lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; element r of lane l is D[4*(l/16) + r][l%16].
// Tiles below walk an inner dimension in blocks of 16: lane group l/16 takes
// inner indices 16b + 4*(l/16) + s, s = 0..3 (one MFMA per s).
__device__ __forceinline__ v4f mma(v4f c, float a, float b) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f ld4(const float *p) { return *(const v4f *)p; }

template <int S>
struct WorkLayout {
    static constexpr int W = 0, U = kC * S, P = 2 * kC * S, GAM = 2 * kC * S + kC * kC, GEND = GAM + kC, GC = GEND + kC;
    static constexpr int SIZE = GC + 4;
};

template <int S>
constexpr size_t prep_lds_bytes() { return (size_t)(3 * kC * (S + 4) + kC * (kC + 4)) * 4; }
template <int S>
constexpr size_t scan_lds_bytes() { return (size_t)((16 + kC) * (S + 4) + kC * 20) * 4; }

template <int S>
__global__ __launch_bounds__(256) void dc_prep(int H, int T, const float *__restrict__ q, const float *__restrict__ k,
                                               const float *__restrict__ v, const float *__restrict__ decay,
                                               const float *__restrict__ beta, float *__restrict__ work) {
    using WL = WorkLayout<S>;
    constexpr int KS = S + 4, XS = kC + 4;   // LDS row strides (floats)
    extern __shared__ __align__(16) float sm[];
    float *Ks = sm;                // [kC][KS] the chunk's k rows (zero past T)
    float *Vs = Ks + kC * KS;      // [kC][KS] v rows
    float *Qs = Vs + kC * KS;      // [kC][KS] q rows
    float *AX = Qs + kC * KS;      // [kC][XS] A, then X
    __shared__ float lg[kC], bb[kC];
    __shared__ __align__(16) float gam[kC];
    const int n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, l = tid & 63, lr = l & 15, lq = l >> 4;
    float *wk = work + ((int64_t)n * H + h) * WL::SIZE;
    for (int idx = tid; idx < kC * S / 4; idx += 256) {
        const int t = idx / (S / 4), c = 4 * (idx % (S / 4)), tok = n * kC + t;
        v4f kv = {0.f, 0.f, 0.f, 0.f}, vv = kv, qv = kv;
        if (tok < T) {
            kv = ld4(k + ((int64_t)tok * H + h) * S + c);
            vv = ld4(v + ((int64_t)tok * H + h) * S + c);
            qv = ld4(q + ((int64_t)tok * H + h) * S + c);
        }
        *(v4f *)(Ks + t * KS + c) = kv;
        *(v4f *)(Vs + t * KS + c) = vv;
        *(v4f *)(Qs + t * KS + c) = qv;
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
    // A (strictly lower) = beta_s e^(lg_s - lg_r) k_s.k_r: wavefront w takes
    // rows 16w..16w+15, tiles on and below the diagonal
    for (int J = 0; J < 4; J++) {
        v4f kk = {0.f, 0.f, 0.f, 0.f};
        if (J <= w) {
            for (int b = 0; b < S / 16; b++) {
                const int c = 16 * b + 4 * lq;
                const v4f ka = ld4(Ks + (16 * w + lr) * KS + c), kb = ld4(Ks + (16 * J + lr) * KS + c);
#pragma unroll
                for (int s = 0; s < 4; s++) kk = mma(kk, ka[s], kb[s]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int s_ = 16 * w + 4 * lq + r, r_ = 16 * J + lr;
            AX[s_ * XS + r_] = r_ < s_ ? bb[s_] * expf(lg[s_] - lg[r_]) * kk[r] : 0.f;
        }
    }
    __syncthreads();
    if (w == 0) {
        // X = (I + A)^-1 diag(beta) by forward substitution, row by row: lane l
        // owns column l, held in registers (X[s][l] = beta_s [l == s] - sum over
        // m < s of A[s][m] X[m][l]; X is lower triangular), A's rows read as
        // broadcasts, four partial sums per row; then X replaces A in LDS.
        // (row s + 1 of A is requested while row s is computed; the two row
        // buffers alternate with the parity of s, eight partial sums per row)
        float xc[kC];
        v4f arow[2][kC / 4];
#pragma unroll
        for (int s = 0; s < kC; s++) {
            if (s + 1 < kC) {
#pragma unroll
                for (int j = 0; 4 * j < s + 1; j++) arow[(s + 1) & 1][j] = ld4(AX + (s + 1) * XS + 4 * j);
            }
            float pp[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < s; m++) pp[m & 7] = fmaf(-arow[s & 1][m / 4][m & 3], xc[m], pp[m & 7]);
            const float x = ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
            xc[s] = l < s ? x : l == s ? bb[s] : 0.f;
        }
#pragma unroll
        for (int s = 0; s < kC; s++) AX[s * XS + l] = xc[s];    } else {
        // P[t][r] = e^(lg_t - lg_r) q_t.k_r for r <= t (zero elsewhere and past T):
        // the 10 tiles on and below the diagonal over wavefronts 1..3
        for (int tile = w - 1; tile < 16; tile += 3) {
            const int I = tile / 4, J = tile % 4;
            v4f qk = {0.f, 0.f, 0.f, 0.f};
            if (J <= I) {
                for (int b = 0; b < S / 16; b++) {
                    const int c = 16 * b + 4 * lq;
                    const v4f a4 = ld4(Qs + (16 * I + lr) * KS + c);   // zero past T
                    const v4f kb = ld4(Ks + (16 * J + lr) * KS + c);
#pragma unroll
                    for (int s = 0; s < 4; s++) qk = mma(qk, a4[s], kb[s]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t_ = 16 * I + 4 * lq + r, r_ = 16 * J + lr;
                wk[WL::P + t_ * kC + r_] = r_ <= t_ && n * kC + t_ < T ? expf(lg[t_] - lg[r_]) * qk[r] : 0.f;
            }
        }
    }
    __syncthreads();
    // W = X diag(gam) K and U = X V: wavefront w takes key/value column blocks
    // w, w + 4, ...; X is lower triangular, so row block I needs inner blocks <= I
    for (int J = w; J < S / 16; J += 4) {
        for (int I = 0; I < 4; I++) {
            v4f aw = {0.f, 0.f, 0.f, 0.f}, au = aw;
            for (int b = 0; b <= I; b++) {
                const int c = 16 * b + 4 * lq;
                const v4f xa = ld4(AX + (16 * I + lr) * XS + c), g = ld4(gam + c);
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    aw = mma(aw, xa[s] * g[s], Ks[(c + s) * KS + 16 * J + lr]);
                    au = mma(au, xa[s], Vs[(c + s) * KS + 16 * J + lr]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int s_ = 16 * I + 4 * lq + r, i_ = 16 * J + lr;
                wk[WL::W + s_ * S + i_] = aw[r];
                wk[WL::U + s_ * S + i_] = au[r];
            }
        }
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
    constexpr int JB = 16, KS = S + 4, DS = JB + 4;
    extern __shared__ __align__(16) float sm[];
    float *Mb = sm;                // [JB][KS] state rows j0..j0+15 (value) x key
    float *Kc = Mb + JB * KS;      // [kC][KS] the chunk's k rows (zero past T)
    float *dl = Kc + kC * KS;      // [kC][DS] delta[s][j]
    const int h = blockIdx.x, j0 = blockIdx.y * JB, tid = threadIdx.x;
    const int w = tid >> 6, l = tid & 63, lr = l & 15, lq = l >> 4;
    for (int idx = tid; idx < JB * S / 4; idx += 256) {
        const int j = idx / (S / 4), c = 4 * (idx % (S / 4));
        *(v4f *)(Mb + j * KS + c) = ld4(state + ((int64_t)h * S + j0 + j) * S + c);
    }
    const int nch = (T + kC - 1) / kC;
    for (int n = 0; n < nch; n++) {
        const float *wk = work + ((int64_t)n * H + h) * WL::SIZE;
        for (int idx = tid; idx < kC * S / 4; idx += 256) {
            const int t = idx / (S / 4), c = 4 * (idx % (S / 4)), tok = n * kC + t;
            *(v4f *)(Kc + t * KS + c) = tok < T ? ld4(k + ((int64_t)tok * H + h) * S + c) : v4f{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();   // M0 (first chunk) and this chunk's k rows in place
        // delta = U - W M0^T: wavefront w takes rows 16w..16w+15
        {
            v4f acc = {0.f, 0.f, 0.f, 0.f};
            const float *Wr = wk + WL::W + (16 * w + lr) * S;
            for (int b = 0; b < S / 16; b++) {
                const int c = 16 * b + 4 * lq;
                const v4f wa = ld4(Wr + c), mb = ld4(Mb + lr * KS + c);
#pragma unroll
                for (int s = 0; s < 4; s++) acc = mma(acc, wa[s], mb[s]);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int s_ = 16 * w + 4 * lq + r;
                dl[s_ * DS + lr] = wk[WL::U + s_ * S + j0 + lr] - acc[r];
            }
        }
        __syncthreads();
        // O = diag(gam) Q M0^T + P delta: wavefront w takes tokens 16w..16w+15
        {
            v4f aq = {0.f, 0.f, 0.f, 0.f}, ap = aq;
            const int tokA = n * kC + 16 * w + lr;
            const float *qa = q + ((int64_t)tokA * H + h) * S;
            for (int b = 0; b < S / 16; b++) {
                const int c = 16 * b + 4 * lq;
                const v4f a4 = tokA < T ? ld4(qa + c) : v4f{0.f, 0.f, 0.f, 0.f};
                const v4f mb = ld4(Mb + lr * KS + c);
#pragma unroll
                for (int s = 0; s < 4; s++) aq = mma(aq, a4[s], mb[s]);
            }
            const float *Pr = wk + WL::P + (16 * w + lr) * kC;
            for (int b = 0; b <= w; b++) {   // P is zero above the diagonal
                const int c = 16 * b + 4 * lq;
                const v4f pa = ld4(Pr + c);
#pragma unroll
                for (int s = 0; s < 4; s++) ap = mma(ap, pa[s], dl[(c + s) * DS + lr]);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t_ = 16 * w + 4 * lq + r, tok = n * kC + t_;
                if (tok < T) out[((int64_t)tok * H + h) * S + j0 + lr] = (wk[WL::GAM + t_] * aq[r] + ap[r]) * qscale;
            }
        }
        // M_C = gam_C M0 + (delta o gend)^T K: wavefront w takes key blocks w, w + 4, ...
        v4f mc[S / 64];
#pragma unroll
        for (int jj = 0; jj < S / 64; jj++) {
            const int J = w + 4 * jj;
            v4f acc = {0.f, 0.f, 0.f, 0.f};
            for (int b = 0; b < kC / 16; b++) {
                const int c = 16 * b + 4 * lq;
                const v4f ge = ld4(wk + WL::GEND + c);
#pragma unroll
                for (int s = 0; s < 4; s++) acc = mma(acc, dl[(c + s) * DS + lr] * ge[s], Kc[(c + s) * KS + 16 * J + lr]);
            }
            mc[jj] = acc;
        }
        __syncthreads();   // every wavefront has finished reading M0
        const float gC = wk[WL::GC];
#pragma unroll
        for (int jj = 0; jj < S / 64; jj++) {
            const int J = w + 4 * jj;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float *m = Mb + (4 * lq + r) * KS + 16 * J + lr;
                *m = gC * *m + mc[jj][r];
            }
        }
        __syncthreads();   // M_C complete; Kc and dl free for the next chunk
    }
    for (int idx = tid; idx < JB * S / 4; idx += 256) {
        const int j = idx / (S / 4), c = 4 * (idx % (S / 4));
        *(v4f *)(state + ((int64_t)h * S + j0 + j) * S + c) = ld4(Mb + j * KS + c);
    }
}

size_t delta_chunked_work_bytes(int H, int S, int T, int chunk) {
    if (chunk != kC || T < 1 || H < 1) return 0;
    const int64_t nch = (T + kC - 1) / kC;
    if (S == 128) return (size_t)nch * H * WorkLayout<128>::SIZE * 4;
    if (S == 64) return (size_t)nch * H * WorkLayout<64>::SIZE * 4;
    return 0;
}

template <int S>
static int dc_launch(int H, int T, const float *q, const float *k, const float *v, const float *decay,
                     const float *beta, float qscale, float *state, float *out, float *work, hipStream_t st) {
    static const bool raised =
        hipFuncSetAttribute((const void *)dc_prep<S>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)prep_lds_bytes<S>()) == hipSuccess &&
        hipFuncSetAttribute((const void *)dc_scan<S>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)scan_lds_bytes<S>()) == hipSuccess;
    if (!raised) return -1;
    const int nch = (T + kC - 1) / kC;
    hipLaunchKernelGGL(dc_prep<S>, dim3(nch, H), dim3(256), prep_lds_bytes<S>(), st, H, T, q, k, v, decay, beta, work);
    hipLaunchKernelGGL(dc_scan<S>, dim3(H, S / 16), dim3(256), scan_lds_bytes<S>(), st, H, T, q, k, work, qscale, state,
                       out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int delta_chunked_launch(int H, int S, int T, int chunk, const float *q, const float *k, const float *v,
                         const float *decay, const float *beta, float qscale, float *state, float *out, float *work,
                         hipStream_t st) {
    if (chunk != kC || T < 1 || H < 1) return -1;
    // the row loads are 16-byte vectors
    for (const void *p : {(const void *)q, (const void *)k, (const void *)v, (const void *)state, (const void *)work})
        if ((uintptr_t)p & 15) return -1;
    if (S == 128) return dc_launch<128>(H, T, q, k, v, decay, beta, qscale, state, out, work, st);
    if (S == 64) return dc_launch<64>(H, T, q, k, v, decay, beta, qscale, state, out, work, st);
    return -1;
}

}  // namespace xjk
