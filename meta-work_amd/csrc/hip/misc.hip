// Small kernels around the token loop (gfx950):
//   embed_kernel     token id -> dequantized embedding row (xj_embed,
//                    src/xiaoju-pipe/core/xj_cpu.c:369-373; out-of-range ids give
//                    zeros). The id comes from a device array, so greedy decoding
//                    never returns to the host between tokens.
//   finalize_kernel  greedy argmax over the LM-head GEMV's per-work-group partial
//                    keys: the first index of the maximum, the rule of
//                    xj_spec.c:12-16; also records the token in the history,
//                    advances the step counter and (decode) writes the token's
//                    embedding row, the next step's input (one work-group per
//                    token row).
//   argmax_rows      plain first-maximum argmax of T rows (test entry point).
//   norm_kernel      RMSNorm / L2 rows (xj_cpu.c:56-61, :185-193); mode 2 is the
//                    RMSNorm with the product order of xj_spec.c:19-25.
//   sample_kernel    top-k 40 / top-p 0.95 sampling at a temperature (the
//                    app's sampler, ios/App/XJGlue.c:251-282, with the random
//                    number passed in); temperature <= 0: the greedy token.
//   swiglu_kernel    g = silu(g) * u (xj_cpu.c:273; test entry point: the
//                    token loop applies SwiGLU inside the gate|up and down GEMVs).
#include "common.h"
#include "dequant.h"
#include "kernels.h"

namespace xjk {

// Row tok of the embedding table into x by the 256 threads of a work-group.
__device__ __forceinline__ void embed_row(const DevW &w, int32_t tok, float *x) {
    const int64_t K = w.k, nch = K / 32;
    const int64_t nblk = xjd::dev_nblk(w.type, w.n_rows, K);
    for (int64_t c = threadIdx.x; c < nch; c += 256) {
        if (tok < 0 || tok >= w.n_rows) {
            for (int l = 0; l < 32; l++) x[c * 32 + l] = 0.f;
        } else {
            xjd::dequant_chunk(w.p, w.type, K, nblk, tok, c, x + c * 32);
        }
    }
}

__global__ __launch_bounds__(256) void embed_kernel(const EmbedArgs a) {
    const int t = blockIdx.x;
    embed_row(a.w, a.tokens[t], a.x + (int64_t)t * a.w.k);
}

// One work-group per token row t. out[t] = argmax; tok_out (optional) gets the
// last row's id; hist/step (optional, T == 1) append it to the history; e.x
// (optional, T == 1): the id's embedding row into e.x, the next decode step's
// input (so the step needs no embedding launch of its own).
__global__ __launch_bounds__(256) void finalize_kernel(const unsigned long long *amax, int n_part, int T,
                                                       int32_t *out, int32_t *tok_out, int32_t *hist, int32_t *step,
                                                       const EmbedArgs e) {
    const int t = blockIdx.x, tid = threadIdx.x;
    __shared__ unsigned long long red[256];
    unsigned long long m = 0ull;
    for (int i0 = tid; i0 < n_part; i0 += 256 * 8) {   // eight loads in flight per thread
        unsigned long long k[8];
#pragma unroll
        for (int j = 0; j < 8; j++) k[j] = i0 + 256 * j < n_part ? amax[(int64_t)t * n_part + i0 + 256 * j] : 0ull;
#pragma unroll
        for (int j = 0; j < 8; j++) m = k[j] > m ? k[j] : m;
    }
    red[tid] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s && red[tid + s] > red[tid]) red[tid] = red[tid + s];
        __syncthreads();
    }
    const int32_t id = (int32_t)xjd::argmax_key_index(red[0]);   // red[0] is final for every thread
    if (tid == 0) {
        if (out) out[t] = id;
        if (tok_out && t == T - 1) *tok_out = id;
        if (hist && step) {
            hist[*step] = id;
            *step += 1;
        }
    }
    if (e.x) embed_row(e.w, id, e.x);
}

__global__ __launch_bounds__(256) void argmax_rows_kernel(const float *x, int n, int32_t *out) {
    const int t = blockIdx.x, tid = threadIdx.x;
    __shared__ unsigned long long red[256];
    unsigned long long m = 0ull;
    for (int i = tid; i < n; i += 256) {
        const unsigned long long k = xjd::argmax_key(x[(int64_t)t * n + i], (uint32_t)i);
        m = k > m ? k : m;
    }
    red[tid] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s && red[tid + s] > red[tid]) red[tid] = red[tid + s];
        __syncthreads();
    }
    if (tid == 0) out[t] = (int32_t)xjd::argmax_key_index(red[0]);
}

__global__ __launch_bounds__(256) void norm_kernel(int mode, const float *x, int64_t xs, const float *w, int n, float eps,
                                                   float *out, int64_t os) {
    const int r = blockIdx.x, tid = threadIdx.x;
    __shared__ double red[4];
    const float *xr = x + (int64_t)r * xs;
    double ss = 0;
    for (int i = tid; i < n; i += 256) ss += (double)xr[i] * xr[i];
    ss = xjd::block_sum_d(ss, red);
    const float sc = mode != 1 ? 1.0f / sqrtf((float)(ss / n) + eps) : 1.0f / sqrtf((float)ss + eps);
    if (mode == 2)   // x * (sc * w): the speculative driver's in-place norm (xj_spec.c:19-25)
        for (int i = tid; i < n; i += 256) out[(int64_t)r * os + i] = xr[i] * (sc * w[i]);
    else
        for (int i = tid; i < n; i += 256) out[(int64_t)r * os + i] = w ? xr[i] * sc * w[i] : xr[i] * sc;
}

int embed_launch(const EmbedArgs &a, hipStream_t st) {
    if (a.w.k % 32) return -1;
    hipLaunchKernelGGL(embed_kernel, dim3(a.T), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int argmax_finalize_launch(const unsigned long long *amax, int n_part, int T, int32_t *out, int32_t *tok_out,
                           int32_t *hist, int32_t *step, hipStream_t st, const EmbedArgs *embed) {
    if (hist && T != 1) return -1;
    if (embed && (T != 1 || embed->w.k % 32 || !embed->x)) return -1;
    const EmbedArgs e = embed ? *embed : EmbedArgs{};
    hipLaunchKernelGGL(finalize_kernel, dim3(T), dim3(256), 0, st, amax, n_part, T, out, tok_out, hist, step, e);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int argmax_rows_launch(const float *x, int n, int T, int32_t *out, hipStream_t st) {
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(T), dim3(256), 0, st, x, n, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

__global__ __launch_bounds__(256) void swiglu_kernel(float *g, const float *u, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) g[i] = xjd::silu(g[i]) * u[i];
}

int swiglu_launch(float *g, const float *u, int64_t n, hipStream_t st) {
    if (n < 0) return -1;
    if (n == 0) return 0;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Row t of lg: radix-select the 40th largest value (ordered 32-bit keys, 8 bits
// per pass, LDS histograms), take every value above it and the lowest indices
// of those equal to it, then one thread sorts the 40 by value (equal values in
// index order) - the app's result whenever the kept values are distinct (its
// replace-the-minimum loop and exchange sort keep and order equal values by
// slot, not index; a value tied at the 40th place is never drawn, the 0.95 cut
// always ending before the last kept value) - forms
// p_i = exp((v_i - v_0) / temp) in double, cuts where the running share first
// reaches 0.95 and picks with r = rnd[t] / 2^30 times the kept mass.
constexpr int kTopK = 40;
__device__ __forceinline__ uint32_t okey(float v) {
    const uint32_t b = __float_as_uint(v);
    return v != v ? 0u : (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__global__ __launch_bounds__(256) void sample_kernel(const float *lg, int V, float temp, const uint32_t *rnd, int32_t *out) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *x = lg + (int64_t)t * V;
    __shared__ unsigned long long best_sh[4];
    if (!(temp > 0.f)) {   // the greedy token: first maximum
        unsigned long long b = 0ull;
        for (int i = tid; i < V; i += 256) {
            const unsigned long long k = xjd::argmax_key(x[i], (uint32_t)i);
            b = k > b ? k : b;
        }
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long q = __shfl_xor(b, off, 64);
            b = q > b ? q : b;
        }
        if ((tid & 63) == 0) best_sh[tid >> 6] = b;
        __syncthreads();
        if (tid == 0) {
            unsigned long long m = best_sh[0];
            for (int w = 1; w < 4; w++) m = best_sh[w] > m ? best_sh[w] : m;
            out[t] = (int32_t)xjd::argmax_key_index(m);
        }
        return;
    }
    __shared__ uint32_t hist[256];
    __shared__ uint32_t pre_sh;
    __shared__ int need_sh, ngt_sh;
    __shared__ int cnt_eq[256];
    __shared__ float cv[kTopK];
    __shared__ int ci[kTopK];
    const int K = V < kTopK ? V : kTopK;
    uint32_t pre = 0, mask = 0;
    int need = K;   // how many of the elements matching the prefix are still to be taken from the top
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < V; i += 256) {
            const uint32_t k = okey(x[i]);
            if ((k & mask) == pre) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            int cum = 0, b = 255;
            for (; b > 0; b--) {
                if (cum + (int)hist[b] >= need) break;
                cum += hist[b];
            }
            pre_sh = pre | ((uint32_t)b << shift);
            need_sh = need - cum;
        }
        __syncthreads();
        pre = pre_sh;
        need = need_sh;
        mask |= 0xFFu << shift;
        __syncthreads();
    }
    // pre = the K-th largest key; take every key above it and the `need` lowest
    // indices equal to it. Thread tid scans the contiguous chunk [i0, i1).
    const int chunk = (V + 255) / 256, i0 = tid * chunk, i1 = i0 + chunk < V ? i0 + chunk : V;
    int my_eq = 0;
    for (int i = i0; i < i1; i++) my_eq += okey(x[i]) == pre;
    cnt_eq[tid] = my_eq;
    if (tid == 0) ngt_sh = 0;
    __syncthreads();
    int before = 0;
    for (int j = 0; j < tid; j++) before += cnt_eq[j];
    const int n_gt = K - need;
    for (int i = i0; i < i1; i++) {
        const uint32_t k = okey(x[i]);
        if (k > pre) {
            const int slot = atomicAdd(&ngt_sh, 1);
            cv[slot] = x[i];
            ci[slot] = i;
        } else if (k == pre) {
            if (before < need) {
                cv[n_gt + before] = x[i];
                ci[n_gt + before] = i;
            }
            before++;
        }
    }
    __syncthreads();
    if (tid == 0) {
        // descending by value, ties by index
        for (int i = 1; i < K; i++) {
            const float v = cv[i];
            const int id = ci[i];
            int j = i - 1;
            while (j >= 0 && (cv[j] < v || (cv[j] == v && ci[j] > id))) { cv[j + 1] = cv[j]; ci[j + 1] = ci[j]; j--; }
            cv[j + 1] = v;
            ci[j + 1] = id;
        }
        double p[kTopK], sum = 0;
        for (int i = 0; i < K; i++) { p[i] = exp((double)((cv[i] - cv[0]) / temp)); sum += p[i]; }
        double acc = 0;
        int cut = K;
        for (int i = 0; i < K; i++) { acc += p[i] / sum; if (acc >= 0.95) { cut = i + 1; break; } }
        double s2 = 0;
        for (int i = 0; i < cut; i++) s2 += p[i];
        double r = (double)rnd[t] / (double)(1u << 30) * s2;
        int pick = ci[0];
        for (int i = 0; i < cut; i++) { r -= p[i]; if (r <= 0) { pick = ci[i]; break; } }
        out[t] = pick;
    }
}

int sample_launch(const float *lg, int V, int T, float temp, const uint32_t *rnd, int32_t *out, hipStream_t st) {
    if (V < 1 || T < 1) return -1;
    hipLaunchKernelGGL(sample_kernel, dim3(T), dim3(256), 0, st, lg, V, temp, rnd, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int norm_launch(int mode, const float *x, const float *w, int n, int rows, float eps, float *out, hipStream_t st) {
    return norm_rows_launch(mode, x, n, w, n, rows, eps, out, n, st);
}

int norm_rows_launch(int mode, const float *x, int64_t xs, const float *w, int n, int rows, float eps, float *out,
                     int64_t os, hipStream_t st) {
    if (rows < 1 || n < 1) return rows == 0 ? 0 : -1;
    hipLaunchKernelGGL(norm_kernel, dim3(rows), dim3(256), 0, st, mode, x, xs, w, n, eps, out, os);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
