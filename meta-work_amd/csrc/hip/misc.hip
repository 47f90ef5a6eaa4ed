// Small kernels around the token loop (gfx950):
//   embed_kernel     token id -> dequantized embedding row (xj_embed,
//                    src/xiaoju-pipe/core/xj_cpu.c:369-373; out-of-range ids give
//                    zeros). The id comes from a device array, so greedy decoding
//                    never returns to the host between tokens.
//   finalize_kernel  greedy argmax over the LM-head GEMV's per-work-group partial
//                    keys: the first index of the maximum, the rule of
//                    xj_spec.c:12-16; also records the token in the history and
//                    advances the step counter (one work-group per token row).
//   argmax_rows      plain first-maximum argmax of T rows (test entry point).
//   norm_kernel      RMSNorm / L2 rows (xj_cpu.c:56-61, :185-193).
//   swiglu_kernel    g = silu(g) * u (xj_cpu.c:273; test entry point: the
//                    token loop applies SwiGLU inside the gate|up and down GEMVs).
#include "common.h"
#include "dequant.h"
#include "kernels.h"

namespace xjk {

__global__ __launch_bounds__(256) void embed_kernel(const EmbedArgs a) {
    const int t = blockIdx.x;
    const int32_t tok = a.tokens[t];
    const int64_t K = a.w.k, nch = K / 32;
    float *x = a.x + (int64_t)t * K;
    const int64_t nblk = xjd::dev_nblk(a.w.type, a.w.n_rows, K);
    for (int64_t c = threadIdx.x; c < nch; c += 256) {
        if (tok < 0 || tok >= a.w.n_rows) {
            for (int l = 0; l < 32; l++) x[c * 32 + l] = 0.f;
        } else {
            xjd::dequant_chunk(a.w.p, a.w.type, K, nblk, tok, c, x + c * 32);
        }
    }
}

// One work-group per token row t. out[t] = argmax; tok_out (optional) gets the
// last row's id; hist/step (optional, T == 1) append it to the history.
__global__ __launch_bounds__(256) void finalize_kernel(const unsigned long long *amax, int n_part, int T,
                                                       int32_t *out, int32_t *tok_out, int32_t *hist, int32_t *step) {
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
    if (tid == 0) {
        const int32_t id = (int32_t)xjd::argmax_key_index(red[0]);
        if (out) out[t] = id;
        if (tok_out && t == T - 1) *tok_out = id;
        if (hist && step) {
            hist[*step] = id;
            *step += 1;
        }
    }
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
    const float sc = mode == 0 ? 1.0f / sqrtf((float)(ss / n) + eps) : 1.0f / sqrtf((float)ss + eps);
    for (int i = tid; i < n; i += 256) out[(int64_t)r * os + i] = w ? xr[i] * sc * w[i] : xr[i] * sc;
}

int embed_launch(const EmbedArgs &a, hipStream_t st) {
    if (a.w.k % 32) return -1;
    hipLaunchKernelGGL(embed_kernel, dim3(a.T), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int argmax_finalize_launch(const unsigned long long *amax, int n_part, int T, int32_t *out, int32_t *tok_out,
                           int32_t *hist, int32_t *step, hipStream_t st) {
    if (hist && T != 1) return -1;
    hipLaunchKernelGGL(finalize_kernel, dim3(T), dim3(256), 0, st, amax, n_part, T, out, tok_out, hist, step);
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
