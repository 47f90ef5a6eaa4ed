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

// Row tok of the embedding table into x by the first nthreads threads of a work-group.
__device__ __forceinline__ void embed_row(const DevW &w, int32_t tok, float *x, int nthreads = 256) {
    const int64_t K = w.k, nch = K / 32;
    const int64_t nblk = xjd::dev_nblk(w.type, w.n_rows, K);
    for (int64_t c = threadIdx.x; c < nch; c += nthreads) {
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
constexpr int kFinThreads = 1024;
__global__ __launch_bounds__(kFinThreads) void finalize_kernel(const unsigned long long *amax, int n_part, int T,
                                                               int32_t *out, int32_t *tok_out, int32_t *hist,
                                                               int32_t *step, const EmbedArgs e) {
    const int t = blockIdx.x, tid = threadIdx.x;
    __shared__ unsigned long long red[kFinThreads / 64];
    unsigned long long m = 0ull;
    // eight loads in flight per thread: the 4B head's 4748 partials in one round
    for (int i0 = tid; i0 < n_part; i0 += kFinThreads * 8) {
        unsigned long long k[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            k[j] = i0 + kFinThreads * j < n_part ? amax[(int64_t)t * n_part + i0 + kFinThreads * j] : 0ull;
#pragma unroll
        for (int j = 0; j < 8; j++) m = k[j] > m ? k[j] : m;
    }
    // the keys are distinct (each holds its index), so any order of maxima gives the same key
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long q = __shfl_xor(m, off, 64);
        m = q > m ? q : m;
    }
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = 0ull;
#pragma unroll
    for (int w = 0; w < kFinThreads / 64; w++) m = red[w] > m ? red[w] : m;
    const int32_t id = (int32_t)xjd::argmax_key_index(m);
    if (tid == 0) {
        if (out) out[t] = id;
        if (tok_out && t == T - 1) *tok_out = id;
        if (hist && step) {
            hist[*step] = id;
            *step += 1;
        }
    }
    if (e.x) embed_row(e.w, id, e.x, kFinThreads);
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
    hipLaunchKernelGGL(finalize_kernel, dim3(T), dim3(kFinThreads), 0, st, amax, n_part, T, out, tok_out, hist, step, e);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int argmax_rows_launch(const float *x, int n, int T, int32_t *out, hipStream_t st) {
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(T), dim3(256), 0, st, x, n, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Entry blockIdx.y of the list, 16 bytes per thread and step where both ends
// are 16-byte aligned and the count a multiple of 4 (the states), else 4.
__global__ __launch_bounds__(256) void copy_list_kernel(const CopyList c) {
    const int e = blockIdx.y;
    if (e >= c.cnt) return;
    const float *s = c.src[e];
    float *d = c.dst[e];
    const int64_t n = c.n[e], stride = (int64_t)gridDim.x * 256;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (!(((uintptr_t)s | (uintptr_t)d) & 15) && !(n & 3)) {
        const float4 *s4 = (const float4 *)s;
        float4 *d4 = (float4 *)d;
        for (int64_t i = i0; i < n / 4; i += stride) d4[i] = s4[i];
    } else {
        for (int64_t i = i0; i < n; i += stride) d[i] = s[i];
    }
}

int copy_list_launch(const CopyList &c, hipStream_t st) {
    if (c.cnt < 0 || c.cnt > kCopyMax) return -1;
    if (c.cnt == 0) return 0;
    int64_t most = 0;
    for (int i = 0; i < c.cnt; i++) {
        if (c.n[i] < 0 || (c.n[i] && (!c.src[i] || !c.dst[i]))) return -1;
        most = c.n[i] > most ? c.n[i] : most;
    }
    if (!most) return 0;
    // up to 64 work-groups per entry, each copying 4 KB per step
    const int64_t want = (most / 4 + 255) / 256;
    const unsigned gx = (unsigned)(want < 1 ? 1 : want > 64 ? 64 : want);
    hipLaunchKernelGGL(copy_list_kernel, dim3(gx, c.cnt), dim3(256), 0, st, c);
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

// ---------------------------------------------------------------- sampler --
// The app's sampler (ios/App/XJGlue.c:251-282), one work-group of 1024
// threads per row, the uniform number passed in. Its loop keeps 40 slots:
// the first 40 values fill them, a later value v enters when v > val[mi] and
// takes slot mi, mi being the first slot holding the minimum (a strict `<`
// scan from slot 0); then an exchange sort orders the slots by value,
// p_i = exp((v_i - v_0) / temp) in double, the kept prefix ends where the
// running share first reaches 0.95, and r = rand30 / 2^30 times the kept mass
// picks. The slots always hold the 40 largest values seen so far (a NaN
// never enters), so when the first 40 values hold no NaN, the kept values are
// distinct and no other element equals the smallest of them, the result is
// the 40 largest in descending order whatever the slot history. The fast path
// finds them from the row's partial maxima (the LM head's argmax partials, or
// a partials launch): the 40th largest partial maximum T bounds the 40th
// value from below, so only partials whose maximum reaches T are read; their
// elements at or above T are compacted in LDS and radix-selected. Otherwise
// the slot history decides the order of equal values and which of them are
// kept: one wavefront replays the app's loop over the row in index order
// (tiles staged in LDS, only values above the tile's starting minimum
// examined) and one thread runs the exchange sort as written.
constexpr int kTopK = 40;
constexpr int kSmpThreads = 1024;
constexpr int kSmpWaves = kSmpThreads / 64;
constexpr int kSmpCap = 4096;      // candidates held in LDS (fast path); tile of the replay
constexpr int kSmpScan = 16384;    // elements of the partials read by the fast path, at most
constexpr int kSmpParts = 1024;    // partials read by the fast path, at most
constexpr int kSmpPartLds = 6144;  // partial maxima staged in LDS (more: read from memory)
static_assert(kSmpCap == 4 * kSmpThreads, "a replay tile is four elements per thread");

// ordered key: larger value, larger key (NaN lowest; -0 below +0)
__device__ __forceinline__ uint32_t okey(float v) {
    const uint32_t b = __float_as_uint(v);
    return v != v ? 0u : (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// the value part of an argmax key (zeros of either sign alike)
__device__ __forceinline__ uint32_t ordc(float v) { return (uint32_t)(xjd::argmax_key(v, 1u) >> 32); }

struct SampleShared {
    uint32_t hist[256];
    uint32_t pord[kSmpPartLds];   // value parts of the partial maxima
    float cv[kSmpCap];
    int32_t ci[kSmpCap];
    int32_t plist[kSmpParts];
    unsigned long long gmask[kSmpCap / 64];
    unsigned long long red[kSmpWaves];
    float kv[kTopK];      // the kept values and indices, in the app's final order
    int32_t kix[kTopK];
    int n_kept, ncand, npart, tie, need, cnt;
    uint32_t pre, rand30;
    float thr;
};

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long q = __shfl_xor(v, off, 64);
        v = q > v ? q : v;
    }
    return v;
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long q = __shfl_xor(v, off, 64);
        v = q < v ? q : v;
    }
    return v;
}
// inclusive prefix sum over the lanes of a wavefront
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v, int lane) {
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t q = __shfl_up(v, off, 64);
        if (lane >= off) v += q;
    }
    return v;
}

// The k-th largest (1 <= k <= n) of the n keys get(i), by 8-bit radix
// passes with LDS histograms; *gt = how many keys are larger, *eq = how many
// equal it. With fewer than four passes the result is that key with its
// remaining low bits cleared (a lower bound; gt and eq then count prefixes).
// Every thread of the work-group calls it.
template <class Get>
__device__ uint32_t block_kth_largest(Get get, int n, int k, SampleShared &sh, int *gt, int *eq, int passes = 4) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint32_t pre = 0, mask = 0;
    int need = k, cnt = n;
    for (int shift = 24; shift >= 32 - 8 * passes; shift -= 8) {
        if (tid < 256) sh.hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kSmpThreads) {
            const uint32_t v = get(i);
            if ((v & mask) == pre) atomicAdd(&sh.hist[(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wid == 0) {   // lane l holds bins 255-4l .. 252-4l, counted from the top
            uint32_t h[4], tot = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) { h[j] = sh.hist[255 - 4 * lane - j]; tot += h[j]; }
            const uint32_t hi = wave_incl_sum(tot, lane), lo = hi - tot;
            if (lo < (uint32_t)need && hi >= (uint32_t)need) {
                uint32_t c = lo;
                int j = 0;
                while (c + h[j] < (uint32_t)need) c += h[j++];
                sh.pre = pre | ((uint32_t)(255 - 4 * lane - j) << shift);
                sh.need = need - (int)c;   // still to take from that bin
                sh.cnt = (int)h[j];        // keys in that bin
            }
        }
        __syncthreads();
        pre = sh.pre;
        need = sh.need;
        cnt = sh.cnt;
        mask |= 255u << shift;
        __syncthreads();
    }
    *gt = k - need;
    *eq = cnt;
    return pre;
}

// The app's mi after a slot changed: the first slot holding the minimum by
// `val[j] < val[mi]` from slot 0 - NaN slots are never below anything, and
// nothing is below a NaN in slot 0 (mi stays 0); -0 and +0 are equal.
// Lane j < k of wavefront 0 holds slot j's value sv.
__device__ __forceinline__ int app_min_slot(float sv, int lane, int k, float sv0) {
    const float c = sv == 0.f ? 0.f : sv;
    const unsigned long long key =
        lane < k && sv == sv ? ((unsigned long long)okey(c) << 32) | (unsigned long long)lane : ~0ull;
    const unsigned long long m = wave_min_u64(key);
    return sv0 != sv0 || m == ~0ull ? 0 : (int)(m & 0xFFFFFFFFull);
}

__device__ __forceinline__ double readlane_d(double v, int i) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, i), hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), i);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// The pick from the k kept slots in their final order (XJGlue.c:272-281, in
// double, every sum in the app's order), by wavefront 0: lane i forms p_i and
// p_i / sum, the running sums walk the lanes in order.
__device__ int app_pick(const float *kv, const int32_t *kix, int k, float temp, uint32_t rand30, int lane) {
    const float v0 = kv[0];
    const double p = lane < k ? exp((double)((kv[lane] - v0) / temp)) : 0.0;
    double sum = 0;
    for (int i = 0; i < k; i++) sum += readlane_d(p, i);
    const double q = p / sum;
    double acc = 0;
    int cut = k;
    for (int i = 0; i < k; i++) {
        acc += readlane_d(q, i);
        if (acc >= 0.95) { cut = i + 1; break; }
    }
    double s2 = 0;
    for (int i = 0; i < cut; i++) s2 += readlane_d(p, i);
    double r = (double)rand30 / (double)(1u << 30) * s2;
    for (int i = 0; i < cut; i++) {
        r -= readlane_d(p, i);
        if (r <= 0) return kix[i];
    }
    return kix[0];
}

// One row: the greedy token (temp <= 0) or the app's draw, returned to every
// thread; rand30 matters on thread 0 only. part[p] (n_part of them) is the
// largest argmax key of elements [p * part_rows, (p + 1) * part_rows).
__device__ int sample_row(const float *__restrict__ x, int V, float temp, uint32_t rand30,
                          const unsigned long long *__restrict__ part, int n_part, int part_rows, SampleShared &sh) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int K = kTopK;
    const bool sampling = !(temp <= 0.f);
    if (tid == 0) { sh.ncand = 0; sh.n_kept = 0; sh.tie = 0; sh.npart = 0; sh.rand30 = rand30; }
    // the first maximum: the largest partial key; the fill's values checked
    // for NaN and the partials' value parts staged in LDS on the way
    const bool lds_part = n_part <= kSmpPartLds;
    int bad = V < K || n_part < K;
    float f = 0.f;
    if (sampling && !bad && tid < K) f = x[tid];
    unsigned long long best = 0ull;
    for (int p = tid; p < n_part; p += kSmpThreads) {
        const unsigned long long q = part[p];
        best = q > best ? q : best;
        if (lds_part) sh.pord[p] = (uint32_t)(q >> 32);
    }
    best = wave_max_u64(best);
    if (lane == 0) sh.red[wid] = best;
    bad = bad || f != f;
    bad = __syncthreads_or(bad);
    if (!sampling) {
        unsigned long long m = sh.red[0];
        for (int w = 1; w < kSmpWaves; w++) m = sh.red[w] > m ? sh.red[w] : m;
        return (int)xjd::argmax_key_index(m);
    }
    // the fast path needs 40 values without NaN in the fill and 40 partials
    bool kept = false;   // the fast path settled the kept values and their order
    if (!bad) {
        // T: the 40th largest partial maximum, its low 16 bits cleared (a lower
        // bound of the 40th value); the partials reaching it, listed
        int gt, eq;
        auto pv = [&](int i) { return lds_part ? sh.pord[i] : (uint32_t)(part[i] >> 32); };
        const uint32_t T = block_kth_largest(pv, n_part, K, sh, &gt, &eq, 2);
        for (int p0 = 0; p0 < n_part; p0 += kSmpThreads) {
            const int p = p0 + tid;
            const bool c = p < n_part && pv(p) >= T;
            const unsigned long long m = __ballot(c);
            if (!m) continue;
            int base = 0;
            if (lane == 0) base = atomicAdd(&sh.npart, __popcll(m));
            base = __shfl(base, 0, 64);
            const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
            if (c && pos < kSmpParts) sh.plist[pos] = p;
        }
        __syncthreads();
        const int np = sh.npart;
        if (T > 0u && np <= kSmpParts && (int64_t)np * part_rows <= kSmpScan) {   // (T = 0: NaN partials)
            // their elements at or above T, compacted (any order)
            const int ne = np * part_rows;
            for (int e0 = 0; e0 < ne; e0 += kSmpThreads) {
                const int e = e0 + tid;
                int i = V;
                float v = 0.f;
                if (e < ne) {
                    i = sh.plist[e / part_rows] * part_rows + e % part_rows;
                    if (i < V) v = x[i];
                }
                const bool c = i < V && v == v && ordc(v) >= T;
                const unsigned long long m = __ballot(c);
                if (!m) continue;
                int base = 0;
                if (lane == 0) base = atomicAdd(&sh.ncand, __popcll(m));
                base = __shfl(base, 0, 64);
                const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
                if (c && pos < kSmpCap) { sh.cv[pos] = v; sh.ci[pos] = i; }
            }
            __syncthreads();
            const int C = sh.ncand;
            if (C <= kSmpCap && C >= K) {
                // the 40th largest key among them; a tie there, or a zero (whose
                // sign the key tells apart and the app's comparisons do not),
                // needs the replay
                const uint32_t pre = block_kth_largest([&](int i) { return okey(sh.cv[i]); }, C, K, sh, &gt, &eq);
                const float v40 = __uint_as_float((pre & 0x80000000u) ? (pre & 0x7FFFFFFFu) : ~pre);
                if (eq == K - gt && v40 != 0.f) {
                    for (int j = tid; j < C; j += kSmpThreads)
                        if (okey(sh.cv[j]) >= pre) {
                            const int pos = atomicAdd(&sh.n_kept, 1);
                            if (pos < K) { sh.kv[pos] = sh.cv[j]; sh.kix[pos] = sh.ci[j]; }
                        }
                    __syncthreads();
                    if (wid == 0) {
                        // the 40 in descending order (bitonic over the wavefront);
                        // equal neighbours are a tie among the kept values
                        const bool in = lane < K && lane < sh.n_kept;
                        unsigned long long key =
                            in ? ((unsigned long long)okey(sh.kv[lane]) << 32) | (uint32_t)sh.kix[lane] : 0ull;
                        for (int kk = 2; kk <= 64; kk <<= 1)
                            for (int j = kk >> 1; j > 0; j >>= 1) {
                                const unsigned long long q = __shfl_xor(key, j, 64);
                                const bool desc = (lane & kk) == 0, low = (lane & j) == 0;
                                key = (low == desc) ? (q > key ? q : key) : (q < key ? q : key);
                            }
                        const uint32_t ok = (uint32_t)(key >> 32);
                        const float v = __uint_as_float((ok & 0x80000000u) ? (ok & 0x7FFFFFFFu) : ~ok);
                        const float prev = __shfl_up(v, 1, 64);
                        if (__ballot(lane > 0 && lane < K && v == prev)) {
                            if (lane == 0) sh.tie = 1;
                        } else if (lane < K) {
                            sh.kv[lane] = v;
                            sh.kix[lane] = (int32_t)(key & 0xFFFFFFFFull);
                        }
                    }
                    __syncthreads();
                    kept = sh.n_kept == K && !sh.tie;
                }
            }
        }
    }
    int k = K;
    if (!kept) {
        // the app's loop replayed in index order by wavefront 0 (lane j < kf
        // holds slot j), the row staged in LDS a tile at a time
        const int kf = V < K ? V : K;
        k = kf;
        float sv = 0.f, thr = 0.f;
        int si = 0, mi = 0;
        if (wid == 0) {
            if (lane < kf) { sv = x[lane]; si = lane; }
            const float sv0 = __shfl(sv, 0, 64);
            mi = app_min_slot(sv, lane, kf, sv0);
            thr = __shfl(sv, mi, 64);
            if (lane == 0) sh.thr = thr;
        }
        __syncthreads();
        // once slot 0 holds NaN nothing can enter (v > NaN is false)
        const bool stop = sh.thr != sh.thr;
        for (int t0 = kf; t0 < V && !stop; t0 += kSmpCap) {
            const int n = V - t0 < kSmpCap ? V - t0 : kSmpCap;
            const float thr0 = sh.thr;   // the minimum at the tile's start bounds every entry below
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int e = r * kSmpThreads + tid;
                const float v = e < n ? x[t0 + e] : __builtin_nanf("");
                sh.cv[e] = v;
                const unsigned long long m = __ballot(v > thr0);
                if (lane == 0) sh.gmask[r * kSmpWaves + wid] = m;
            }
            __syncthreads();
            if (wid == 0) {
                for (int g = 0; g * 64 < n; g++) {
                    if (!sh.gmask[g]) continue;
                    const float v = sh.cv[g * 64 + lane];
                    unsigned long long m = __ballot(v > thr);
                    while (m) {
                        const int l = __ffsll((long long)m) - 1;
                        const float nv = __shfl(v, l, 64);
                        if (lane == mi) { sv = nv; si = t0 + g * 64 + l; }
                        const float sv0 = __shfl(sv, 0, 64);
                        mi = app_min_slot(sv, lane, kf, sv0);
                        thr = __shfl(sv, mi, 64);
                        m = l == 63 ? 0ull : __ballot(v > thr) & (~0ull << (l + 1));
                    }
                }
                if (lane == 0) sh.thr = thr;
            }
            __syncthreads();
        }
        if (wid == 0 && lane < kf) { sh.kv[lane] = sv; sh.kix[lane] = si; }
        __syncthreads();
        if (tid == 0) {   // the exchange sort as written (XJGlue.c:271)
            float v[kTopK];
            int32_t id[kTopK];
#pragma unroll
            for (int i = 0; i < kTopK; i++) { v[i] = i < kf ? sh.kv[i] : 0.f; id[i] = i < kf ? sh.kix[i] : 0; }
#pragma unroll
            for (int i = 0; i < kTopK; i++)
#pragma unroll
                for (int j = i + 1; j < kTopK; j++)
                    if (j < kf && v[j] > v[i]) {
                        const float tv = v[i]; v[i] = v[j]; v[j] = tv;
                        const int32_t ti = id[i]; id[i] = id[j]; id[j] = ti;
                    }
#pragma unroll
            for (int i = 0; i < kTopK; i++)
                if (i < kf) { sh.kv[i] = v[i]; sh.kix[i] = id[i]; }
        }
        __syncthreads();
    }
    if (wid == 0) {
        const int pick = app_pick(sh.kv, sh.kix, k, temp, sh.rand30, lane);
        if (lane == 0) sh.ncand = pick;
    }
    __syncthreads();
    return sh.ncand;
}

// Partial maxima for the sampler: part[t][p] = the largest argmax key of row
// t's elements [p * part_rows, (p + 1) * part_rows), one wavefront per partial.
__global__ __launch_bounds__(256) void sample_part_kernel(const float *lg, int V, int part_rows, int n_part,
                                                          unsigned long long *part) {
    const int t = blockIdx.y, p = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (p >= n_part) return;
    const float *x = lg + (int64_t)t * V;
    unsigned long long m = 0ull;
    for (int j = lane; j < part_rows; j += 64) {
        const int i = p * part_rows + j;
        if (i < V) {
            const unsigned long long k = xjd::argmax_key(x[i], (uint32_t)i);
            m = k > m ? k : m;
        }
    }
    m = wave_max_u64(m);
    if (lane == 0) part[(int64_t)t * n_part + p] = m;
}

__global__ __launch_bounds__(kSmpThreads) void sample_kernel(const SampleArgs a) {
    __shared__ SampleShared sh;
    const int t = blockIdx.x;
    const float temp = a.temp_dev ? *a.temp_dev : a.temp;
    uint32_t r30 = 0;
    if (threadIdx.x == 0 && !(temp <= 0.f)) r30 = a.rnd[(a.rbase ? *a.rbase : 0) + (a.step ? *a.step : 0) + t];
    const int id = sample_row(a.lg + (int64_t)t * a.V, a.V, temp, r30, a.part + (int64_t)t * a.n_part, a.n_part,
                              a.part_rows, sh);
    if (threadIdx.x == 0) {
        if (a.out) a.out[t] = id;
        if (a.tok_out && t == a.T - 1) *a.tok_out = id;
        if (a.hist && a.step) {
            a.hist[*a.step] = id;
            *a.step += 1;
        }
    }
    if (a.embed.x) embed_row(a.embed.w, id, a.embed.x, kSmpThreads);
}

int sample_part_rows(int V) {
    const int r = V / 64;
    return r < 1 ? 1 : r > 256 ? 256 : r;
}

int sample_part_launch(const float *lg, int V, int T, unsigned long long *part, hipStream_t st) {
    if (V < 1 || T < 1) return -1;
    const int rows = sample_part_rows(V), n = (V + rows - 1) / rows;
    hipLaunchKernelGGL(sample_part_kernel, dim3((n + 3) / 4, T), dim3(256), 0, st, lg, V, rows, n, part);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int sample_launch(const SampleArgs &a, hipStream_t st) {
    if (a.V < 1 || a.T < 1 || !a.part || a.n_part < 1 || a.part_rows < 1) return -1;
    if ((int64_t)a.n_part * a.part_rows < a.V) return -1;
    if ((a.hist || a.embed.x) && a.T != 1) return -1;
    if (a.embed.x && a.embed.w.k % 32) return -1;
    if (a.hist && !a.step) return -1;
    hipLaunchKernelGGL(sample_kernel, dim3(a.T), dim3(kSmpThreads), 0, st, a);
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
