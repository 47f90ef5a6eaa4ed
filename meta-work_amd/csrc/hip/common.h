// Device-side helpers shared by the gfx950 kernels: fp16 conversion, 16-lane
// DPP reductions, block reductions, and the error plumbing of the host side.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#define XJ_CHECK(call, err, errlen, ...)                                                     \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess) {                                                              \
            snprintf(err, errlen, "%s: %s", #call, hipGetErrorString(e_));                   \
            return __VA_ARGS__;                                                              \
        }                                                                                    \
    } while (0)

namespace xjd {

// fp16 bits -> fp32; the hardware conversion is exact, subnormals included.
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    _Float16 h;
    uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// fp32 -> fp16 bits, round to nearest even (overflow -> inf).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float sigm(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

// DPP row (16-lane) butterfly: after the four steps every lane of the row holds
// the sum over the row. The order of additions is fixed, so results are
// reproducible run to run.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}

template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Sum over the 64 lanes of a wavefront in double, in a fixed order: DPP
// butterflies inside each row of 16 lanes, then the four row sums (read into
// scalar registers) as (r0 + r1) + (r2 + r3). Every lane gets the total; all
// 64 lanes must be active.
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Block-wide sum (blockDim.x a multiple of 64, <= 1024) in double; every
// thread gets the total. red must hold blockDim.x/64 doubles.
__device__ __forceinline__ double block_sum_d(double v, double *red) {
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    double s = 0;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}
// Sum over the first NW wavefronts of the work-group (threads beyond hold
// nothing): those wavefronts reduce, every thread gets the total. red must
// hold NW doubles; all threads must call it.
template <int NW>
__device__ __forceinline__ double head_sum_d(double v, double *red) {
    const int w = threadIdx.x >> 6;
    if (w < NW) {
        v = wave_sum_d(v);
        if ((threadIdx.x & 63) == 0) red[w] = v;
    }
    __syncthreads();
    double s = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) s += red[i];
    return s;
}

// Two block-wide sums with one exchange (same order as two block_sum_d calls);
// red must hold 2 * blockDim.x/64 doubles.
__device__ __forceinline__ void block_sum2_d(double &a, double &b, double *red) {
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    a = wave_sum_d(a);
    b = wave_sum_d(b);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        red[w] = a;
        red[nw + w] = b;
    }
    __syncthreads();
    double s = 0, t = 0;
    for (int i = 0; i < nw; i++) {
        s += red[i];
        t += red[nw + i];
    }
    a = s;
    b = t;
}
__device__ __forceinline__ float block_max(float v, float *red) {
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < nw; i++) m = fmaxf(m, red[i]);
    return m;
}

// Greedy argmax key: larger key = larger value, ties -> lower index, NaN lowest.
// Key of element idx for the first maximum of `if (x[i] > x[b]) b = i` from
// b = 0 (xj_spec.c:12-16): the largest key wins, equal values (-0 == +0
// included) give the lowest index, NaN never wins - except at index 0, which
// no later value can replace.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    const uint32_t b = v == 0.f ? 0u : __float_as_uint(v);
    uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    if (v != v) ord = idx == 0 ? 0xFFFFFFFFu : 0u;
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t argmax_key_index(unsigned long long k) {
    return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull);
}

}  // namespace xjd
