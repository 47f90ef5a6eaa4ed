// Prepared GEMV activations ("xq"), shared by the prep kernel, the producers
// that emit them directly (GEMV tails, the DeltaNet and attention kernels)
// and the GEMV that stages them in LDS.
//
// Per token, for each 32-element group g of the K inputs (v = the activation
// after its prologue: RMSNorm, SwiGLU, gated RMSNorm or none):
//   dig [G][3][32] int8   balanced base-128 digits a, b, c of
//                         X = rint(v * 2^(20 - E_g)) = a*2^14 + b*2^7 + c,
//                         |X| <= 2^20, |a| <= 64, b, c in [-64, 63]
//   f   [G] float         2^(E_g - 20), where max|v| over the group < 2^E_g
//   sx  [2G] int32        sum of X over each 16-element half of the group
//   ss  [G] double        for an RMSNorm input stored as u = x * w: sum of x^2
//                         over the group (the consumer forms the norm's scale)
//   v   [K] float         v itself (read by F32 rows only)
// Integer dot products of quantized weights with X are exact in 32 bits for
// every block type, so sub-block sums do not depend on the summation order.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace xjk {

// Bytes per group of digits (the three planes).
constexpr int kDigStride = 96;

struct XqOff {
    int G, f_off, sx_off, ss_off, v_off, stride;   // bytes; v_off = the LDS bytes per token
};
__host__ __device__ inline XqOff xq_off(int K) {
    XqOff o;
    o.G = K / 32;
    o.f_off = o.G * kDigStride;
    o.sx_off = o.f_off + ((o.G * 4 + 15) & ~15);
    o.ss_off = o.sx_off + ((o.G * 8 + 15) & ~15);
    o.v_off = o.ss_off + ((o.G * 8 + 15) & ~15);
    o.stride = (o.v_off + K * 4 + 255) & ~255;
    return o;
}

// The matrix-core GEMM's activations ("hq"), built by the same prep launches
// for chunks of tokens. Per token, for each 256-element block b of the K
// inputs, a record of kHqBlk bytes:
//   hi [256] f16, lo [256] f16   v * 2^-e = hi + lo, each rounded to nearest:
//                                e is the block's exponent, max|v| < 2^(e+14),
//                                so hi + lo carries about 22 bits of v
//   sx [8] float                 sum of (hi + lo) * 2^e over each 32-element group
//   e  int32, then 12 bytes of padding
// The record is 67 chunks of 16 bytes (an odd count, so the GEMM's LDS reads
// of 16 tokens fall on distinct banks); tokens are hq_stride(K) bytes apart.
constexpr int kHqBlk = 1072;
__host__ __device__ inline int64_t hq_stride(int K) { return ((int64_t)(K / 256) * kHqBlk + 255) & ~(int64_t)255; }

}  // namespace xjk

#ifdef __HIPCC__
#include "common.h"

namespace xjd {

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
__device__ __forceinline__ int row16_sum_i(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    v += dpp_i<0x141>(v);
    v += dpp_i<0x140>(v);
    return v;
}

// Bytes d' in [0, 128] -> d' - 64 as int8, in every byte of a word: d' ^ 0xC0
// is d' - 64 when bit 6 of d' is clear; bit 6 set flips bit 7 back.
__device__ __forceinline__ uint32_t unbias_bytes(uint32_t p) { return p ^ 0xC0C0C0C0u ^ ((p << 1) & 0x80808080u); }

// Writes element k (value v) of one token's xq at dst. Called by all 64
// lanes of a wavefront with k = k0 + lane, k0 a multiple of 64, so that each
// half-wavefront holds one 32-element group; lanes with in == false (k >= K,
// always whole groups since K % 32 == 0) pass v = 0 and store nothing.
// dst may be global memory or LDS (with_v = false: the LDS copy has no v).
__device__ __forceinline__ void emit_xq(float v, int k, bool in, uint8_t *dst, const xjk::XqOff &o, bool with_v = true) {
    float m = fabsf(v);
    m = row16_max(m);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    int E = 0;
    (void)frexpf(m, &E);
    if (E < -100) E = -100;
    const int X = (int)rintf(v * ldexpf(1.0f, 20 - E));
    // X + 64 * (2^14 + 2^7 + 1) >= 0 (|X| <= 2^20): its base-128 digits are the
    // balanced digits + 64
    const int Xb = X + 1056832;
    const int c = (Xb & 127) - 64, b = ((Xb >> 7) & 127) - 64, a = (Xb >> 14) - 64;
    const int sx = row16_sum_i(X);
    if (!in) return;
    const int g = k >> 5, l = k & 31;
    dst[g * xjk::kDigStride + l] = (uint8_t)(int8_t)a;
    dst[g * xjk::kDigStride + 32 + l] = (uint8_t)(int8_t)b;
    dst[g * xjk::kDigStride + 64 + l] = (uint8_t)(int8_t)c;
    if (l == 0) ((float *)(dst + o.f_off))[g] = ldexpf(1.0f, E - 20);
    if ((k & 15) == 0) ((int *)(dst + o.sx_off))[k >> 4] = sx;
    if (with_v) ((float *)(dst + o.v_off))[k] = v;
}

// Writes element tid (value v) of one token's block record rec (kHqBlk bytes,
// layout above). Called by all 256 threads of a work-group, tid = threadIdx.x,
// with the block's 256 elements; red4 is 4 floats of LDS. Contains a barrier.
__device__ __forceinline__ void emit_hq(float v, int tid, uint8_t *rec, float *red4) {
    float m = wave_max(fabsf(v));
    if ((tid & 63) == 0) red4[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
    int E = 0;
    (void)frexpf(m, &E);   // m < 2^E
    if (E < -100) E = -100;
    const int e = E - 14;
    const float s = ldexpf(v, -e);
    const _Float16 hi = (_Float16)s;
    const _Float16 lo = (_Float16)(s - (float)hi);   // s - hi is exact in fp32
    ((_Float16 *)rec)[tid] = hi;
    ((_Float16 *)(rec + 512))[tid] = lo;
    float r = (float)hi + (float)lo;
    for (int off = 1; off < 32; off <<= 1) r += __shfl_xor(r, off, 64);
    if ((tid & 31) == 0) ((float *)(rec + 1024))[tid >> 5] = ldexpf(r, e);
    if (tid < 4) ((int *)(rec + 1056))[tid] = tid ? 0 : e;
}

// Sum of x^2 (double) over the 32 lanes of a half-wavefront, in a fixed
// butterfly order; every lane of the half gets the sum.
__device__ __forceinline__ double group_ss(float x) {
    double s = (double)x * x;
    for (int off = 1; off < 32; off <<= 1) s += __shfl_xor(s, off, 64);
    return s;
}

// Cross-work-group hand-off inside one launch. The producers store the
// values a tail will read with system-scope stores (written through every
// cache level) and the tail reads them with system-scope loads (which bypass
// the caches), so no cache write-back or invalidation is needed: a store is
// complete, and visible to such loads, once the storing thread's vmcnt has
// drained. The arrival counter itself is a device-scope atomic.
__device__ __forceinline__ void store_sys(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float load_sys(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// "The last work-group finishes the job": every thread's earlier stores are
// drained, then one thread counts the arrival; returns true (to every
// thread) in the work-group that arrives as number `target`, which also
// resets the counter for the next launch. Every work-group reaches this point
// once and none waits for another.
__device__ __forceinline__ bool arrive_last(int *cnt, int target, int *flag_sh) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int n = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = n == target - 1;
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag_sh = last;
    }
    __syncthreads();
    return *flag_sh != 0;
}

}  // namespace xjd
#endif
