// Bit-exact decode of one 32-element chunk of a row in the device layout
// (see kernels.h). Same products in the same order as xj_dequant_row
// (src/xiaoju-pipe/core/xj_quant.h:57-118): F16 / BF16 widened, Q4_K and
// Q5_K (d*sc)*q - dmin*m, Q6_K (d*sc)*q, Q8_0 d*q. Used by the dequant
// check kernel and by the device-side embedding lookup.
#pragma once
#include "common.h"
#include "xj_abi.h"

namespace xjd {

// chunk c of row `row` (elements 32c .. 32c+31) -> out[0..31]
__device__ __forceinline__ void dequant_chunk(const uint8_t *__restrict__ W, uint32_t type, int64_t K, int64_t nblk,
                                              int64_t row, int64_t c, float *__restrict__ out) {
    if (type == XJ_F32) {
        const float *src = (const float *)W + row * K + c * 32;
        for (int l = 0; l < 32; l++) out[l] = src[l];
    } else if (type == XJ_F16 || type == XJ_BF16) {
        const uint16_t *src = (const uint16_t *)W + row * K + c * 32;
        for (int l = 0; l < 32; l++)
            out[l] = type == XJ_F16 ? f16_to_f32(src[l]) : __uint_as_float((uint32_t)src[l] << 16);
    } else if (type == XJ_Q5_K) {
        // as Q4_K, with bit j of qh[l] (j = the sub-block) as the fifth bit of element l
        const int64_t b = c >> 3;
        const int j = (int)(c & 7), p = j >> 1, hi = j & 1;
        const uint8_t *blk = W + (row * (K / 256) + b) * 176;
        const float d = f16_to_f32(*(const uint16_t *)blk), dmin = f16_to_f32(*(const uint16_t *)(blk + 2));
        const uint8_t *s = blk + 4;
        uint32_t sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float dj = d * (float)sc, mj = dmin * (float)mn;
        const uint8_t *qh = blk + 16, *ql = blk + 48 + 32 * p;
        for (int l = 0; l < 32; l++) {
            const int q = (hi ? (ql[l] >> 4) : (ql[l] & 0xF)) + (((qh[l] >> j) & 1) << 4);
            out[l] = dj * (float)q - mj;
        }
    } else if (type == XJ_Q8_0) {
        const int64_t g = row * (K / 32) + c;
        const float d = f16_to_f32(*(const uint16_t *)(W + nblk * 32 + g * 2));
        const int8_t *q = (const int8_t *)(W + g * 32);
        for (int l = 0; l < 32; l++) out[l] = d * (float)q[l];
    } else if (type == XJ_Q4_K) {
        // chunk = sub-block j of block b: low nibbles (j even) or high nibbles (j odd) of pair j/2
        const int64_t b = c >> 3;
        const int j = (int)(c & 7), p = j >> 1, hi = j & 1;
        const uint8_t *blk = W + (row * (K / 256) + b) * 144;
        const float d = f16_to_f32(*(const uint16_t *)blk), dmin = f16_to_f32(*(const uint16_t *)(blk + 2));
        const uint8_t *s = blk + 4;
        uint32_t sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float dj = d * (float)sc, mj = dmin * (float)mn;
        const uint8_t *qs = blk + 16 + 32 * p;
        for (int l = 0; l < 32; l++) {
            const int q = hi ? (qs[l] >> 4) : (qs[l] & 0xF);
            out[l] = dj * (float)q - mj;
        }
    } else if (type == XJ_Q6_K) {
        const int64_t g = row * (K / 256) + (c >> 3);
        const uint8_t *ql = W + g * 128, *qh = W + nblk * 128 + g * 64;
        const int8_t *sc = (const int8_t *)(W + nblk * 192 + g * 16);
        const float d = f16_to_f32(*(const uint16_t *)(W + nblk * 208 + g * 2));
        const int e0 = (int)(c & 7) * 32;       // elements e0 .. e0+31 of the block
        const int h = e0 >> 7, G = (e0 >> 5) & 3;
        for (int l = 0; l < 32; l++) {
            const uint8_t lo = ql[64 * h + 32 * (G & 1) + l];
            const int nib = G < 2 ? (lo & 0xF) : (lo >> 4);
            const int q = (nib | (((qh[32 * h + l] >> (2 * G)) & 3) << 4)) - 32;
            out[l] = d * (float)sc[(e0 + l) >> 4] * (float)q;
        }
    } else {
        for (int l = 0; l < 32; l++) out[l] = 0.f;
    }
}

__host__ __device__ inline int64_t dev_nblk(uint32_t type, int64_t n_rows, int64_t k) {
    return type == XJ_Q8_0 ? n_rows * (k / 32) : n_rows * (k / 256);
}

}  // namespace xjd
