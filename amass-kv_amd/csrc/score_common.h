// Front end shared by the quad and r8 page-score kernels (gfx950): 2-limb int8 query
// words, (d, r) int8/int4 code rows -> d-contiguous dot4 words, fp16 scale vectors.
#pragma once
#include "common.h"

namespace amass {

// ---- V rows -> d-contiguous int8 words: w[k][wi] = rows 4wi..4wi+3 of column k -------
template <int RP, int VB>
__device__ __forceinline__ void unpack_v(const uint32_t* raw, uint32_t (&w)[RP][4]) {
    if constexpr (VB == 8 && RP == 8) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi)
#pragma unroll
            for (int kq = 0; kq < 2; ++kq)
                transpose4x4(raw[2 * (4 * wi + 0) + kq], raw[2 * (4 * wi + 1) + kq],
                             raw[2 * (4 * wi + 2) + kq], raw[2 * (4 * wi + 3) + kq],
                             w[4 * kq + 0][wi], w[4 * kq + 1][wi], w[4 * kq + 2][wi],
                             w[4 * kq + 3][wi]);
    } else if constexpr (VB == 8 && RP == 4) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi)
            transpose4x4(raw[4 * wi + 0], raw[4 * wi + 1], raw[4 * wi + 2], raw[4 * wi + 3],
                         w[0][wi], w[1][wi], w[2][wi], w[3][wi]);
    } else if constexpr (VB == 8 && RP == 2) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            const uint32_t a = raw[2 * wi], b = raw[2 * wi + 1];
            w[0][wi] = perm(b, a, 0x06040200u);
            w[1][wi] = perm(b, a, 0x07050301u);
        }
    } else if constexpr (VB == 4 && RP == 8) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t x = raw[4 * wi + i] ^ 0x88888888u;
                lo[i] = x & 0x0F0F0F0Fu;
                hi[i] = (x >> 4) & 0x0F0F0F0Fu;
            }
            transpose4x4(lo[0], lo[1], lo[2], lo[3], w[0][wi], w[2][wi], w[4][wi], w[6][wi]);
            transpose4x4(hi[0], hi[1], hi[2], hi[3], w[1][wi], w[3][wi], w[5][wi], w[7][wi]);
        }
    } else if constexpr (VB == 4 && RP == 4) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            const uint32_t a = raw[2 * wi] ^ 0x88888888u, b = raw[2 * wi + 1] ^ 0x88888888u;
            const uint32_t alo = a & 0x0F0F0F0Fu, ahi = (a >> 4) & 0x0F0F0F0Fu;
            const uint32_t blo = b & 0x0F0F0F0Fu, bhi = (b >> 4) & 0x0F0F0F0Fu;
            w[0][wi] = perm(blo, alo, 0x06040200u);
            w[2][wi] = perm(blo, alo, 0x07050301u);
            w[1][wi] = perm(bhi, ahi, 0x06040200u);
            w[3][wi] = perm(bhi, ahi, 0x07050301u);
        }
    } else if constexpr (VB == 4 && RP == 2) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            const uint32_t x = raw[wi] ^ 0x88888888u;
            w[0][wi] = x & 0x0F0F0F0Fu;
            w[1][wi] = (x >> 4) & 0x0F0F0F0Fu;
        }
    }
}

// ---- 2-limb int8 query words for 16 d of head row `qrow` ------------------------------
// Returns packed hi/lo words (4 d per word, d ascending in bytes), qs and sum(qi) over
// the unit's full d (8 lanes x 16).
__device__ __forceinline__ void quantize_q16(const uint16_t* qrow, uint32_t (&hw)[4],
                                             uint32_t (&lw)[4], float& qs, int& qsum) {
    const uint4 a = *reinterpret_cast<const uint4*>(qrow);
    const uint4 b = *reinterpret_cast<const uint4*>(qrow + 8);
    const uint32_t raw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float f[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        f[2 * i] = bf16lo(raw[i]);
        f[2 * i + 1] = bf16hi(raw[i]);
    }
    float mx = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, fabsf(f[e]));
    mx = unit8_maxf(mx);
    qs = fmaxf(mx, 1e-12f) / 16383.0f;  // correctly rounded divide
    int s = 0;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        uint32_t hv = 0, lv = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int qi = (int)rintf(f[4 * wi + j] / qs);
            qi = max(-16383, min(16383, qi));
            int h = (int)rintf((float)qi * 0.0078125f);
            h = max(-127, min(127, h));
            int l = max(-127, min(127, qi - 128 * h));
            s += qi;
            hv |= ((uint32_t)(h & 0xFF)) << (8 * j);
            lv |= ((uint32_t)(l & 0xFF)) << (8 * j);
        }
        hw[wi] = hv;
        lw[wi] = lv;
    }
    qsum = unit8_sum(s);
}

template <int RP>
__device__ __forceinline__ void load_scales(const uint16_t* base, float (&out)[RP]) {
    if constexpr (RP == 8) {
        const uint4 u = *reinterpret_cast<const uint4*>(base);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = fp16_to_f32((uint16_t)(w[i] & 0xFFFF));
            out[2 * i + 1] = fp16_to_f32((uint16_t)(w[i] >> 16));
        }
    } else if constexpr (RP == 4) {
        const uint2 u = *reinterpret_cast<const uint2*>(base);
        out[0] = fp16_to_f32((uint16_t)(u.x & 0xFFFF));
        out[1] = fp16_to_f32((uint16_t)(u.x >> 16));
        out[2] = fp16_to_f32((uint16_t)(u.y & 0xFFFF));
        out[3] = fp16_to_f32((uint16_t)(u.y >> 16));
    } else {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(base);
        out[0] = fp16_to_f32((uint16_t)(u & 0xFFFF));
        out[1] = fp16_to_f32((uint16_t)(u >> 16));
    }
}

}  // namespace amass
