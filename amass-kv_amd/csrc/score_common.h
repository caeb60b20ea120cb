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
// qs = max(amax, 1e-12) / 16383 and inv = 16383 / max(amax, 1e-12) (one IEEE divide
// each per head), qi = rint(q * inv) clamped to +-16383, hi = rint(qi / 128) clamped to
// +-127, lo = qi - 128 hi.  Returns packed hi/lo words (4 d per word, d ascending in
// bytes), qs and sum(qi) over the unit's full d (8 lanes x 16).
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
    mx = fmaxf(unit8_maxf(mx), 1e-12f);
    qs = mx / 16383.0f;                // correctly rounded divides
    const float inv = 16383.0f / mx;
    int s = 0;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        uint32_t hv = 0, lv = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int qi = (int)rintf(__fmul_rn(f[4 * wi + j], inv));
            qi = max(-16383, min(16383, qi));
            int h = (int)rintf((float)qi * 0.0078125f);
            h = max(-127, min(127, h));
            const int l = qi - 128 * h;           // |l| <= 64
            s += qi;
            hv |= ((uint32_t)(h & 0xFF)) << (8 * j);
            lv |= ((uint32_t)(l & 0xFF)) << (8 * j);
        }
        hw[wi] = hv;
        lw[wi] = lv;
    }
    qsum = unit8_sum(s);
}

// comb = sum over the lane's 16 d of qi * x = 128 * (hi . x) + (lo . x), exact in int32:
// the lo chain starts from the shifted hi sum, so no separate combine is needed.
__device__ __forceinline__ int dot16_2limb(const uint32_t (&qh)[4], const uint32_t (&ql)[4],
                                           const uint32_t x0, const uint32_t x1,
                                           const uint32_t x2, const uint32_t x3) {
    int ah = sdot4(qh[0], x0, 0);
    ah = sdot4(qh[1], x1, ah);
    ah = sdot4(qh[2], x2, ah);
    ah = sdot4(qh[3], x3, ah);
    int al = sdot4(ql[0], x0, ah << 7);
    al = sdot4(ql[1], x1, al);
    al = sdot4(ql[2], x2, al);
    return sdot4(ql[3], x3, al);
}

// Transpose-reduce of an 8-lane unit: v holds G x (RP+1) per-lane partial sums ordered
// [g][k].  Each split step halves the g range (the lane keeps the half selected by one bit
// of its unit index and adds the partner's copy of it via DPP); after log2(G) splits the
// remaining steps are plain butterflies.  On return out[k] is the unit-wide sum of
// column k for g = unit_g(lane) = sum_i bit_(2-i)(sub) << (log2(G)-1-i).
template <int G, int RP>
__device__ __forceinline__ void unit8_reduce_own_g(const int (&v)[G][RP + 1], int sub,
                                                   int (&out)[RP + 1]) {
    constexpr int K = RP + 1;
    if constexpr (G == 1) {
#pragma unroll
        for (int k = 0; k < K; ++k) out[k] = unit8_sum(v[0][k]);
    } else if constexpr (G == 2) {
        const bool up = (sub >> 2) & 1;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int send = up ? v[0][k] : v[1][k];
            const int keep = up ? v[1][k] : v[0][k];
            int x = keep + dpp_i<DPP_HALF_MIRROR>(send);
            x += dpp_i<DPP_XOR2>(x);
            x += dpp_i<DPP_XOR1>(x);
            out[k] = x;
        }
    } else if constexpr (G == 4) {
        const bool u2 = (sub >> 2) & 1, u1 = (sub >> 1) & 1;
        int h[2][K];
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int send = u2 ? v[gg][k] : v[gg + 2][k];
                const int keep = u2 ? v[gg + 2][k] : v[gg][k];
                h[gg][k] = keep + dpp_i<DPP_HALF_MIRROR>(send);
            }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int send = u1 ? h[0][k] : h[1][k];
            const int keep = u1 ? h[1][k] : h[0][k];
            int x = keep + dpp_i<DPP_XOR2>(send);
            out[k] = x + dpp_i<DPP_XOR1>(x);
        }
    } else {  // G == 8
        const bool u2 = (sub >> 2) & 1, u1 = (sub >> 1) & 1, u0 = sub & 1;
        int h[4][K];
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int send = u2 ? v[gg][k] : v[gg + 4][k];
                const int keep = u2 ? v[gg + 4][k] : v[gg][k];
                h[gg][k] = keep + dpp_i<DPP_HALF_MIRROR>(send);
            }
        int e[2][K];
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int send = u1 ? h[gg][k] : h[gg + 2][k];
                const int keep = u1 ? h[gg + 2][k] : h[gg][k];
                e[gg][k] = keep + dpp_i<DPP_XOR2>(send);
            }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int send = u0 ? e[0][k] : e[1][k];
            const int keep = u0 ? e[1][k] : e[0][k];
            out[k] = keep + dpp_i<DPP_XOR1>(send);
        }
    }
}

// Per-column variant: reduce the G per-lane partial sums of ONE column to the unit-wide
// sum for the lane's own g (same split/butterfly schedule as unit8_reduce_own_g), so the
// caller can reduce each column as soon as its dot products exist.
template <int G>
__device__ __forceinline__ int unit8_reduce_col(const int (&v)[G], int sub) {
    if constexpr (G == 1) {
        return unit8_sum(v[0]);
    } else if constexpr (G == 2) {
        const bool up = (sub >> 2) & 1;
        int x = (up ? v[1] : v[0]) + dpp_i<DPP_HALF_MIRROR>(up ? v[0] : v[1]);
        x += dpp_i<DPP_XOR2>(x);
        return x + dpp_i<DPP_XOR1>(x);
    } else if constexpr (G == 4) {
        const bool u2 = (sub >> 2) & 1, u1 = (sub >> 1) & 1;
        const int h0 = (u2 ? v[2] : v[0]) + dpp_i<DPP_HALF_MIRROR>(u2 ? v[0] : v[2]);
        const int h1 = (u2 ? v[3] : v[1]) + dpp_i<DPP_HALF_MIRROR>(u2 ? v[1] : v[3]);
        const int x = (u1 ? h1 : h0) + dpp_i<DPP_XOR2>(u1 ? h0 : h1);
        return x + dpp_i<DPP_XOR1>(x);
    } else {
        const bool u2 = (sub >> 2) & 1, u1 = (sub >> 1) & 1, u0 = sub & 1;
        int h[4];
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
            h[gg] = (u2 ? v[gg + 4] : v[gg]) + dpp_i<DPP_HALF_MIRROR>(u2 ? v[gg] : v[gg + 4]);
        const int e0 = (u1 ? h[2] : h[0]) + dpp_i<DPP_XOR2>(u1 ? h[0] : h[2]);
        const int e1 = (u1 ? h[3] : h[1]) + dpp_i<DPP_XOR2>(u1 ? h[1] : h[3]);
        return (u0 ? e1 : e0) + dpp_i<DPP_XOR1>(u0 ? e0 : e1);
    }
}

template <int G>
__device__ __forceinline__ int unit_g(int sub) {
    if constexpr (G == 1) return 0;
    else if constexpr (G == 2) return (sub >> 2) & 1;
    else if constexpr (G == 4) return ((sub >> 2) & 1) * 2 + ((sub >> 1) & 1);
    else return ((sub >> 2) & 1) * 4 + ((sub >> 1) & 1) * 2 + (sub & 1);
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
