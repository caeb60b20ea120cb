// Low-rank per-key logsumexp page scores for gfx950: r8 and CLSE (the kernel shared by
// r8_score.hip and clse_score.hip).
//
// Math per (request r, kv-head h, page p < n_sel_hi[r]) and GQA head g (reference:
// selection/score.py:3-16,30-120; int path selection/score_cuda.py:160-448):
//   q~[g,k]  = (Vk_code[:,k] * Vk_scale[k]) . q_g                       k < r
//   tok[g,t] = s * c_scale[t] * (c_code[t,:] . q~[g,:])                t < page, 16p+t < seq_len
//   S_g      = s * (mu_code * mu_scale) . q_g + logsumexp_t tok[g,t]
//   score    = max_g S_g   (kv-union group max)
//
// Front end: the quad kernel's int8 matrix-core product (score_mfma.h) over the page's
// tiled Vk and its mean codes -- exact int32 sums comb = sum_d qi * code.  The Vk product
// runs on column groups (16 / r pages x r ranks, loads of 64 r contiguous bytes per page,
// non-temporal); its int32 pairs go through a per-wave LDS transpose back to one page
// per lane -- lane n carries page lane_page(n) of the tile, whose mu codes, scales and c
// rows it loads.  For G < 8 the unused M rows repeat the group's limb rows, so lane
// (kg, n) receives the sums of heads g0 = 2 (kg % GP), g1 = g0 + 1 (GP = max(G/2, 1)
// head pairs) and the 4 / GP lane groups holding the same pair split the page's 16 tokens
// between them (TPL tokens each): the token tail needs no exchange of q~, only a max and
// a sum across those groups for the logsumexp, and a max across pairs for the group max.
//
// r8 layout (AMASS_R8_REC_BYTES per kv head).  Per block, the n_kv heads' records
// [Vk tiled: 16 bytes per (K-step t, d group kg, column k) at ((t * 4 + kg) * r + k) * 16
// (int4: t folded into the nibbles) | 128 mu codes | c: 16 token rows of r * c_bits / 8
// bytes], then the n_kv heads' 64-byte fp16 scale blocks (Vk_scale at half 0, c_scale at
// halves 8..23, mu_scale at half 24).  c rows keep the reference order (int4: two columns
// per byte, low nibble = even column).  Each tile is two load groups -- column groups
// [0, r/2) + mu + scales, then [r/2, r) + the lane's c rows -- double-buffered as in the
// quad kernel.
//
// CLSE (reference selection/quad_score.py:156-276, score="clse") is the same computation
// over its quad_V / quad_mu / quad_c / c_scale and the residual scatter energy, plus an
// isotropic term for the key variance outside the stored subspace:
//   iso_g = max(|q_g|^2 - |q~_g|^2, 0) * resid * s^2 / (2 P (d - r))
//   S_g   = s mu.q_g + logsumexp_t tok[g,t] + iso_g ; combine "max" or per head ("nrm").
// |q_g|^2 comes from the bf16 query in fp32, |q~_g|^2 from the lane's own q~.
// Its record (AMASS_CLSE_REC_BYTES per kv head) keeps no dead bytes in the lines it
// streams: per block the n_kv heads' [V tiled | 128 mu codes] (whole lines), then per
// head a tail of TB bytes: the c rows, then fp16 c_scale[0..16), V_scale[0..r) at half
// 16, mu_scale at half 16 + r and the residual at half 17 + r.  (The r8 layout's 64-byte
// scale block leaves 24 of its bytes unused at r = 2, and its 272-byte head records at
// r = 2, int4 split lines between heads.)  The lanes load the tail's scale part so that
// `meta` holds what the r8 layout's 16 bytes kg would: lane group 0 the V scales (bytes
// 32.., which at r <= 4 also hold mu_scale and the residual), 1 and 2 the c scales of
// tokens 0..7 and 8..15, 3 at r = 8 the bytes 48.. (mu_scale and the residual; at
// r <= 4 it repeats group 0's load).
#pragma once
#include "score_mfma.h"

namespace amass {

constexpr int R8_MAXW = 8;      // waves (kv heads) per workgroup

struct R8Params {
    const uint16_t* q; int64_t q_st, q_hs;
    const int8_t* rec; int64_t rec_sb;
    const int32_t* bt; int64_t bt_st;
    const int32_t* sl;
    const int32_t* nsh;
    float* score; int64_t sc_sr, sc_sh;
    float* score_h; int64_t sh_sr, sh_sh, sh_sg;   // CLSE per-head output (combine 1)
    float* tmax; int64_t tm_sr, tm_sh, tm_sg;      // optional per-tile per-head maxima (nrm)
    int c_fp32;                                   // r8: one fp32 c scale per page
    int32_t* comb_out;
    float scale;
    float iso_coef;                               // CLSE: s^2 / (2 P (d - r))
    float scale_l2;                               // scale * log2(e) (base-2 token logits)
    float iso_k;                                  // iso_coef / scale_l2^2
    int combine;                                  // CLSE: 0 group max, 1 per head
    int n_req, n_kv, page, max_pages;
    int hw;         // kv heads (waves) per workgroup
    int target;     // workgroups the batch's tiles are balanced over
};

template <int RP, int VB, int CBITS, bool CLSE>
struct R8Geom {
    static constexpr int CB = col_bytes<VB>();
    static constexpr int CROW = RP * CBITS / 8;          // bytes per token row of c
    // a head's record before the scales (r8: V, mu, c) or before its tail (CLSE: V, mu)
    static constexpr int VM = RP * CB + 128 + (CLSE ? 0 : 16 * CROW);
    // bytes of a head's scale block (r8) or tail (CLSE: c rows + scale part)
    static constexpr int TB = CLSE ? 16 * CROW + 16 * ((36 + 2 * RP + 15) / 16) : 64;
    // V loads non-temporal for whole-line records with runs of >= 256 bytes per page; at
    // r = 2 (128-byte runs) plain loads measured faster (CLSE config-1 shape: 20.1 against
    // 20.4-20.7 us)
    static constexpr bool NT = VM % 128 == 0 && RP >= 4;
};

template <int G>
struct R8Split {
    static constexpr int GP = G >= 2 ? G / 2 : 1;       // head pairs over the 4 lane groups
    static constexpr int TPL = 4 * GP;                  // tokens per lane (16 / (4 / GP))
};

template <int RP, int VB>
struct R8GroupA {                         // column groups [0, RP/2), mu, the page's scales
    static constexpr int NG = RP / 2;
    i32x4_t v[NG * loads_per_col<VB>()];
    i32x4_t mu[2];
    i32x4_t meta;                         // 16 bytes kg of the 64-byte scale block
};
template <int RP, int VB>
struct R8GroupB {                         // column groups [RP/2, RP)
    static constexpr int NG = RP - RP / 2;
    i32x4_t v[NG * loads_per_col<VB>()];
};
template <int CL>
struct R8GroupC {                         // the lane's c rows
    uint32_t c[CL / 4];
};

// group j's V at rec + gb[j] (the record offset of the lane's group page j) + lv (h * VM +
// the lane's V offset); `lr` = the lane's own-page record (its block's records + h * VM +
// 16 kg), `moff` = its 16 bytes of the scale block (r8) or tail (CLSE) - lr
template <int RP, int VB, bool NT>
__device__ __forceinline__ void r8_load_a(const int8_t* rec, int lv, const int (&gb)[RP],
                                          const int8_t* lr, R8GroupA<RP, VB>& a, int moff) {
    load_groups<RP, VB, 0, RP / 2, NT>(rec, lv, gb, a.v);
    a.mu[0] = ld16(lr + RP * col_bytes<VB>());
    a.mu[1] = ld16(lr + RP * col_bytes<VB>() + 64);
    a.meta = ld16(lr + moff);
}

template <int RP, int VB, bool NT>
__device__ __forceinline__ void r8_load_b(const int8_t* rec, int lv, const int (&gb)[RP],
                                          R8GroupB<RP, VB>& b) {
    load_groups<RP, VB, RP / 2, RP - RP / 2, NT>(rec, lv, gb, b.v);
}

template <int CL>
__device__ __forceinline__ void r8_load_c(const int8_t* cp, R8GroupC<CL>& g) {
    if constexpr (CL >= 16) {
#pragma unroll
        for (int i = 0; i < CL / 16; ++i) {
            const i32x4_t x = ld16(cp + 16 * i);
            g.c[4 * i] = (uint32_t)x[0]; g.c[4 * i + 1] = (uint32_t)x[1];
            g.c[4 * i + 2] = (uint32_t)x[2]; g.c[4 * i + 3] = (uint32_t)x[3];
        }
    } else if constexpr (CL == 8) {
        const uint2 x = *reinterpret_cast<const uint2*>(cp);
        g.c[0] = x.x; g.c[1] = x.y;
    } else {                              // CL == 4 (r = 2, int4 c, G <= 2)
        g.c[0] = *reinterpret_cast<const uint32_t*>(cp);
    }
}

// fp16 scales of one page for this lane: Vk_scale (from lane group 0), mu_scale (group 3)
// and the c_scale of the lane's TPL tokens (groups 1 and 2 hold tokens 0..7 / 8..15).
template <int RP, int TPL>
struct R8Scales {
    uint32_t vs[4];
    float mus;
    float resid;                          // CLSE residual energy (half 25)
    float cs[TPL];
};

template <int RP, int TPL, bool CLSE>
__device__ __forceinline__ R8Scales<RP, TPL> r8_gather_scales(i32x4_t meta, int n, int part,
                                                              bool c_fp32) {
    R8Scales<RP, TPL> s;
    constexpr int NW = RP / 2;            // dwords holding r halves
#pragma unroll
    for (int i = 0; i < 4; ++i) s.vs[i] = i < NW ? (uint32_t)__shfl(meta[i], n, WAVE) : 0u;
    // mu_scale and the residual: halves 24, 25 of the r8 scale block (lane group 3); in
    // the CLSE tail at r <= 4 they follow the V scales in lane group 0's dword r / 2
    uint32_t w24;
    if constexpr (CLSE && RP <= 4) w24 = (uint32_t)__shfl(meta[RP / 2], n, WAVE);
    else w24 = (uint32_t)__shfl(meta[0], n + 48, WAVE);
    s.mus = fp16_to_f32((uint16_t)(w24 & 0xFFFFu));
    s.resid = fp16_to_f32((uint16_t)(w24 >> 16));
    if (c_fp32) {                         // one fp32 for the page: bytes 16..19 (group 1)
        const float c = __uint_as_float((uint32_t)__shfl(meta[0], n + 16, WAVE));
#pragma unroll
        for (int t = 0; t < TPL; ++t) s.cs[t] = c;
        return s;
    }
    if constexpr (TPL == 16) {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = (uint32_t)__shfl(meta[i], n + 16, WAVE);
            w[4 + i] = (uint32_t)__shfl(meta[i], n + 32, WAVE);
        }
#pragma unroll
        for (int t = 0; t < 16; ++t)
            s.cs[t] = fp16_to_f32((uint16_t)((w[t >> 1] >> (16 * (t & 1))) & 0xFFFFu));
    } else {
        const int t0 = part * TPL;        // first token of the lane
        const int src = n + 16 * (1 + (t0 >> 3));
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (uint32_t)__shfl(meta[i], src, WAVE);
        if constexpr (TPL == 8) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                s.cs[t] = fp16_to_f32((uint16_t)((w[t >> 1] >> (16 * (t & 1))) & 0xFFFFu));
        } else {                          // TPL == 4: tokens t0 % 8 .. + 4 of the source
            const bool up = (t0 & 7) != 0;
            const uint32_t x0 = up ? w[2] : w[0], x1 = up ? w[3] : w[1];
            s.cs[0] = fp16_to_f32((uint16_t)(x0 & 0xFFFFu));
            s.cs[1] = fp16_to_f32((uint16_t)(x0 >> 16));
            s.cs[2] = fp16_to_f32((uint16_t)(x1 & 0xFFFFu));
            s.cs[3] = fp16_to_f32((uint16_t)(x1 >> 16));
        }
    }
    return s;
}

// q~ of the lane's two heads (e = 0: g0, e = 1: g1) times scale * log2(e), and their mu
// terms.
template <int RP>
struct R8Acc {
    float qt[2][RP];
    float qmu[2];
};

template <int RP>
__device__ __forceinline__ int32_t* r8_comb_row(const R8Params& p, int G, int req, int h,
                                                int page, int g) {
    return p.comb_out + (((int64_t)req * p.n_kv + h) * p.max_pages + page) * (G * (RP + 1)) +
           (int64_t)g * (RP + 1);
}

// The int32 contractions of the column groups pass through LDS back to one page per
// lane: lane (kg, n) of group j stores its (g0, g1) pair at [kg][page j PP + n / r][rank
// n % r]; after the last group, lane n reads the r ranks of its own page lane_page(n).
struct __align__(16) R8Lds {
    int2 x[R8_MAXW][4][SC_TILE][8];
};

template <int RP, int VB, int J0, int NG>
__device__ __forceinline__ void r8_groups(const i32x4_t (&qa)[2], const i32x4_t* v,
                                          int2 (&row)[SC_TILE][8], int n) {
    constexpr int PP = group_pages<RP>();
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        int x0, x1;
        comb2<VB>(col_mfma<VB>(qa, &v[j * loads_per_col<VB>()]), x0, x1);
        row[(J0 + j) * PP + n / RP][n % RP] = make_int2(x0, x1);
    }
}

template <int RP, int VB, int G, bool COMB>
__device__ __forceinline__ void r8_tile_start(const R8Params& p, const i32x4_t (&qa)[2],
                                              const R8GroupA<RP, VB>& a,
                                              const R8Scales<RP, R8Split<G>::TPL>& sc, float qs0,
                                              float qs1, R8Acc<RP>& acc, int2 (&row)[SC_TILE][8],
                                              int req, int h, int page, bool valid, int pair,
                                              int part, int n) {
    r8_groups<RP, VB, 0, RP / 2>(qa, a.v, row, n);
    i32x4_t m = {0, 0, 0, 0};
    m = mfma_i8(qa[0], a.mu[0], m);
    m = mfma_i8(qa[1], a.mu[1], m);
    const int cmu[2] = {m[0] * 128 + m[1], m[2] * 128 + m[3]};
    acc.qmu[0] = (float)cmu[0] * qs0 * sc.mus * p.scale;
    acc.qmu[1] = (float)cmu[1] * qs1 * sc.mus * p.scale;
    if (COMB && valid && part == 0) {
        r8_comb_row<RP>(p, G, req, h, page, 2 * pair)[RP] = cmu[0];
        if (G >= 2) r8_comb_row<RP>(p, G, req, h, page, 2 * pair + 1)[RP] = cmu[1];
    }
}

template <int RP, int VB, int G, bool COMB>
__device__ __forceinline__ void r8_tile_mid(const R8Params& p, const i32x4_t (&qa)[2],
                                            const R8GroupB<RP, VB>& b,
                                            const R8Scales<RP, R8Split<G>::TPL>& sc, float qs0,
                                            float qs1, R8Acc<RP>& acc, int2 (&row)[SC_TILE][8],
                                            int req, int h, int page, bool valid, int pair,
                                            int part, int n) {
    r8_groups<RP, VB, RP / 2, RP - RP / 2>(qa, b.v, row, n);
    int2 x[8];
    const int own = lane_page<RP>(n);
#pragma unroll
    for (int k = 0; k < RP; k += 2) {
        const int4 w = *reinterpret_cast<const int4*>(&row[own][k]);
        x[k] = make_int2(w.x, w.y);
        x[k + 1] = make_int2(w.z, w.w);
    }
    const bool co_on = COMB && valid && part == 0;
    int32_t* co0 = co_on ? r8_comb_row<RP>(p, G, req, h, page, 2 * pair) : nullptr;
    int32_t* co1 = (co_on && G >= 2) ? r8_comb_row<RP>(p, G, req, h, page, 2 * pair + 1)
                                     : nullptr;
#pragma unroll
    for (int k = 0; k < RP; ++k) {
        const float vsc = half_at(sc.vs, k);
        acc.qt[0][k] = (float)x[k].x * (qs0 * p.scale_l2) * vsc;
        acc.qt[1][k] = (float)x[k].y * (qs1 * p.scale_l2) * vsc;
        if (co0) co0[k] = x[k].x;
        if (co1) co1[k] = x[k].y;
    }
}

// Code k of token row t of the lane's c words as a float.  int8: the signed byte.
// int4: from `cu`, the words with every nibble's sign bit flipped and split into low
// (cu[2i]) and high (cu[2i + 1]) nibbles, one per byte -- the nibble's value + 8, taken
// with one byte conversion; the caller subtracts 8 sum_k q~_k once per head.
template <int RP, int CBITS>
__device__ __forceinline__ float c_code(const uint32_t* cw, const uint32_t* cu, int t, int k) {
    constexpr int CROW = RP * CBITS / 8;
    if constexpr (CBITS == 8) {
        const int byte = t * CROW + k;
        return (float)(((int)(cw[byte >> 2] << (24 - 8 * (byte & 3)))) >> 24);
    } else {
        const int nib = t * 2 * CROW + k;       // low nibble = even column
        const uint32_t w = cu[2 * (nib >> 3) + (nib & 1)];
        return (float)((w >> (8 * ((nib & 7) >> 1))) & 0xFFu);
    }
}

// Token logits and their logsumexp over the lane's TPL tokens, in base 2: acc.qt holds
// q~ * scale * log2(e) (so a logit is c_scale * c . qt), the logsumexp is
// ln 2 (m + log2 sum 2^(l - m)) on the hardware's exp2 / log2; tokens >= seq_len are
// masked.  (An unmasked variant for the tiles that end below seq_len measured slower: the
// compiler's schedule for it needs more registers and the launch loses a wave per SIMD.)
template <int RP, int CBITS, int G>
__device__ __forceinline__ void r8_lse(const R8GroupC<R8Split<G>::TPL * RP * CBITS / 8>& b,
                                       const R8Scales<RP, R8Split<G>::TPL>& sc,
                                       const R8Acc<RP>& acc, int tok0, int sl, float (&lse)[2]) {
    constexpr int TPL = R8Split<G>::TPL;
    constexpr int GP = R8Split<G>::GP;
    constexpr int NCW = TPL * RP * CBITS / 32 > 0 ? TPL * RP * CBITS / 32 : 1;
    uint32_t cu[CBITS == 4 ? 2 * NCW : 1];
    float a0i = 0.f, a1i = 0.f;
    if constexpr (CBITS == 4) {
#pragma unroll
        for (int i = 0; i < NCW; ++i) {
            const uint32_t x = b.c[i] ^ 0x88888888u;
            cu[2 * i] = x & 0x0F0F0F0Fu;
            cu[2 * i + 1] = (x >> 4) & 0x0F0F0F0Fu;
        }
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < RP; ++k) {
            s0 += acc.qt[0][k];
            s1 += acc.qt[1][k];
        }
        a0i = -8.f * s0;
        a1i = -8.f * s1;
    }
    float lg[2][TPL];
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
        float a0 = a0i, a1 = a1i;
#pragma unroll
        for (int k = 0; k < RP; ++k) {
            const float cf = c_code<RP, CBITS>(b.c, cu, t, k);
            a0 += cf * acc.qt[0][k];
            a1 += cf * acc.qt[1][k];
        }
        lg[0][t] = a0 * sc.cs[t];
        lg[1][t] = a1 * sc.cs[t];
        if (tok0 + t >= sl) {
            lg[0][t] = -INFINITY;
            lg[1][t] = -INFINITY;
        }
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        float m = lg[e][0];
#pragma unroll
        for (int t = 1; t < TPL; ++t) m = fmaxf(m, lg[e][t]);
        if constexpr (GP == 2) m = xor32_maxf(m);
        if constexpr (GP == 1) m = xor32_maxf(xor16_maxf(m));
        const float mm = m == -INFINITY ? 0.f : m;
        float se = 0.f;
#pragma unroll
        for (int t = 0; t < TPL; ++t) se += __builtin_amdgcn_exp2f(lg[e][t] - mm);
        if constexpr (GP == 2) se = xor32_sumf(se);
        if constexpr (GP == 1) se = xor32_sumf(xor16_sumf(se));
        lse[e] = 0.69314718055994531f * (m + __builtin_amdgcn_logf(se));
    }
}

// CLSE: acc.qt carries scale log2 e, so |q~|^2 takes p.iso_k = iso_coef / (scale log2 e)^2.
template <int RP, int CBITS, int G, bool CLSE>
__device__ __forceinline__ void r8_tile_tail(const R8Params& p,
                                             const R8GroupC<R8Split<G>::TPL * RP * CBITS / 8>& b,
                                             const R8Scales<RP, R8Split<G>::TPL>& sc,
                                             const R8Acc<RP>& acc, int req, int h, int page,
                                             bool valid, int pair, int part, int kg, int sl,
                                             float qsq0, float qsq1) {
    constexpr int TPL = R8Split<G>::TPL;
    constexpr int GP = R8Split<G>::GP;
    float lse[2];
    r8_lse<RP, CBITS, G>(b, sc, acc, page * p.page + part * TPL, sl, lse);
    float S[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        S[e] = acc.qmu[e] + lse[e];
        if constexpr (CLSE) {
            float qh = 0.f;
#pragma unroll
            for (int k = 0; k < RP; ++k) qh = fmaf(acc.qt[e][k], acc.qt[e][k], qh);
            S[e] += fmaxf((e ? qsq1 : qsq0) * p.iso_coef - qh * p.iso_k, 0.f) * sc.resid;
        }
    }
    if (CLSE && p.combine == 1) {             // per-head scores (the nrm combine's input)
        if (valid && part == 0) {
            const int64_t row = (int64_t)req * p.sh_sr + (int64_t)h * p.sh_sh + page;
            p.score_h[row + (int64_t)(2 * pair) * p.sh_sg] = S[0];
            if (G >= 2) p.score_h[row + (int64_t)(2 * pair + 1) * p.sh_sg] = S[1];
        }
        if (p.tmax) {
            // the tile's maximum per head: the 16 lanes of row kg hold its 16 pages
            float m0 = valid ? S[0] : -INFINITY, m1 = valid ? S[1] : -INFINITY;
            m0 = row16_maxf(m0);
            m1 = row16_maxf(m1);
            if (part == 0 && (threadIdx.x & 15) == 0) {
                const int64_t t = (int64_t)req * p.tm_sr + (int64_t)h * p.tm_sh +
                                  page / SC_TILE;
                p.tmax[t + (int64_t)(2 * pair) * p.tm_sg] = m0;
                if (G >= 2) p.tmax[t + (int64_t)(2 * pair + 1) * p.tm_sg] = m1;
            }
        }
        return;
    }
    float smax = G >= 2 ? fmaxf(S[0], S[1]) : S[0];
    if constexpr (GP == 4) smax = xor32_maxf(xor16_maxf(smax));
    if constexpr (GP == 2) smax = xor16_maxf(smax);
    if (valid && kg == 0) p.score[(int64_t)req * p.sc_sr + (int64_t)h * p.sc_sh + page] = smax;
}

// COMB: also write the int32 contractions to comb_out (a test entry).  CLSE: the CLSE
// score (iso term, optional per-head output) instead of r8.
template <int RP, int VB, int CBITS, int G, bool COMB, bool CLSE>
__global__ __launch_bounds__(R8_MAXW * WAVE)
void r8_score_kernel(const R8Params p) {
    using Geo = R8Geom<RP, VB, CBITS, CLSE>;
    constexpr int VM = Geo::VM;
    constexpr int TPL = R8Split<G>::TPL;
    constexpr int GP = R8Split<G>::GP;
    constexpr int CL = TPL * Geo::CROW;              // c bytes per lane
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, kg = lane >> 4;
    const int pair = kg % GP, part = kg / GP;
    const int h = blockIdx.y * p.hw + wave;
    TileWalk tw;
    if (!tile_walk(p.nsh, p.n_req, p.max_pages, p.target, blockIdx.x, tw) ||
        tw.count <= 0)
        return;
    const int req = tw.req;
    const int nsh = tw.nsh;
    const int sl = p.sl[req];
    const int cnt = tw.count;
    const int t0 = tw.first;
    const int wstride = tw.stride;

    uint32_t qw[2][8];
    load_q_rows(p.q, p.q_st, p.q_hs, req, h, G, n, kg, true, qw);

    // lane n carries page lane_page(n) of a tile (mu, scales, c rows, score); clamped
    // pages load valid data and are never written
    const int own = lane_page<RP>(n);
    auto page_of = [&](int tile) { return tile * SC_TILE + own; };
    // the record offset (rec_off) of the lane's own page of a tile
    auto lane_off = [&](int tile) -> int {
        const int page = page_of(tile);
        return rec_off(p.bt[(int64_t)req * p.bt_st + (page < nsh ? page : nsh - 1)],
                       p.rec_sb);
    };
    const int rhead = h * VM + 16 * kg;
    // lr + moff: the lane's 16 bytes of the head's scale block (r8) or tail (CLSE);
    // lr + coff: its c rows
    const int tail = p.n_kv * VM + h * (Geo::TB - VM) - 16 * kg;   // the head's tail - lr
    const int moff = CLSE ? tail + 16 * Geo::CROW +
                                (kg == 0 ? 32 : (kg == 3 ? (RP == 8 ? 48 : 32) : 16 * (kg - 1)))
                          : tail + 16 * kg;
    const int coff = CLSE ? tail + part * CL : RP * Geo::CB + 128 + part * CL - 16 * kg;
    auto lane_rec = [&](int off) { return at_off(p.rec, off, rhead); };
    const int lv = h * VM + 16 * (kg * RP + n % RP);   // the lane's V bytes in a block
    __shared__ R8Lds lds;
    int2 (&row)[SC_TILE][8] = lds.x[wave][kg];

    // Three load groups per tile, each refilled right after its last use: A (column
    // groups [0, r/2), mu, scales) and B (groups [r/2, r)) are consumed by the
    // matrix-core product, C (the lane's c rows) by the token tail, so both column groups
    // of the next tile are in flight during this tile's tail.
    int tile = t0;
    int off = lane_off(tile);
    int gbk[RP];
    group_blocks<RP>(off, n, gbk);
    const int8_t* lr = lane_rec(off);
    R8GroupA<RP, VB> ga;
    R8GroupB<RP, VB> gb;
    R8GroupC<CL> gc;
    r8_load_a<RP, VB, Geo::NT>(p.rec, lv, gbk, lr, ga, moff);
    int on_next = lane_off(cnt > 1 ? tile + wstride : tile);
    __builtin_amdgcn_sched_barrier(0);
    r8_load_b<RP, VB, Geo::NT>(p.rec, lv, gbk, gb);
    __builtin_amdgcn_sched_barrier(0);
    r8_load_c<CL>(lr + coff, gc);

    i32x4_t qa[2];
    const float qs = quantize_q_rows(qw, n, qa);
    const float qs0 = __shfl(qs, 4 * kg, WAVE);        // row 4kg: limb hi of g0
    const float qs1 = __shfl(qs, 4 * kg + 2, WAVE);
    float qsq0 = 0.f, qsq1 = 0.f;                      // CLSE: |q_g0|^2, |q_g1|^2 (fp32)
    if constexpr (CLSE) {
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float lo = bf16lo(qw[t][i]), hi = bf16hi(qw[t][i]);
                ss += lo * lo + hi * hi;
            }
        ss = xor32_sumf(xor16_sumf(ss));               // the row's four 32-d quarters
        qsq0 = __shfl(ss, 4 * kg, WAVE);               // rows 4kg, 4kg+2: g0, g1
        qsq1 = __shfl(ss, 4 * kg + 2, WAVE);
    }

    R8Acc<RP> acc;
    for (int i = 0; i + 1 < cnt; ++i) {
        const int page = page_of(tile);
        const bool valid = page < nsh;
        const auto sc = r8_gather_scales<RP, TPL, CLSE>(ga.meta, n, part, p.c_fp32 != 0);
        r8_tile_start<RP, VB, G, COMB>(p, qa, ga, sc, qs0, qs1, acc, row, req, h, page, valid,
                                       pair, part, n);
        __builtin_amdgcn_sched_barrier(0);
        group_blocks<RP>(on_next, n, gbk);
        const int8_t* ln = lane_rec(on_next);
        r8_load_a<RP, VB, Geo::NT>(p.rec, lv, gbk, ln, ga, moff);
        on_next = lane_off((i + 2 < cnt) ? tile + 2 * wstride : tile + wstride);
        r8_tile_mid<RP, VB, G, COMB>(p, qa, gb, sc, qs0, qs1, acc, row, req, h, page, valid,
                                     pair, part, n);
        __builtin_amdgcn_sched_barrier(0);
        r8_load_b<RP, VB, Geo::NT>(p.rec, lv, gbk, gb);
        r8_tile_tail<RP, CBITS, G, CLSE>(p, gc, sc, acc, req, h, page, valid, pair, part, kg, sl,
                                         qsq0, qsq1);
        __builtin_amdgcn_sched_barrier(0);
        r8_load_c<CL>(ln + coff, gc);
        tile += wstride;
    }
    const int page = page_of(tile);
    const bool valid = page < nsh;
    const auto sc = r8_gather_scales<RP, TPL, CLSE>(ga.meta, n, part, p.c_fp32 != 0);
    r8_tile_start<RP, VB, G, COMB>(p, qa, ga, sc, qs0, qs1, acc, row, req, h, page, valid, pair,
                                   part, n);
    r8_tile_mid<RP, VB, G, COMB>(p, qa, gb, sc, qs0, qs1, acc, row, req, h, page, valid, pair,
                                 part, n);
    r8_tile_tail<RP, CBITS, G, CLSE>(p, gc, sc, acc, req, h, page, valid, pair, part, kg, sl,
                                     qsq0, qsq1);
}

template <int RP, int VB, int CBITS, int G, bool COMB, bool CLSE>
static int launch_r8_k(R8Params p, hipStream_t s) {
    auto k = r8_score_kernel<RP, VB, CBITS, G, COMB, CLSE>;
    int cus = 0, per_cu = 1;
    p.hw = pick_heads((const void*)k, p.n_kv, per_cu, cus);
    const int hg = p.n_kv / p.hw;
    p.target = score_target(per_cu * cus, hg);
    hipLaunchKernelGGL(k, dim3(p.target + p.n_req, hg), dim3(p.hw * WAVE), 0, s, p);
    return check_launch();
}

template <int RP, int VB, int CBITS, bool CLSE>
static int launch_r8_g(const R8Params& p, int G, bool comb, hipStream_t s) {
    switch (G) {
        case 1: return comb ? launch_r8_k<RP, VB, CBITS, 1, true, CLSE>(p, s)
                            : launch_r8_k<RP, VB, CBITS, 1, false, CLSE>(p, s);
        case 2: return comb ? launch_r8_k<RP, VB, CBITS, 2, true, CLSE>(p, s)
                            : launch_r8_k<RP, VB, CBITS, 2, false, CLSE>(p, s);
        case 4: return comb ? launch_r8_k<RP, VB, CBITS, 4, true, CLSE>(p, s)
                            : launch_r8_k<RP, VB, CBITS, 4, false, CLSE>(p, s);
        case 8: return comb ? launch_r8_k<RP, VB, CBITS, 8, true, CLSE>(p, s)
                            : launch_r8_k<RP, VB, CBITS, 8, false, CLSE>(p, s);
    }
    return AMASS_ERR_GEOMETRY;
}

}  // namespace amass
