// Quad page-score tile machinery for gfx950, shared by the score kernel (quad_score.hip)
// and the per-unit pipeline kernel (unit.hip).  The design notes are at the top of
// quad_score.hip.
#pragma once
#include "score_mfma.h"

namespace amass {


constexpr int QS_MAXW = 8;      // waves (kv heads) per workgroup
constexpr int QS_TILE = SC_TILE;

struct QuadParams {
    const uint16_t* q; int64_t q_st, q_hs;
    const int8_t* rec; int64_t rec_sb;
    const int32_t* bt; int64_t bt_st;
    const int32_t* nsh;
    float* score; int64_t sc_sr, sc_sh;
    float* score_h; int64_t sh_sr, sh_sh, sh_sg;
    float* tmax; int64_t tm_sr, tm_sh, tm_sg;      // optional per-tile per-head maxima (nrm)
    int32_t* comb_out;
    float scale;
    int n_req, n_kv, G, page, max_pages;
    int hw;         // kv heads (waves) per workgroup
    int target;     // workgroups the batch's tiles are balanced over
};

template <int RP, int VB> constexpr int vm_bytes() { return RP * col_bytes<VB>() + 128; }
constexpr int QS_SCALE_BYTES = 48;   // a head's scale block: V_scale, sig2, mu_scale

template <int RP, int VB>
struct QuadGroupA {                       // groups [0, RP/2), mu, the page's scales
    static constexpr int NG = RP / 2;
    i32x4_t v[NG * loads_per_col<VB>()];
    i32x4_t mu[2];
    i32x4_t meta;                         // 16 bytes kg of the 48-byte scale block
};
template <int RP, int VB>
struct QuadGroupB {                       // groups [RP/2, RP)
    static constexpr int NG = RP - RP / 2;
    i32x4_t v[NG * loads_per_col<VB>()];
};

// Per-(page, rank) V_scale and sig2 for this lane's groups, through an LDS transpose:
// lanes (kg 0, m) / (kg 1, m) hold V_scale / sig2 of page lane_page(m) (halves 0..7 of
// their 16 scale-block bytes); T[kg][k][m] is written, and lane n reads the r' halves
// T[.][n % r'][(n / r') r' + j], j = 0..r'-1, in one load each.
struct __align__(16) QuadLds {
    uint16_t t[QS_MAXW][2][8][SC_TILE];
};

template <int RP>
struct GroupScales {
    uint32_t vs[(RP + 1) / 2], sg[(RP + 1) / 2];   // halves j
};

template <int RP>
__device__ __forceinline__ GroupScales<RP> group_scales(QuadLds& L, int wave, i32x4_t meta,
                                                        int n, int kg) {
    if (kg < 2) {
#pragma unroll
        for (int k = 0; k < RP; ++k)
            L.t[wave][kg][k][n] = (uint16_t)(((uint32_t)meta[k >> 1] >> (16 * (k & 1))) & 0xFFFFu);
    }
    GroupScales<RP> s;
    const int k = n % RP, m0 = (n / RP) * RP;
    if constexpr (RP == 8) {
        const uint4 a = *reinterpret_cast<const uint4*>(&L.t[wave][0][k][m0]);
        const uint4 b = *reinterpret_cast<const uint4*>(&L.t[wave][1][k][m0]);
        s.vs[0] = a.x; s.vs[1] = a.y; s.vs[2] = a.z; s.vs[3] = a.w;
        s.sg[0] = b.x; s.sg[1] = b.y; s.sg[2] = b.z; s.sg[3] = b.w;
    } else if constexpr (RP == 4) {
        const uint2 a = *reinterpret_cast<const uint2*>(&L.t[wave][0][k][m0]);
        const uint2 b = *reinterpret_cast<const uint2*>(&L.t[wave][1][k][m0]);
        s.vs[0] = a.x; s.vs[1] = a.y;
        s.sg[0] = b.x; s.sg[1] = b.y;
    } else {
        s.vs[0] = *reinterpret_cast<const uint32_t*>(&L.t[wave][0][k][m0]);
        s.sg[0] = *reinterpret_cast<const uint32_t*>(&L.t[wave][1][k][m0]);
    }
    return s;
}

template <int RP>
__device__ __forceinline__ float group_half(const uint32_t (&w)[(RP + 1) / 2], int j) {
    return fp16_to_f32((uint16_t)((w[j >> 1] >> (16 * (j & 1))) & 0xFFFFu));
}

// Sum over the r' lanes of each set n / r' (the ranks of one page) of q[j], leaving
// lane n with group j = n % r': a butterfly in which each stage halves the registers a
// lane keeps (the half of j its lane bit selects) and adds the partner's copy of them.
// Partners: lane ^ 7 (row half mirror), ^ 2, ^ 1 -- opposite in the stage's bit.
template <int C>
__device__ __forceinline__ void rank_stage(float* q, int n) {
    constexpr int H = C / 2;
    constexpr int CTRL = C == 8 ? DPP_HALF_MIRROR : (C == 4 ? DPP_XOR2 : DPP_XOR1);
    const bool up = (n & H) != 0;
#pragma unroll
    for (int m = 0; m < H; ++m) {
        const float keep = up ? q[m + H] : q[m];
        const float send = up ? q[m] : q[m + H];
        q[m] = keep + dpp_f<CTRL>(send);
    }
}

template <int RP>
__device__ __forceinline__ float rank_sum(float (&q)[RP], int n) {
    if constexpr (RP >= 8) rank_stage<8>(q, n);
    if constexpr (RP >= 4) rank_stage<4>(q, n);
    if constexpr (RP >= 2) rank_stage<2>(q, n);
    return q[0];
}

// comb_out row of (request, head, page, g); the row of g + 1 follows at +RP+1.
template <int RP>
__device__ __forceinline__ int32_t* comb_row(const QuadParams& p, int req, int h, int page,
                                             int g) {
    return p.comb_out + (((int64_t)req * p.n_kv + h) * p.max_pages + page) * (p.G * (RP + 1)) +
           (int64_t)g * (RP + 1);
}

// Groups [J0, J0 + NG): the r'-rank products of lane (kg, n)'s page of each group, for
// g = 2kg + e, into q[e][j] = sig2_k qh_k^2 (qh_k = comb * qs * V_scale_k).
template <int RP, int VB, int J0, int NG, bool COMB>
__device__ __forceinline__ void group_terms(const QuadParams& p, const i32x4_t (&qa)[2],
                                            const i32x4_t* v, const GroupScales<RP>& sc,
                                            float qs0, float qs1, float (&q)[2][RP], int req,
                                            int h, int tile, int nsh, int n, int kg) {
    constexpr int PP = group_pages<RP>();
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        int x[2];
        comb2<VB>(col_mfma<VB>(qa, &v[j * loads_per_col<VB>()]), x[0], x[1]);
        const float vsc = group_half<RP>(sc.vs, J0 + j), sgc = group_half<RP>(sc.sg, J0 + j);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float qhk = (float)x[e] * (e ? qs1 : qs0) * vsc;
            q[e][J0 + j] = sgc * qhk * qhk;
        }
        if constexpr (COMB) {
            const int page = tile * QS_TILE + (J0 + j) * PP + n / RP;
            if (page < nsh) {
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    if (2 * kg + e < p.G) comb_row<RP>(p, req, h, page, 2 * kg + e)[n % RP] = x[e];
            }
        }
    }
}

template <int RP, int VB, bool COMB>
__device__ __forceinline__ void tile_start(const QuadParams& p, const i32x4_t (&qa)[2],
                                           const QuadGroupA<RP, VB>& a, const GroupScales<RP>& sc,
                                           float qs0, float qs1, float (&q)[2][RP],
                                           float (&qmu)[2], int req, int h, int tile,
                                           int nsh, int n, int kg) {
    group_terms<RP, VB, 0, RP / 2, COMB>(p, qa, a.v, sc, qs0, qs1, q, req, h, tile, nsh, n, kg);
    i32x4_t m = {0, 0, 0, 0};
    m = mfma_i8(qa[0], a.mu[0], m);
    m = mfma_i8(qa[1], a.mu[1], m);
    const int cmu[2] = {m[0] * 128 + m[1], m[2] * 128 + m[3]};
    const uint32_t mus = (uint32_t)__shfl(a.meta[0], n + 32, WAVE);   // lane (2, n): half 16
    const float musf = fp16_to_f32((uint16_t)(mus & 0xFFFFu));
#pragma unroll
    for (int e = 0; e < 2; ++e) qmu[e] = (float)cmu[e] * (e ? qs1 : qs0) * musf * p.scale;
    if constexpr (COMB) {
        const int page = tile * QS_TILE + lane_page<RP>(n);
        if (page < nsh) {
#pragma unroll
            for (int e = 0; e < 2; ++e)
                if (2 * kg + e < p.G) comb_row<RP>(p, req, h, page, 2 * kg + e)[RP] = cmu[e];
        }
    }
}

template <int RP, int VB, bool NRM, bool COMB>
__device__ __forceinline__ void tile_finish(const QuadParams& p, const i32x4_t (&qa)[2],
                                            const QuadGroupB<RP, VB>& b,
                                            const GroupScales<RP>& sc, float (&q)[2][RP],
                                            const float (&qmu)[2], int req, int h, int tile,
                                            int nsh, int n, int kg, float qs0, float qs1,
                                            float qcoef) {
    group_terms<RP, VB, RP / 2, RP - RP / 2, COMB>(p, qa, b.v, sc, qs0, qs1, q, req, h, tile,
                                                   nsh, n, kg);
    const int page = tile * QS_TILE + lane_page<RP>(n);
    const bool valid = page < nsh;
    float S[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) S[e] = qmu[e] + qcoef * rank_sum<RP>(q[e], n);
    const int g0 = 2 * kg, g1 = 2 * kg + 1;
    if constexpr (NRM) {
        const int64_t row = (int64_t)req * p.sh_sr + (int64_t)h * p.sh_sh;
        if (p.G <= 4) {
            // lanes kg 2,3 take g 1,3 from lanes kg 0,1: one store per lane
            const float odd = xor32_f(S[1]);
            const int g = kg < 2 ? 2 * kg : 2 * kg - 3;
            const float v = kg < 2 ? S[0] : odd;
            if (valid && g < p.G) p.score_h[row + g * (int)p.sh_sg + page] = v;
        } else {
            const int off = g0 * (int)p.sh_sg + page;
            if (valid && g0 < p.G) p.score_h[row + off] = S[0];
            if (valid && g1 < p.G) p.score_h[row + off + (int)p.sh_sg] = S[1];
        }
        if (p.tmax) {
            // the tile's maximum of S_g0 / S_g1: the 16 lanes of row kg hold its 16 pages
            float m0 = valid ? S[0] : -INFINITY, m1 = valid ? S[1] : -INFINITY;
            m0 = row16_maxf(m0);
            m1 = row16_maxf(m1);
            if (n == 0) {
                const int64_t t = (int64_t)req * p.tm_sr + (int64_t)h * p.tm_sh + tile;
                if (g0 < p.G) p.tmax[t + g0 * p.tm_sg] = m0;
                if (g1 < p.G) p.tmax[t + g1 * p.tm_sg] = m1;
            }
        }
    } else {
        float m = g0 < p.G ? (g1 < p.G ? fmaxf(S[0], S[1]) : S[0]) : -INFINITY;
        if (p.G > 2) m = xor16_maxf(m);
        if (p.G > 4) m = xor32_maxf(m);
        if (valid && kg == 0)
            p.score[(int64_t)req * p.sc_sr + (int64_t)h * p.sc_sh + page] = m;
    }
}

// One wave scores tiles t0, t0 + wstride, ... (cnt >= 1 of them) of kv head h of request
// req (nsh scored pages), using the wave's slot `wave` of the LDS transpose.  COMB: also
// write the int32 contractions to comb_out (a test entry; the production instances have
// no extra stores in their loop, which keeps the load wait counts exact).
template <int RP, int VB, bool NRM, bool COMB>
__device__ __forceinline__ void quad_walk(const QuadParams& p, QuadLds& lds, int wave, int h,
                                          int req, int nsh, int t0, int cnt, int wstride) {
    constexpr int VM = vm_bytes<RP, VB>();
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, kg = lane >> 4;

    // ---- query limbs: lane row m = n holds limb (n & 1) of g = n >> 1 -------------------
    uint32_t qw[2][8];          // bf16 pairs, d = 64 t + 16 kg + 2 i (+1)
    load_q_rows(p.q, p.q_st, p.q_hs, req, h, p.G, n, kg, false, qw);

    // lane n's own page (mu, scales, score) is lane_page(n) of the tile; clamped pages
    // load valid data and are never written
    const int own = lane_page<RP>(n);
    // the record offset (rec_off) of the lane's own page of a tile
    auto own_off = [&](int tile) -> int {
        const int page = tile * QS_TILE + own;
        return rec_off(p.bt[(int64_t)req * p.bt_st + (page < nsh ? page : nsh - 1)],
                       p.rec_sb);
    };
    const int lv = h * VM + 16 * (kg * RP + n % RP);   // the lane's V bytes in a block
    const int rhead = h * VM + 16 * kg;
    // lr + moff: the lane's 16 bytes of the head's 48-byte scale block (lane group 3,
    // whose bytes the kernel does not use, repeats group 2's load)
    const int moff = p.n_kv * VM + h * (QS_SCALE_BYTES - VM) + (kg == 3 ? -16 : 0);
    auto lane_rec = [&](int off) { return at_off(p.rec, off, rhead); };

    int tile = t0;
    int off = own_off(tile);
    int gb[RP];
    group_blocks<RP>(off, n, gb);
    QuadGroupA<RP, VB> ga;
    QuadGroupB<RP, VB> gbuf;
    load_groups<RP, VB, 0, RP / 2>(p.rec, lv, gb, ga.v);
    ga.mu[0] = ld16(lane_rec(off) + RP * col_bytes<VB>());
    ga.mu[1] = ld16(lane_rec(off) + RP * col_bytes<VB>() + 64);
    ga.meta = ld16(lane_rec(off) + moff);
    int off_next = own_off(cnt > 1 ? tile + wstride : tile);
    __builtin_amdgcn_sched_barrier(0);
    load_groups<RP, VB, RP / 2, RP - RP / 2>(p.rec, lv, gb, gbuf.v);

    i32x4_t qa[2];
    const float qs = quantize_q_rows(qw, n, qa);
    const float qs0 = __shfl(qs, 4 * kg, WAVE);        // lane 4kg: row 4kg = g 2kg
    const float qs1 = __shfl(qs, 4 * kg + 2, WAVE);
    const float qcoef = p.scale * p.scale / (2.0f * (float)p.page);

    // ---- tile loop: group A of tile i+1 streams in while group B of tile i is used,
    // and group B of tile i+1 while group A of tile i+1 is used.  Every load in the
    // steady state is unconditional so the wait counts stay exact.  The loop runs from
    // the middle of one tile to the middle of the next (it enters with tile i's group A
    // used and group B in flight): written with the tile boundary at the back edge, the
    // compiler put group B's refill after a full drain of the memory counter at the loop
    // header (every load waited for, every tile) and kept a second copy of group A,
    // 178 VGPRs against 128 here. ------------------------------------------------------
    float q[2][RP];
    float qmu[2];
    GroupScales<RP> sc = group_scales<RP>(lds, wave, ga.meta, n, kg);
    tile_start<RP, VB, COMB>(p, qa, ga, sc, qs0, qs1, q, qmu, req, h, tile, nsh, n, kg);
    for (int i = 0; i + 1 < cnt; ++i) {
        // keep the refill of a buffer after its last use (bounds the live registers)
        __builtin_amdgcn_sched_barrier(0);
        group_blocks<RP>(off_next, n, gb);
        load_groups<RP, VB, 0, RP / 2>(p.rec, lv, gb, ga.v);
        ga.mu[0] = ld16(lane_rec(off_next) + RP * col_bytes<VB>());
        ga.mu[1] = ld16(lane_rec(off_next) + RP * col_bytes<VB>() + 64);
        ga.meta = ld16(lane_rec(off_next) + moff);
        off_next = own_off((i + 2 < cnt) ? tile + 2 * wstride : tile + wstride);
        tile_finish<RP, VB, NRM, COMB>(p, qa, gbuf, sc, q, qmu, req, h, tile, nsh, n, kg, qs0,
                                       qs1, qcoef);
        __builtin_amdgcn_sched_barrier(0);
        load_groups<RP, VB, RP / 2, RP - RP / 2>(p.rec, lv, gb, gbuf.v);
        tile += wstride;
        sc = group_scales<RP>(lds, wave, ga.meta, n, kg);
        tile_start<RP, VB, COMB>(p, qa, ga, sc, qs0, qs1, q, qmu, req, h, tile, nsh, n, kg);
    }
    tile_finish<RP, VB, NRM, COMB>(p, qa, gbuf, sc, q, qmu, req, h, tile, nsh, n, kg, qs0, qs1,
                                   qcoef);
}


}  // namespace amass
