// Quad (Gaussian-MGF quadratic) page score for gfx950.
//
// Math per (request r, kv-head h, page p < n_sel_hi[r]) and GQA head g
// (reference: selection/quad_score.py:7-24,35-107, selection/quad_score_cuda.py:10-17):
//   qh_k = (V_code[:,k] * V_scale[k]) . q_g        k < r'
//   quad = s^2 / (2P) * sum_k sig2_k * qh_k^2
//   qmu  = s * (mu_code * mu_scale) . q_g
//   S_g  = qmu + quad ; score = max_g S_g ("max") or S_g -> score_h ("nrm")
//
// Design.  The d-contractions of a page are a small int8 matrix product,
// [2G query limbs x d] x [d x (r'+1) columns], so they run on the matrix cores:
// v_mfma_i32_16x16x64_i8 with M = the 2G limb rows of one kv-head's queries, N = 16
// pages of a tile and K = 64 d per instruction.  q is quantised once per wave to two
// int8 limbs (qi = rn(q*inv), inv = 16383/max|q|, hi = rn(qi/128), lo = qi - 128hi;
// the recipe of selection/quad_score_cuda.py:902-935 with IEEE divides) and every
// contraction is an exact int32 sum: comb = 128 * (hi . x) + (lo . x).
//
// Layout.  Per block, the n_kv heads' records [quad_V tiled (r' CB bytes) | 128 mu
// codes], then the n_kv heads' 64-byte fp16 scale blocks (V_scale at half 0, sig2 at half
// 8, mu_scale at half 16) -- AMASS_QUAD_REC_BYTES per head.  quad_V holds 16 bytes per
// (K-step t, d group kg, column k) at ((t * 4 + kg) * r' + k) * 16 (byte i = code of
// d = 64 t + 16 kg + i); int4 (CB = 64) folds t into the nibbles (byte i of (kg, k) =
// code[16 kg + i] | code[16 kg + i + 64] << 4; shifting the low nibble up and masking
// gives 16 * code as a signed byte with two ALU ops per word, the sums divided by 16
// exactly).
//
// Lanes.  lane = 16 kg + n.  The V product's 16 columns are PP = 16 / r' pages x r'
// ranks (a tile of 16 pages is r' column groups): lane (kg, n) of group j feeds d group kg
// of rank n % r' of page j PP + n / r', so one 16-byte load per lane reads, for each of
// the group's PP pages, 64 r' contiguous bytes -- with the non-temporal hint this streams
// at ~6.6 TB/s where one column of 16 pages (64 bytes each) streams at ~5.8 (measured
// gathers of 1344-byte records).  A lane's rank terms sig2_k qh_k^2 of its r' groups are
// summed over the r' lanes of each page by a DPP butterfly (rank_sum) that leaves lane n
// with the page of group n % r' -- lane_page(n), whose mu codes, scales and score the lane
// then carries (the mu product keeps pages on the columns).  Per-(page, rank) scales
// reach the lanes through a 512-byte LDS transpose per wave.  A workgroup holds one wave
// per kv head (up to 8) of one request; all its waves walk the same 16-page tiles, and
// each tile is two load groups (column groups [0, r'/2) + mu + scales, then [r'/2, r')),
// double-buffered so one group streams in while the other is multiplied.  Result rows
// 4kg..4kg+3 of lane (kg, n) are limbs (hi, lo) of g = 2kg and 2kg+1, so the fp32
// epilogue runs on every lane with 2kg < G.
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

template <int RP, int VB>
struct QuadGroupA {                       // groups [0, RP/2), mu, the page's scales
    static constexpr int NG = RP / 2;
    i32x4_t v[NG * loads_per_col<VB>()];
    i32x4_t mu[2];
    i32x4_t meta;                         // 16 bytes kg of the 64-byte scale block
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

// COMB: also write the int32 contractions to comb_out (a test entry; the production
// instance has no extra stores in its loop, which keeps the load wait counts exact).
template <int RP, int VB, bool NRM, bool COMB>
__global__ __launch_bounds__(QS_MAXW * WAVE)
void quad_score_kernel(const QuadParams p) {
    constexpr int VM = vm_bytes<RP, VB>();
    __shared__ QuadLds lds;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, kg = lane >> 4;
    // workgroup (unit u = (request, z), head group y): wave w serves head y * hw + w
    const int h = blockIdx.y * p.hw + wave;
    TileWalk tw;
    if (!tile_walk(p.nsh, p.n_req, p.target, blockIdx.x, tw) || tw.count <= 0) return;
    const int req = tw.req;
    const int nsh = tw.nsh;
    const int cnt = tw.count;
    const int t0 = tw.first;
    const int wstride = tw.stride;

    // ---- query limbs: lane row m = n holds limb (n & 1) of g = n >> 1 -------------------
    uint32_t qw[2][8];          // bf16 pairs, d = 64 t + 16 kg + 2 i (+1)
    load_q_rows(p.q, p.q_st, p.q_hs, req, h, p.G, n, kg, false, qw);

    // lane n's own page (mu, scales, score) is lane_page(n) of the tile; clamped pages
    // load valid data and are never written
    const int own = lane_page<RP>(n);
    auto own_blk = [&](int tile) -> int {
        const int page = tile * QS_TILE + own;
        return p.bt[(int64_t)req * p.bt_st + (page < nsh ? page : nsh - 1)];
    };
    const int8_t* hrec = p.rec + (int64_t)h * VM;
    const int8_t* vbase = hrec + 16 * (kg * RP + n % RP);          // + block * rec_sb
    const int64_t rhead = (int64_t)h * VM + 16 * kg;
    const int moff = p.n_kv * VM + h * (64 - VM);     // this head's scale block - lr
    auto lane_rec = [&](int blk) { return p.rec + (int64_t)blk * p.rec_sb + rhead; };

    int tile = t0;
    int blk = own_blk(tile);
    int gb[RP];
    group_blocks<RP>(blk, n, gb);
    QuadGroupA<RP, VB> ga;
    QuadGroupB<RP, VB> gbuf;
    load_groups<RP, VB, 0, RP / 2>(vbase, p.rec_sb, gb, ga.v);
    ga.mu[0] = ld16(lane_rec(blk) + RP * col_bytes<VB>());
    ga.mu[1] = ld16(lane_rec(blk) + RP * col_bytes<VB>() + 64);
    ga.meta = ld16(lane_rec(blk) + moff);
    int blk_next = own_blk(cnt > 1 ? tile + wstride : tile);
    __builtin_amdgcn_sched_barrier(0);
    load_groups<RP, VB, RP / 2, RP - RP / 2>(vbase, p.rec_sb, gb, gbuf.v);

    i32x4_t qa[2];
    const float qs = quantize_q_rows(qw, n, qa);
    const float qs0 = __shfl(qs, 4 * kg, WAVE);        // lane 4kg: row 4kg = g 2kg
    const float qs1 = __shfl(qs, 4 * kg + 2, WAVE);
    const float qcoef = p.scale * p.scale / (2.0f * (float)p.page);

    // ---- tile loop: group A of tile i+1 streams in while group B of tile i is used,
    // and group B of tile i+1 while group A of tile i+1 is used.  Every load in the
    // steady state is unconditional so the wait counts stay exact. -----------------------
    float q[2][RP];
    float qmu[2];
    for (int i = 0; i + 1 < cnt; ++i) {
        const GroupScales<RP> sc = group_scales<RP>(lds, wave, ga.meta, n, kg);
        tile_start<RP, VB, COMB>(p, qa, ga, sc, qs0, qs1, q, qmu, req, h, tile, nsh, n, kg);
        // keep the refill of a buffer after its last use (bounds the live registers)
        __builtin_amdgcn_sched_barrier(0);
        group_blocks<RP>(blk_next, n, gb);
        load_groups<RP, VB, 0, RP / 2>(vbase, p.rec_sb, gb, ga.v);
        ga.mu[0] = ld16(lane_rec(blk_next) + RP * col_bytes<VB>());
        ga.mu[1] = ld16(lane_rec(blk_next) + RP * col_bytes<VB>() + 64);
        ga.meta = ld16(lane_rec(blk_next) + moff);
        blk_next = own_blk((i + 2 < cnt) ? tile + 2 * wstride : tile + wstride);
        tile_finish<RP, VB, NRM, COMB>(p, qa, gbuf, sc, q, qmu, req, h, tile, nsh, n, kg, qs0,
                                       qs1, qcoef);
        __builtin_amdgcn_sched_barrier(0);
        load_groups<RP, VB, RP / 2, RP - RP / 2>(vbase, p.rec_sb, gb, gbuf.v);
        tile += wstride;
    }
    const GroupScales<RP> sc = group_scales<RP>(lds, wave, ga.meta, n, kg);
    tile_start<RP, VB, COMB>(p, qa, ga, sc, qs0, qs1, q, qmu, req, h, tile, nsh, n, kg);
    tile_finish<RP, VB, NRM, COMB>(p, qa, gbuf, sc, q, qmu, req, h, tile, nsh, n, kg, qs0, qs1,
                                   qcoef);
}

template <int RP, int VB, bool NRM, bool COMB>
static int launch_quad_k(QuadParams p, hipStream_t s) {
    auto k = quad_score_kernel<RP, VB, NRM, COMB>;
    // all min(n_kv, 8) heads of a block in one workgroup: measured faster for this kernel
    // than the 4-head split even where that keeps more waves resident
    int cus = 0;
    p.hw = p.n_kv < QS_MAXW ? p.n_kv : QS_MAXW;
    const int per_cu = resident_per_cu((const void*)k, p.hw * WAVE, cus);
    const int hg = p.n_kv / p.hw;
    p.target = score_target(per_cu * cus, hg);
    hipLaunchKernelGGL(k, dim3(p.target + p.n_req, hg), dim3(p.hw * WAVE), 0, s, p);
    return check_launch();
}

template <int RP, int VB>
static int launch_quad_rv(const QuadParams& p, bool nrm, hipStream_t s) {
    if (p.comb_out != nullptr)
        return nrm ? launch_quad_k<RP, VB, true, true>(p, s)
                   : launch_quad_k<RP, VB, false, true>(p, s);
    return nrm ? launch_quad_k<RP, VB, true, false>(p, s)
               : launch_quad_k<RP, VB, false, false>(p, s);
}

}  // namespace amass

using namespace amass;

extern "C" int amass_quad_score(const amass_quad_score_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->q || !a->rec || !a->block_table || !a->n_sel_hi) return AMASS_ERR_NULL;
    if (a->combine == 0 && !a->score) return AMASS_ERR_NULL;
    if (a->combine == 1 && !a->score_h) return AMASS_ERR_NULL;
    if (a->combine != 0 && a->combine != 1) return AMASS_ERR_GEOMETRY;
    if (a->d != 128 || a->n_req < 0 || a->max_pages < 1 || a->n_kv < 1) return AMASS_ERR_GEOMETRY;
    if (a->n_kv > QS_MAXW && a->n_kv % QS_MAXW != 0) return AMASS_ERR_GEOMETRY;
    if (a->G < 1 || a->G > 8) return AMASS_ERR_GEOMETRY;
    if (a->v_bits != 8 && a->v_bits != 4) return AMASS_ERR_GEOMETRY;
    if (a->rank != 2 && a->rank != 4 && a->rank != 8) return AMASS_ERR_UNSUPPORTED;
    // 16-byte loads: the records (and so the block stride) must be 16-byte aligned
    if ((((uintptr_t)a->rec) & 15) != 0 || (a->rec_sb & 15) != 0) return AMASS_ERR_GEOMETRY;
    if (a->rec_sb < (int64_t)a->n_kv * AMASS_QUAD_REC_BYTES(a->rank, a->v_bits))
        return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    QuadParams p;
    p.q = (const uint16_t*)a->q; p.q_st = a->q_st; p.q_hs = a->q_hs;
    p.rec = a->rec; p.rec_sb = a->rec_sb;
    p.bt = a->block_table; p.bt_st = a->bt_st;
    p.nsh = a->n_sel_hi;
    p.score = a->score; p.sc_sr = a->sc_sr; p.sc_sh = a->sc_sh;
    p.score_h = a->score_h; p.sh_sr = a->sh_sr; p.sh_sh = a->sh_sh; p.sh_sg = a->sh_sg;
    p.tmax = a->combine == 1 ? a->tile_max : nullptr;
    p.tm_sr = a->tm_sr; p.tm_sh = a->tm_sh; p.tm_sg = a->tm_sg;
    p.comb_out = a->comb_out;
    p.scale = a->scale;
    p.n_req = a->n_req; p.n_kv = a->n_kv; p.G = a->G; p.page = a->page;
    p.max_pages = a->max_pages;
    p.hw = a->n_kv < QS_MAXW ? a->n_kv : QS_MAXW;
    p.target = 1;
    hipStream_t s = (hipStream_t)stream;
    const bool nrm = a->combine == 1;
    if (a->v_bits == 8) {
        switch (a->rank) {
            case 2: return launch_quad_rv<2, 8>(p, nrm, s);
            case 4: return launch_quad_rv<4, 8>(p, nrm, s);
            case 8: return launch_quad_rv<8, 8>(p, nrm, s);
        }
    } else {
        switch (a->rank) {
            case 2: return launch_quad_rv<2, 4>(p, nrm, s);
            case 4: return launch_quad_rv<4, 4>(p, nrm, s);
            case 8: return launch_quad_rv<8, 4>(p, nrm, s);
        }
    }
    return AMASS_ERR_UNSUPPORTED;
}
