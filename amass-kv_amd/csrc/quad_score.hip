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
// Layout.  Per block, the n_kv heads' records [quad_V column-major (r' columns of CB
// bytes) | 128 mu codes], then the n_kv heads' 64-byte fp16 scale blocks (V_scale at
// half 0, sig2 at half 8, mu_scale at half 16) -- AMASS_QUAD_REC_BYTES per head.  The 16
// bytes a lane feeds to one MFMA (16 consecutive d of one column of one page) are one
// dwordx4 load, the two K-steps of a column read one whole 128-byte line, every V / mu
// record is whole 128-byte lines, and a page's scales are one more 16-byte load per lane
// spread over the tile's four lane groups and exchanged with ds_bpermute.  int4 V
// (CB = 64) has byte j = code[j] | code[j + 64] << 4: shifting the low nibble up and
// masking gives 16 * code as a signed byte for d = j (K-step 0) and d = j + 64 (K-step
// 1) with two ALU ops per word; the sums are divided by 16 exactly.
//
// Lanes.  lane = 16 kg + n: column n of the MFMA is page n of the tile, kg the 16-d
// group of each K-step (d = 64 t + 16 kg + s for slot s).  A workgroup holds one wave per
// kv head (up to 8) of one request and all its waves walk the same 16-page tiles, so a
// block's records are read by one CU together; each tile is two load groups (columns
// [0, r'/2) + mu + scales, then [r'/2, r')), double-buffered so one group streams in
// while the other is multiplied.  Result rows 4kg..4kg+3 of lane (kg, n) are limbs
// (hi, lo) of g = 2kg and 2kg+1, so the fp32 epilogue runs on every lane with 2kg < G.
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
    int32_t* comb_out;
    float scale;
    int n_req, n_kv, G, page, max_pages;
    int hw;         // kv heads (waves) per workgroup
    int target;     // workgroups the batch's tiles are balanced over
};

template <int RP, int VB> constexpr int vm_bytes() { return RP * col_bytes<VB>() + 128; }

template <int RP, int VB>
struct QuadGroupA {                       // columns [0, RP/2), mu, the page's scales
    static constexpr int NC = RP / 2;
    i32x4_t v[NC * loads_per_col<VB>()];
    i32x4_t mu[2];
    i32x4_t meta;                         // 16 bytes kg of the 64-byte scale block
};
template <int RP, int VB>
struct QuadGroupB {                       // columns [RP/2, RP)
    static constexpr int NC = RP - RP / 2;
    i32x4_t v[NC * loads_per_col<VB>()];
};

// fp16 scales of one page, gathered to every lane of the page
struct PageScales {
    uint32_t vs[4], sg[4];                // halves k of V_scale / sig2
    uint32_t mus;                         // mu_scale in the low half
};

// `lr` = the lane's record (block + head * VM + 16 kg); `moff` = its scale block - lr
template <int RP, int VB>
__device__ __forceinline__ void load_a(const int8_t* lr, QuadGroupA<RP, VB>& a, int moff) {
    constexpr int CB = col_bytes<VB>();
#pragma unroll
    for (int c = 0; c < QuadGroupA<RP, VB>::NC; ++c) {
        if constexpr (VB == 8) {
            a.v[2 * c] = ld16(lr + c * CB);
            a.v[2 * c + 1] = ld16(lr + c * CB + 64);
        } else {
            a.v[c] = ld16(lr + c * CB);
        }
    }
    a.mu[0] = ld16(lr + RP * CB);
    a.mu[1] = ld16(lr + RP * CB + 64);
    a.meta = ld16(lr + moff);
}

template <int RP, int VB>
__device__ __forceinline__ void load_b(const int8_t* lr, QuadGroupB<RP, VB>& b) {
    constexpr int CB = col_bytes<VB>();
    constexpr int C0 = RP / 2;
#pragma unroll
    for (int c = 0; c < QuadGroupB<RP, VB>::NC; ++c) {
        if constexpr (VB == 8) {
            b.v[2 * c] = ld16(lr + (C0 + c) * CB);
            b.v[2 * c + 1] = ld16(lr + (C0 + c) * CB + 64);
        } else {
            b.v[c] = ld16(lr + (C0 + c) * CB);
        }
    }
}

// lane n (kg 0) holds V_scale, lane n + 16 (kg 1) sig2, lane n + 32 (kg 2) mu_scale
template <int RP>
__device__ __forceinline__ PageScales gather_scales(i32x4_t meta, int n) {
    PageScales s;
    constexpr int NW = (RP + 1) / 2;      // dwords holding r' halves
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s.vs[i] = i < NW ? (uint32_t)__shfl(meta[i], n, WAVE) : 0u;
        s.sg[i] = i < NW ? (uint32_t)__shfl(meta[i], n + 16, WAVE) : 0u;
    }
    s.mus = (uint32_t)__shfl(meta[0], n + 32, WAVE);
    return s;
}

// Running fp32 epilogue of one tile for g = 2kg + e: the quad sum in column order and
// the mu term (the same operations, in the same order, as one pass over all columns).
struct QuadAcc {
    float quad[2];
    float qmu[2];
};

template <int NC, int VB>
__device__ __forceinline__ void cols_epilogue(const i32x4_t (&qa)[2], const i32x4_t* v,
                                              const PageScales& sc, int col0, float qs0,
                                              float qs1, QuadAcc& acc, int32_t* co, int co_g,
                                              bool co_on) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int x[2];
        comb2<VB>(col_mfma<VB>(qa, &v[c * loads_per_col<VB>()]), x[0], x[1]);
        const float vsc = half_at(sc.vs, col0 + c), sgc = half_at(sc.sg, col0 + c);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float qhk = (float)x[e] * (e ? qs1 : qs0) * vsc;
            acc.quad[e] += sgc * qhk * qhk;
        }
        if (co_on) {
            co[col0 + c] = x[0];
            co[co_g + col0 + c] = x[1];
        }
    }
}

// comb_out row of (request, head, page, g = 2kg); the row of g + 1 follows at +RP+1.
template <int RP>
__device__ __forceinline__ int32_t* comb_row(const QuadParams& p, int req, int h, int page,
                                             int kg) {
    return p.comb_out + (((int64_t)req * p.n_kv + h) * p.max_pages + page) * (p.G * (RP + 1)) +
           (int64_t)(2 * kg) * (RP + 1);
}

template <int RP, int VB, bool COMB>
__device__ __forceinline__ void tile_start(const QuadParams& p, const i32x4_t (&qa)[2],
                                           const QuadGroupA<RP, VB>& a, const PageScales& sc,
                                           float qs0, float qs1, QuadAcc& acc, int req, int h,
                                           int page, bool valid, int kg) {
    constexpr int CA = RP / 2;
    const bool co_on = COMB && valid && 2 * kg < p.G;
    const bool co1 = 2 * kg + 1 < p.G;
    int32_t* co = co_on ? comb_row<RP>(p, req, h, page, kg) : nullptr;
    acc.quad[0] = acc.quad[1] = 0.f;
    cols_epilogue<CA, VB>(qa, a.v, sc, 0, qs0, qs1, acc, co, co1 ? RP + 1 : 0, co_on);
    i32x4_t m = {0, 0, 0, 0};
    m = mfma_i8(qa[0], a.mu[0], m);
    m = mfma_i8(qa[1], a.mu[1], m);
    const int cmu[2] = {m[0] * 128 + m[1], m[2] * 128 + m[3]};
    const float musf = fp16_to_f32((uint16_t)(sc.mus & 0xFFFFu));
#pragma unroll
    for (int e = 0; e < 2; ++e) acc.qmu[e] = (float)cmu[e] * (e ? qs1 : qs0) * musf * p.scale;
    if (co_on) {
        co[RP] = cmu[0];
        if (co1) co[2 * RP + 1] = cmu[1];
    }
}

template <int RP, int VB, bool NRM, bool COMB>
__device__ __forceinline__ void tile_finish(const QuadParams& p, const i32x4_t (&qa)[2],
                                            const QuadGroupB<RP, VB>& b, const PageScales& sc,
                                            QuadAcc& acc, int req, int h, int page, bool valid,
                                            int kg, float qs0, float qs1, float qcoef) {
    constexpr int CA = RP / 2;
    const bool co_on = COMB && valid && 2 * kg < p.G;
    const bool co1 = 2 * kg + 1 < p.G;
    int32_t* co = co_on ? comb_row<RP>(p, req, h, page, kg) : nullptr;
    cols_epilogue<RP - CA, VB>(qa, b.v, sc, CA, qs0, qs1, acc, co, co1 ? RP + 1 : 0, co_on);
    float S[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) S[e] = acc.qmu[e] + qcoef * acc.quad[e];
    const int g0 = 2 * kg, g1 = 2 * kg + 1;
    if constexpr (NRM) {
        const int64_t row = (int64_t)req * p.sh_sr + (int64_t)h * p.sh_sh;
        if (p.G <= 4) {
            // lanes kg 2,3 take g 1,3 from lanes kg 0,1: one store per lane
            const float odd = __shfl_xor(S[1], 32, WAVE);
            const int g = kg < 2 ? 2 * kg : 2 * kg - 3;
            const float v = kg < 2 ? S[0] : odd;
            if (valid && g < p.G) p.score_h[row + g * (int)p.sh_sg + page] = v;
        } else {
            const int off = g0 * (int)p.sh_sg + page;
            if (valid && g0 < p.G) p.score_h[row + off] = S[0];
            if (valid && g1 < p.G) p.score_h[row + off + (int)p.sh_sg] = S[1];
        }
    } else {
        float m = g0 < p.G ? (g1 < p.G ? fmaxf(S[0], S[1]) : S[0]) : -INFINITY;
        if (p.G > 2) m = fmaxf(m, __shfl_xor(m, 16, WAVE));
        if (p.G > 4) m = fmaxf(m, __shfl_xor(m, 32, WAVE));
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
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, kg = lane >> 4;
    // workgroup (unit u = (request, z), head group y): wave w serves head y * hw + w
    const int h = blockIdx.y * p.hw + wave;
    TileWalk tw;
    if (!tile_walk(p.nsh, p.n_req, p.target, blockIdx.x, tw) || tw.count <= 0) return;
    const int req = tw.req;
    const int nsh = p.nsh[req];
    const int cnt = tw.count;
    const int t0 = tw.first;
    const int wstride = tw.stride;

    // ---- query limbs: lane row m = n holds limb (n & 1) of g = n >> 1 -------------------
    uint32_t qw[2][8];          // bf16 pairs, d = 64 t + 16 kg + 2 i (+1)
    load_q_rows(p.q, p.q_st, p.q_hs, req, h, p.G, n, kg, false, qw);

    // tile addressing: lane n owns page 16 tile + n; clamped pages load valid data and
    // are never written
    auto page_of = [&](int tile) { return tile * QS_TILE + n; };
    auto lane_blk = [&](int tile) -> int64_t {
        const int page = page_of(tile);
        const int pc = page < nsh ? page : nsh - 1;
        return (int64_t)p.bt[(int64_t)req * p.bt_st + pc];
    };
    // the loop carries block ids, not record pointers: carried pointers made the
    // compiler double the load buffers and copy them at the loop head
    const int64_t rhead = (int64_t)h * VM + 16 * kg;
    const int moff = p.n_kv * VM + h * (64 - VM);     // this head's scale block - lr
    auto lane_rec = [&](int64_t blk) { return p.rec + blk * p.rec_sb + rhead; };

    int tile = t0;
    const int8_t* lr = lane_rec(lane_blk(tile));
    QuadGroupA<RP, VB> ga;
    QuadGroupB<RP, VB> gb;
    load_a<RP, VB>(lr, ga, moff);
    int64_t bn_next = lane_blk(cnt > 1 ? tile + wstride : tile);
    // issue order A, next block id, B -- the order the loop keeps, so the loop's wait
    // counts hold on entry as well
    __builtin_amdgcn_sched_barrier(0);
    load_b<RP, VB>(lr, gb);

    i32x4_t qa[2];
    const float qs = quantize_q_rows(qw, n, qa);
    const float qs0 = __shfl(qs, 4 * kg, WAVE);        // lane 4kg: row 4kg = g 2kg
    const float qs1 = __shfl(qs, 4 * kg + 2, WAVE);
    const float qcoef = p.scale * p.scale / (2.0f * (float)p.page);

    // ---- tile loop: group A of tile i+1 streams in while group B of tile i is used,
    // and group B of tile i+1 while group A of tile i+1 is used.  Every load in the
    // steady state is unconditional so the wait counts stay exact. -----------------------
    QuadAcc acc;
    for (int i = 0; i + 1 < cnt; ++i) {
        const int page = page_of(tile);
        const bool valid = page < nsh;
        const PageScales sc = gather_scales<RP>(ga.meta, n);
        tile_start<RP, VB, COMB>(p, qa, ga, sc, qs0, qs1, acc, req, h, page, valid, kg);
        // keep the refill of a buffer after its last use (bounds the live registers)
        __builtin_amdgcn_sched_barrier(0);
        const int8_t* ln = lane_rec(bn_next);
        load_a<RP, VB>(ln, ga, moff);
        bn_next = lane_blk((i + 2 < cnt) ? tile + 2 * wstride : tile + wstride);
        tile_finish<RP, VB, NRM, COMB>(p, qa, gb, sc, acc, req, h, page, valid, kg, qs0, qs1,
                                       qcoef);
        __builtin_amdgcn_sched_barrier(0);
        load_b<RP, VB>(ln, gb);
        tile += wstride;
    }
    const int page = page_of(tile);
    const bool valid = page < nsh;
    const PageScales sc = gather_scales<RP>(ga.meta, n);
    tile_start<RP, VB, COMB>(p, qa, ga, sc, qs0, qs1, acc, req, h, page, valid, kg);
    tile_finish<RP, VB, NRM, COMB>(p, qa, gb, sc, acc, req, h, page, valid, kg, qs0, qs1, qcoef);
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
