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
// codes], then the n_kv heads' 48-byte fp16 scale blocks (V_scale at half 0, sig2 at half
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
#include "quad_tile.h"

namespace amass {

template <int RP, int VB, bool NRM, bool COMB>
__global__ __launch_bounds__(QS_MAXW * WAVE)
void quad_score_kernel(const QuadParams p) {
    __shared__ QuadLds lds;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroup (unit u = (request, z), head group y): wave w serves head y * hw + w
    const int h = blockIdx.y * p.hw + wave;
    TileWalk tw;
    if (!tile_walk(p.nsh, p.n_req, p.max_pages, p.target, blockIdx.x, tw) ||
        tw.count <= 0)
        return;
    quad_walk<RP, VB, NRM, COMB>(p, lds, wave, h, tw.req, tw.nsh, tw.first, tw.count,
                                 tw.stride);
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
