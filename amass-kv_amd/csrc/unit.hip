// Per-unit pipeline for small batches on gfx950: quad score -> nrm combine + top-b /
// coverage selection -> (optionally) the sparse decode of each (request, kv head) unit,
// one launch.
//
// The three Stage-A/B launches of a layer (quad_score.hip, select.hip, decode.hip) each
// spread a small batch over few workgroups and each pays a launch, a chain of dependent
// memory rounds before its first useful load, and the gap to the next graph node; at
// batch 1 those fixed costs are most of the step (three launches of 6-10 us for 2.5 MB).
// Here the unit's workgroups run the same device code back to back:
//   score   wave w of the unit's workgroup j (of c) walks tiles 8 j + w, 8 (j + c) + w,
//           ... of the unit's kv head (quad_walk, the score kernel's tile loop), writing
//           score_h and the per-tile maxima;
//   select  the selection kernel's body (select_unit, fused nrm staging) reads them back
//           (after a workgroup barrier, or the ticket hand-over below) and writes score,
//           page_table, page_cnt;
//   attend  (ATTEND) the decode's whole layout (attend_whole): the 8 waves split the kept
//           pages and merge through LDS into the output.
// Global stores of one phase are read by other waves of the same workgroup in the next;
// the workgroup barrier orders them (every wave of a workgroup runs on one CU, whose
// vector L1 is write-through).  The outputs are those of the three separate launches bit
// for bit: the same instructions compute them (the decode's whole layout is what the
// separate decode picks for such batches, and what its fused path always runs).
//
// One workgroup streams a unit's summaries at only ~40 GB/s, so a long row's score phase
// is spread over several workgroups per unit: each scores every c-th group of 8 tiles,
// releases its stores device-wide (one agent-scope fence per workgroup) and takes a
// ticket; the last of the unit's workgroups acquires the others' stores and runs the
// selection and attend.  c is the caller's wgs_per_unit, or (0) the balanced plan's
// count per request, which spreads a ragged batch's long rows over more workgroups.
// The per-unit tickets are the caller's zeroed int32 array, left zero by every launch.
//
// Served: quad nrm states (score_h and tile maxima), r' = 8 int8 summaries, G <= 8, rows
// of at most 2048 pages (4 per selection thread), resident V.  The host asks for the
// attend phase only when it can bound every unit's kept pages (top-b with a small
// budget): a unit of many kept pages streams faster through the decode's split layout.
#include "attend.h"
#include "quad_tile.h"
#include "select_unit.h"

namespace amass {

constexpr int UN_THREADS = 512;                 // 8 waves: the selection's and decode's
constexpr int UN_WAVES = UN_THREADS / WAVE;
constexpr int UN_MAXP = 4 * UN_THREADS;         // pages per row: 4 per selection thread
constexpr int UN_MAXWG = 16;                    // workgroups per unit: a 2048-page row's
                                                // 128 tiles at one tile per wave

// ---- the balanced plan (wgs_per_unit 0) ----------------------------------------------
// Request r's n_kv units take c_r = max(1, ceil(T_r / tpw)) workgroups each, T_r the tiles
// of its scored pages.  First choice: tpw = max(8, ceil(n_kv sum T / target)), about one
// resident round's share of the batch's tiles per workgroup (at least a tile per wave):
// a uniform batch then takes one round, and in a ragged one the long rows' units take
// many workgroups and the short ones one each.  That may exceed a round; it is kept
// while the excess is at most a quarter round (those workgroups start where short units
// finish), since each late workgroup adds its unit's selection and attend to the step's
// tail.  Otherwise tpw is the smallest count whose total fits one round, or the longest
// row's tiles (one workgroup per unit) when none does.  Every wave computes the plan from
// n_sel_hi -- the same numbers in every workgroup, so the units' ticket counts agree --
// and workgroup x takes the x-th (request, kv head, j) in request-major order; the plan
// takes at most target + units workgroups.
struct UnitPlan {
    int r, kh, j, c;     // unit (r, kh); workgroup j of its c
};

__device__ __forceinline__ int unit_wgs(int t, int tpw) { return max(1, (t + tpw - 1) / tpw); }

// workgroups of the whole batch at tpw (every lane gets the sum); t0 = lane_tiles(0)
__device__ __forceinline__ int plan_wgs(const QuadParams& qp, int t0, int tpw) {
    const int lane = threadIdx.x & 63;
    int tot = wave_sum_uniform(lane < qp.n_req ? unit_wgs(t0, tpw) : 0);
    for (int base = WAVE; base < qp.n_req; base += WAVE)
        tot += wave_sum_uniform(base + lane < qp.n_req
                                    ? unit_wgs(lane_tiles(qp.nsh, qp.n_req, qp.max_pages, base),
                                               tpw)
                                    : 0);
    return tot * qp.n_kv;
}

__device__ __forceinline__ bool unit_plan(const QuadParams& qp, int target, int x, UnitPlan& u) {
    const int lane = threadIdx.x & 63;
    const int t0 = lane_tiles(qp.nsh, qp.n_req, qp.max_pages, 0);
    int total = wave_sum_uniform(t0), tmax = wave_max_uniform(t0);
    for (int base = WAVE; base < qp.n_req; base += WAVE) {
        const int t = lane_tiles(qp.nsh, qp.n_req, qp.max_pages, base);
        total += wave_sum_uniform(t);
        tmax = max(tmax, wave_max_uniform(t));
    }
    const int64_t unit_tiles = (int64_t)total * qp.n_kv;
    int tpw = (int)max((int64_t)UN_WAVES, (unit_tiles + target - 1) / target);
    if (plan_wgs(qp, t0, tpw) > target + target / 4) {
        int a = tpw + 1, b = max(tpw + 1, tmax);     // at tmax every unit takes one
        while (a < b) {
            const int mid = (a + b) >> 1;
            if (plan_wgs(qp, t0, mid) <= target) b = mid;
            else a = mid + 1;
        }
        tpw = a;
    }
    int before = 0;                                  // workgroups of earlier requests
    for (int base = 0; base < qp.n_req; base += WAVE) {
        const int t = base == 0 ? t0 : lane_tiles(qp.nsh, qp.n_req, qp.max_pages, base);
        const int c = base + lane < qp.n_req ? unit_wgs(t, tpw) : 0;
        const int n = c * qp.n_kv;
        const int incl = wave_incl_scan(n);
        const int in_batch = __builtin_amdgcn_readlane(incl, WAVE - 1);
        if (x < before + in_batch) {
            const unsigned long long hit = __ballot(before + incl > x);
            const int src = __ffsll((long long)hit) - 1;
            const int cs = __builtin_amdgcn_readlane(c, src);
            const int off = x - before - __builtin_amdgcn_readlane(incl - n, src);
            u.r = base + src;
            u.c = cs;
            u.kh = off / cs;
            u.j = off - u.kh * cs;
            return true;
        }
        before += in_batch;
    }
    return false;
}

// ns > 0: ns workgroups per unit, grid (n_kv * ns, n_req); ns == 0: the balanced plan,
// grid (target + units).  A unit of c > 1 workgroups hands over behind its ticket.
template <int RP, int VB, int PPT, bool ATTEND>
__global__ __launch_bounds__(UN_THREADS) void unit_kernel(const QuadParams qp,
                                                          const amass_select_args sa,
                                                          const amass_decode_args da,
                                                          int ns, int target, int32_t* tickets) {
    __shared__ QuadLds qlds;
    __shared__ XSel xs;
    __shared__ WholeLds wl;
    UnitPlan u;
    if (ns > 0) {
        u.c = ns;
        u.j = (int)blockIdx.x % ns;
        u.kh = (int)blockIdx.x / ns;
        u.r = blockIdx.y;
    } else if (!unit_plan(qp, target, blockIdx.x, u)) {
        return;                                      // past the plan's workgroups
    }
    const int kh = u.kh, r = u.r;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // ---- score: the unit's tiles over its workgroups' waves -----------------------------
    const int nsh = scored_of(qp.nsh, r, qp.max_pages);
    const int tiles = tiles_of(nsh);
    const int gw = u.j * UN_WAVES + wave, nw = u.c * UN_WAVES;
    if (gw < tiles)
        quad_walk<RP, VB, true, false>(qp, qlds, wave, kh, r, nsh, gw, (tiles - gw + nw - 1) / nw,
                                       nw);
    if (u.c > 1) {
        // the unit's last workgroup to finish scoring runs its selection (the ticket
        // returns to zero for the next launch)
        if (!last_arrival(tickets + (int64_t)r * qp.n_kv + kh, u.c)) return;
    } else {
        __syncthreads();
    }

    // ---- select (fused nrm staging over the unit's score_h and tile maxima) -------------
    const int cnt = select_unit<UN_THREADS, PPT, true>(sa, r, kh, xs);
    if constexpr (ATTEND) {
        __syncthreads();
        // ---- attend the kept pages (the decode's whole layout) --------------------------
        // as many waves as the decode's workgroup has (one per kv head, at most 8), so
        // the pages split, and the output rounds, as in amass_sparse_decode's layout
        attend_whole<0, false>(da, r, kh, da.seq_lens[r], cnt, min(da.n_kv, UN_WAVES), wl);
    }
}

// One resident round of the kernel's workgroups, taken as one per CU (8 waves of up to 168
// VGPRs and 65 KB of LDS each).
static int unit_target() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n < 1)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <int PPT>
static void launch_unit(const QuadParams& qp, const amass_select_args& sa,
                        const amass_decode_args& da, bool attend, int ns, int32_t* tickets,
                        hipStream_t s) {
    const int target = unit_target();
    const int units = sa.n_kv * sa.n_req;
    // a batch of at least a round of units gives each unit one workgroup in any plan:
    // skip the plan's prologue
    if (ns == 0 && units >= target) ns = 1;
    const dim3 grid = ns > 0 ? dim3(sa.n_kv * ns, sa.n_req) : dim3(target + units, 1);
    const dim3 blk(UN_THREADS);
    if (attend)
        hipLaunchKernelGGL((unit_kernel<8, 8, PPT, true>), grid, blk, 0, s, qp, sa, da, ns,
                           target, tickets);
    else
        hipLaunchKernelGGL((unit_kernel<8, 8, PPT, false>), grid, blk, 0, s, qp, sa, da, ns,
                           target, tickets);
}

static int unit_step(const amass_quad_score_args* q, const amass_select_args* sel,
                     const amass_decode_args* dec, int mode, int32_t* tickets, int ns,
                     hipStream_t s) {
    if (!q || !sel) return AMASS_ERR_NULL;
    if (ns < 0 || ns > UN_MAXWG) return AMASS_ERR_GEOMETRY;
    if (ns != 1 && !tickets) return AMASS_ERR_NULL;
    // score: the nrm combine's outputs are what the selection stages
    if (!q->q || !q->rec || !q->block_table || !q->n_sel_hi || !q->score_h || !q->tile_max)
        return AMASS_ERR_NULL;
    if (q->combine != 1) return AMASS_ERR_UNSUPPORTED;
    if (q->d != 128 || q->page != 16 || q->n_req < 0 || q->max_pages < 1 || q->n_kv < 1)
        return AMASS_ERR_GEOMETRY;
    if (q->G < 1 || q->G > 8) return AMASS_ERR_GEOMETRY;
    if (q->rank != 8 || q->v_bits != 8) return AMASS_ERR_UNSUPPORTED;
    if (q->max_pages > UN_MAXP) return AMASS_ERR_UNSUPPORTED;
    if ((((uintptr_t)q->rec) & 15) != 0 || (q->rec_sb & 15) != 0) return AMASS_ERR_GEOMETRY;
    if (q->rec_sb < (int64_t)q->n_kv * AMASS_QUAD_REC_BYTES(8, 8)) return AMASS_ERR_GEOMETRY;
    // select: the same unit geometry, staging from the score's buffers
    if (!sel->score || !sel->n_pages || !sel->n_sel_hi || !sel->page_table || !sel->page_cnt)
        return AMASS_ERR_NULL;
    if (mode != 0 && mode != 1) return AMASS_ERR_GEOMETRY;
    if (mode == 0 && !sel->b_fix) return AMASS_ERR_NULL;
    if (sel->n_req != q->n_req || sel->n_kv != q->n_kv || sel->G != q->G ||
        sel->max_pages != q->max_pages || sel->n_sel_hi != q->n_sel_hi)
        return AMASS_ERR_GEOMETRY;
    if (sel->score_h != q->score_h || sel->sh_sr != q->sh_sr || sel->sh_sh != q->sh_sh ||
        sel->sh_sg != q->sh_sg || sel->tile_max != q->tile_max || sel->tm_sr != q->tm_sr ||
        sel->tm_sh != q->tm_sh || sel->tm_sg != q->tm_sg)
        return AMASS_ERR_GEOMETRY;
    if (sel->sink_pages < 0 || (sel->tie_mode != 0 && sel->tie_mode != 1) ||
        (sel->score_kind != 0 && sel->score_kind != 1))
        return AMASS_ERR_GEOMETRY;
    if (mode == 1 && !(sel->coverage > 0.0 && sel->coverage <= 1.0)) return AMASS_ERR_GEOMETRY;
    // attend: resident V, the selection's page table, the same unit geometry
    if (dec) {
        if (!dec->q || !dec->k || !dec->v || !dec->block_table || !dec->seq_lens || !dec->out)
            return AMASS_ERR_NULL;
        if (dec->v_src != 0 || dec->dense) return AMASS_ERR_UNSUPPORTED;
        if (dec->d != DEC_D || dec->page != DEC_PAGE) return AMASS_ERR_GEOMETRY;
        if (dec->n_req != q->n_req || dec->n_kv != q->n_kv || dec->G != q->G ||
            dec->page_table != sel->page_table || dec->pt_sr != sel->pt_sr ||
            dec->pt_sh != sel->pt_sh || dec->page_cnt != sel->page_cnt ||
            dec->pc_sr != sel->pc_sr || dec->block_table != q->block_table ||
            dec->bt_st != q->bt_st)
            return AMASS_ERR_GEOMETRY;
        const auto off = [](const void* p, uintptr_t align) {
            return ((uintptr_t)p & (align - 1)) != 0;
        };
        if (off(dec->k, 16) || ((dec->k_sb | dec->k_st | dec->k_sh) & 7)) return AMASS_ERR_GEOMETRY;
        if (off(dec->v, 16) || ((dec->v_sb | dec->v_st | dec->v_sh) & 7)) return AMASS_ERR_GEOMETRY;
        if (off(dec->q, 8) || ((dec->q_st | dec->q_hs) & 3)) return AMASS_ERR_GEOMETRY;
        if (off(dec->out, 4) || ((dec->o_st | dec->o_hs) & 1)) return AMASS_ERR_GEOMETRY;
    }
    if (q->n_req == 0) return AMASS_OK;

    QuadParams p;
    p.q = (const uint16_t*)q->q; p.q_st = q->q_st; p.q_hs = q->q_hs;
    p.rec = q->rec; p.rec_sb = q->rec_sb;
    p.bt = q->block_table; p.bt_st = q->bt_st;
    p.nsh = q->n_sel_hi;
    p.score = q->score; p.sc_sr = q->sc_sr; p.sc_sh = q->sc_sh;
    p.score_h = q->score_h; p.sh_sr = q->sh_sr; p.sh_sh = q->sh_sh; p.sh_sg = q->sh_sg;
    p.tmax = q->tile_max; p.tm_sr = q->tm_sr; p.tm_sh = q->tm_sh; p.tm_sg = q->tm_sg;
    p.comb_out = nullptr;
    p.scale = q->scale;
    p.n_req = q->n_req; p.n_kv = q->n_kv; p.G = q->G; p.page = q->page;
    p.max_pages = q->max_pages;
    p.hw = 1;
    p.target = 1;
    amass_select_args sa = *sel;
    sa.mode = mode;
    amass_decode_args da;
    if (dec) da = *dec;
    else __builtin_memset(&da, 0, sizeof(da));
    int ppt = 1;
    while (ppt * UN_THREADS < p.max_pages) ppt *= 2;           // <= 4 (UN_MAXP)
    const bool attend = dec != nullptr;
    if ((int64_t)q->n_kv * q->n_req > 0x7FFFFFFF / UN_MAXWG) return AMASS_ERR_GEOMETRY;
    switch (ppt) {
        case 1: launch_unit<1>(p, sa, da, attend, ns, tickets, s); break;
        case 2: launch_unit<2>(p, sa, da, attend, ns, tickets, s); break;
        default: launch_unit<4>(p, sa, da, attend, ns, tickets, s); break;
    }
    return check_launch();
}

}  // namespace amass

using namespace amass;

extern "C" int amass_quad_select_attend(const amass_quad_score_args* score,
                                        const amass_select_args* select,
                                        const amass_decode_args* decode, int mode,
                                        int32_t* tickets, int wgs_per_unit, void* stream) {
    return unit_step(score, select, decode, mode, tickets, wgs_per_unit, (hipStream_t)stream);
}
