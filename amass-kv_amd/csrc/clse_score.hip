// CLSE page score entry point for gfx950 (kernel in score_lse.h, CLSE mode).
#include "score_lse.h"

using namespace amass;

extern "C" int amass_clse_score(const amass_clse_score_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->q || !a->rec || !a->block_table || !a->seq_lens || !a->n_sel_hi)
        return AMASS_ERR_NULL;
    if (a->combine != 0 && a->combine != 1) return AMASS_ERR_GEOMETRY;
    if ((a->combine == 0 && !a->score) || (a->combine == 1 && !a->score_h))
        return AMASS_ERR_NULL;
    if (a->d != 128 || a->page != 16 || a->n_req < 0 || a->max_pages < 1 || a->n_kv < 1)
        return AMASS_ERR_GEOMETRY;
    if (a->n_kv > R8_MAXW && a->n_kv % R8_MAXW != 0) return AMASS_ERR_GEOMETRY;
    if (a->G != 1 && a->G != 2 && a->G != 4 && a->G != 8) return AMASS_ERR_GEOMETRY;
    if ((a->v_bits != 8 && a->v_bits != 4) || (a->c_bits != 8 && a->c_bits != 4))
        return AMASS_ERR_GEOMETRY;
    if (a->rank != 2 && a->rank != 4 && a->rank != 8) return AMASS_ERR_UNSUPPORTED;
    if ((((uintptr_t)a->rec) & 15) != 0 || (a->rec_sb & 15) != 0) return AMASS_ERR_GEOMETRY;
    if (a->rec_sb < (int64_t)a->n_kv * AMASS_CLSE_REC_BYTES(a->rank, a->v_bits, a->c_bits))
        return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    R8Params p;
    p.q = (const uint16_t*)a->q; p.q_st = a->q_st; p.q_hs = a->q_hs;
    p.rec = a->rec; p.rec_sb = a->rec_sb;
    p.bt = a->block_table; p.bt_st = a->bt_st;
    p.sl = a->seq_lens;
    p.nsh = a->n_sel_hi;
    p.score = a->score; p.sc_sr = a->sc_sr; p.sc_sh = a->sc_sh;
    p.score_h = a->score_h; p.sh_sr = a->sh_sr; p.sh_sh = a->sh_sh; p.sh_sg = a->sh_sg;
    p.tmax = a->combine == 1 ? a->tile_max : nullptr;
    p.tm_sr = a->tm_sr; p.tm_sh = a->tm_sh; p.tm_sg = a->tm_sg;
    p.c_fp32 = 0;
    p.comb_out = a->comb_out;
    p.scale = a->scale;
    const int dr = a->d - a->rank > 1 ? a->d - a->rank : 1;
    p.iso_coef = a->scale * a->scale / (2.0f * (float)a->page * (float)dr);
    p.scale_l2 = p.scale * 1.44269504088896341f;
    p.iso_k = p.iso_coef / (p.scale_l2 * p.scale_l2);
    p.combine = a->combine;
    p.n_req = a->n_req; p.n_kv = a->n_kv; p.page = a->page; p.max_pages = a->max_pages;
    p.hw = a->n_kv < R8_MAXW ? a->n_kv : R8_MAXW;
    p.target = 1;
    hipStream_t s = (hipStream_t)stream;
    const bool comb = a->comb_out != nullptr;
    const int key = (a->rank << 8) | (a->v_bits << 4) | a->c_bits;
    switch (key) {
        case (8 << 8) | (8 << 4) | 8: return launch_r8_g<8, 8, 8, true>(p, a->G, comb, s);
        case (8 << 8) | (8 << 4) | 4: return launch_r8_g<8, 8, 4, true>(p, a->G, comb, s);
        case (8 << 8) | (4 << 4) | 8: return launch_r8_g<8, 4, 8, true>(p, a->G, comb, s);
        case (8 << 8) | (4 << 4) | 4: return launch_r8_g<8, 4, 4, true>(p, a->G, comb, s);
        case (4 << 8) | (8 << 4) | 8: return launch_r8_g<4, 8, 8, true>(p, a->G, comb, s);
        case (4 << 8) | (8 << 4) | 4: return launch_r8_g<4, 8, 4, true>(p, a->G, comb, s);
        case (4 << 8) | (4 << 4) | 8: return launch_r8_g<4, 4, 8, true>(p, a->G, comb, s);
        case (4 << 8) | (4 << 4) | 4: return launch_r8_g<4, 4, 4, true>(p, a->G, comb, s);
        case (2 << 8) | (8 << 4) | 8: return launch_r8_g<2, 8, 8, true>(p, a->G, comb, s);
        case (2 << 8) | (8 << 4) | 4: return launch_r8_g<2, 8, 4, true>(p, a->G, comb, s);
        case (2 << 8) | (4 << 4) | 8: return launch_r8_g<2, 4, 8, true>(p, a->G, comb, s);
        case (2 << 8) | (4 << 4) | 4: return launch_r8_g<2, 4, 4, true>(p, a->G, comb, s);
    }
    return AMASS_ERR_UNSUPPORTED;
}
