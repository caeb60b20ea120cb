// Quad (Gaussian-MGF quadratic) page score for gfx950.
//
// Math per (request r, kv-head h, page p < n_sel_hi[r]) and GQA head g
// (reference: selection/quad_score.py:35-107, selection/quad_score_cuda.py:10-17):
//   qh_k = (V_code[:,k] * V_scale[k]) . q_g        k < r'
//   quad = s^2 / (2P) * sum_k sig2_k * qh_k^2
//   qmu  = s * (mu_code * mu_scale) . q_g
//   S_g  = qmu + quad ; score = max_g S_g ("max") or S_g -> score_h ("nrm")
//
// Design.  A wave owns 8 "units" of 8 lanes; a unit is one (page, kv-head) summary
// record and each lane holds 16 consecutive d rows of it, so a wave reads whole
// (page, 8-head) slabs of the physical-block-keyed layout with 16-byte loads (one
// contiguous 8 KB slab per page at r'=8 int8, n_kv=8).  q is quantised once per wave to
// two int8 limbs (qi = rn(q/qs), qs = max|q|/16383, hi = rn(qi/128), lo = qi-128hi;
// the reference recipe of selection/quad_score_cuda.py:902-935 with an IEEE divide) and
// every d-contraction is an exact int32 sum from v_dot4_i32_i8: the V rows are stored
// (d, r') so each lane byte-transposes its rows into d-contiguous words with v_perm_b32
// (int4 codes are fed biased, nib^8 in [0,15], and the bias is removed exactly with
// 8*sum(qi)).  The 8 lanes of a unit reduce with three DPP adds; the fp32 epilogue
// runs on lane g of the unit.  Pure VALU + VMEM: the contraction per record is G x
// (r'+1) dot products of length d, far below an MFMA tile.
#include "score_common.h"

namespace amass {

constexpr int QS_WAVES = 4;

struct QuadParams {
    const uint16_t* q; int64_t q_st, q_hs;
    const int8_t* mu; int64_t mu_sb;
    const uint16_t* mus; int64_t mus_sb;
    const int8_t* v; int64_t v_sb;
    const uint16_t* vs; int64_t vs_sb;
    const uint16_t* sg; int64_t sg_sb;
    const int32_t* bt; int64_t bt_st;
    const int32_t* nsh;
    float* score; int64_t sc_sr, sc_sh;
    float* score_h; int64_t sh_sr, sh_sh, sh_sg;
    int32_t* comb_out;
    float scale;
    int n_req, n_kv, d, page, max_pages;
    int hpt, ppt;  // heads per tile (min(n_kv,8)), pages per tile (8/hpt)
};

// One page tile's raw loads (double-buffered across the page loop).
template <int NV4>
struct QuadPage {
    uint32_t raw[4 * NV4];
    uint32_t mu[4];
    uint32_t vs[4], sg[4];
    uint32_t mus;
    int page;
    bool valid;
};

template <int RP, int NV4>
__device__ __forceinline__ void quad_load(const QuadParams& p, int req, int h, int nsh, int pg,
                                          int poff, int64_t vh_off, int64_t mh_off,
                                          QuadPage<NV4>& t) {
    int page = pg * p.ppt + poff;
    t.valid = page < nsh;
    if (!t.valid) page = nsh - 1;
    t.page = page;
    const int64_t blk = p.bt[(int64_t)req * p.bt_st + page];
    const uint4* vsrc = reinterpret_cast<const uint4*>(p.v + blk * p.v_sb + vh_off);
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        const uint4 u = vsrc[i];
        t.raw[4 * i] = u.x; t.raw[4 * i + 1] = u.y; t.raw[4 * i + 2] = u.z; t.raw[4 * i + 3] = u.w;
    }
    const uint4 m4 = *reinterpret_cast<const uint4*>(p.mu + blk * p.mu_sb + mh_off);
    t.mu[0] = m4.x; t.mu[1] = m4.y; t.mu[2] = m4.z; t.mu[3] = m4.w;
    const uint16_t* vsp = p.vs + blk * p.vs_sb + (int64_t)h * RP;
    const uint16_t* sgp = p.sg + blk * p.sg_sb + (int64_t)h * RP;
    if constexpr (RP == 8) {
        const uint4 a = *reinterpret_cast<const uint4*>(vsp);
        const uint4 b = *reinterpret_cast<const uint4*>(sgp);
        t.vs[0] = a.x; t.vs[1] = a.y; t.vs[2] = a.z; t.vs[3] = a.w;
        t.sg[0] = b.x; t.sg[1] = b.y; t.sg[2] = b.z; t.sg[3] = b.w;
    } else if constexpr (RP == 4) {
        const uint2 a = *reinterpret_cast<const uint2*>(vsp);
        const uint2 b = *reinterpret_cast<const uint2*>(sgp);
        t.vs[0] = a.x; t.vs[1] = a.y; t.sg[0] = b.x; t.sg[1] = b.y;
    } else {
        t.vs[0] = *reinterpret_cast<const uint32_t*>(vsp);
        t.sg[0] = *reinterpret_cast<const uint32_t*>(sgp);
    }
    t.mus = p.mus[blk * p.mus_sb + h];
}

__device__ __forceinline__ float half_at(const uint32_t* w, int i) {
    return fp16_to_f32((uint16_t)((w[i >> 1] >> (16 * (i & 1))) & 0xFFFF));
}

template <int RP, int VB, int G, bool NRM, int NV4>
__device__ __forceinline__ void quad_compute(const QuadParams& p, const QuadPage<NV4>& t,
                                             const uint32_t (&qh)[G][4],
                                             const uint32_t (&ql)[G][4], float qsg, int qsumg,
                                             int req, int h, int sub, int gown, float qcoef) {
    uint32_t w[RP][4];
    unpack_v<RP, VB>(t.raw, w);
    int cs[RP + 1];
#pragma unroll
    for (int k = 0; k <= RP; ++k) {
        const uint32_t* x = (k < RP) ? w[k < RP ? k : 0] : t.mu;
        int v[G];
#pragma unroll
        for (int g = 0; g < G; ++g) v[g] = dot16_2limb(qh[g], ql[g], x[0], x[1], x[2], x[3]);
        cs[k] = unit8_reduce_col<G>(v, sub);
    }
    if constexpr (VB == 4) {
#pragma unroll
        for (int k = 0; k < RP; ++k) cs[k] -= 8 * qsumg;
    }
    float quad = 0.f;
#pragma unroll
    for (int k = 0; k < RP; ++k) {
        const float qhk = (float)cs[k] * qsg * half_at(t.vs, k);
        quad += half_at(t.sg, k) * qhk * qhk;
    }
    const float musf = fp16_to_f32((uint16_t)t.mus);
    const float qmu = (float)cs[RP] * qsg * musf * p.scale;
    const float S = qmu + qcoef * quad;
    // lanes sub and sub^1 (G=4), sub^{1,2} (G=2) ... hold the same g: one writes
    constexpr int DUP = 8 / G;     // lanes per g inside the unit
    const bool writer = (sub & (DUP - 1)) == 0;
    if constexpr (NRM) {
        if (t.valid && writer)
            p.score_h[(int64_t)req * p.sh_sr + (int64_t)h * p.sh_sh + (int64_t)gown * p.sh_sg +
                      t.page] = S;
    } else {
        const float Sm = unit8_maxf(S);
        if (t.valid && sub == 0)
            p.score[(int64_t)req * p.sc_sr + (int64_t)h * p.sc_sh + t.page] = Sm;
    }
    if (p.comb_out != nullptr && t.valid && writer) {
        int32_t* co = p.comb_out +
                      (((int64_t)req * p.n_kv + h) * p.max_pages + t.page) * (G * (RP + 1)) +
                      gown * (RP + 1);
#pragma unroll
        for (int k = 0; k <= RP; ++k) co[k] = cs[k];
    }
}

template <int RP, int VB, int G, bool NRM>
__global__ __launch_bounds__(QS_WAVES * WAVE) __attribute__((amdgpu_waves_per_eu(G >= 8 ? 2 : 3)))
void quad_score_kernel(const QuadParams p) {
    constexpr int RV = RP * VB / 8;     // bytes per d row
    constexpr int NV4 = RV;             // 16-byte loads per lane (16 rows * RV / 16)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int req = blockIdx.z;
    const int hb = blockIdx.y;
    const int nsh = p.nsh[req];
    const int j = lane >> 3, sub = lane & 7;
    const int h = hb * p.hpt + (j % p.hpt);
    const int poff = j / p.hpt;
    const int npg = (nsh + p.ppt - 1) / p.ppt;
    const int wstride = gridDim.x * QS_WAVES;
    int pg = blockIdx.x * QS_WAVES + wave;
    if (pg >= npg) return;

    const int64_t vh_off = (int64_t)h * p.d * RV + (int64_t)sub * 16 * RV;
    const int64_t mh_off = (int64_t)h * p.d + 16 * sub;
    QuadPage<NV4> ta, tb;
    quad_load<RP, NV4>(p, req, h, nsh, pg, poff, vh_off, mh_off, ta);

    // ---- query limbs for this lane's kv-head group (once per wave) --------------------
    uint32_t qh[G][4], ql[G][4];
    float qsg = 0.f;
    int qsumg = 0;
    const int gown = unit_g<G>(sub);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float qs;
        int qsum;
        quantize_q16(p.q + (int64_t)req * p.q_st + (int64_t)(h * G + g) * p.q_hs + 16 * sub,
                     qh[g], ql[g], qs, qsum);
        if (g == gown) { qsg = qs; qsumg = qsum; }
    }
    const float qcoef = p.scale * p.scale / (2.0f * (float)p.page);

    // ---- page loop, two register stages: steady-state loads are unconditional so the
    // wait counts stay exact and page i+1 streams in while page i is reduced ------------
    const int n = (npg - pg + wstride - 1) / wstride;
    int i = 0;
    for (; i + 2 < n; i += 2) {
        quad_load<RP, NV4>(p, req, h, nsh, pg + (i + 1) * wstride, poff, vh_off, mh_off, tb);
        quad_compute<RP, VB, G, NRM, NV4>(p, ta, qh, ql, qsg, qsumg, req, h, sub, gown, qcoef);
        quad_load<RP, NV4>(p, req, h, nsh, pg + (i + 2) * wstride, poff, vh_off, mh_off, ta);
        quad_compute<RP, VB, G, NRM, NV4>(p, tb, qh, ql, qsg, qsumg, req, h, sub, gown, qcoef);
    }
    if (i + 1 < n) {
        quad_load<RP, NV4>(p, req, h, nsh, pg + (i + 1) * wstride, poff, vh_off, mh_off, tb);
        quad_compute<RP, VB, G, NRM, NV4>(p, ta, qh, ql, qsg, qsumg, req, h, sub, gown, qcoef);
        quad_compute<RP, VB, G, NRM, NV4>(p, tb, qh, ql, qsg, qsumg, req, h, sub, gown, qcoef);
    } else {
        quad_compute<RP, VB, G, NRM, NV4>(p, ta, qh, ql, qsg, qsumg, req, h, sub, gown, qcoef);
    }
}

// One resident round: as many workgroups as the kernel's occupancy lets every CU hold
// at once (queried once per kernel instance), split over (request, head block); each wave
// then strides over its request's page tiles.
template <typename K>
static int resident_wgs(K kernel, int threads) {
    static int cached = 0;
    if (cached == 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
            per_cu < 1)
            return 1024;
        cached = per_cu * cus;
    }
    return cached;
}

static int quad_zsplit(int resident, int n_req, int hb, int tiles) {
    const int per = n_req * hb;
    int z = (resident + per - 1) / per;
    const int zmax = (tiles + QS_WAVES * 2 - 1) / (QS_WAVES * 2);  // >= 2 tiles per wave
    z = z < zmax ? z : zmax;
    return z < 1 ? 1 : z;
}

template <int RP, int VB, int G, bool NRM>
static int launch_quad_k(const QuadParams& p, dim3 grid, int tiles, hipStream_t s) {
    auto k = quad_score_kernel<RP, VB, G, NRM>;
    grid.x = quad_zsplit(resident_wgs(k, QS_WAVES * WAVE), p.n_req, grid.y, tiles);
    hipLaunchKernelGGL(k, grid, dim3(QS_WAVES * WAVE), 0, s, p);
    return check_launch();
}

template <int RP, int VB, int G>
static int launch_quad_g(const QuadParams& p, bool nrm, dim3 grid, int tiles, hipStream_t s) {
    return nrm ? launch_quad_k<RP, VB, G, true>(p, grid, tiles, s)
               : launch_quad_k<RP, VB, G, false>(p, grid, tiles, s);
}

template <int RP, int VB>
static int launch_quad_rv(const QuadParams& p, int G, bool nrm, dim3 grid, int tiles,
                          hipStream_t s) {
    switch (G) {
        case 1: return launch_quad_g<RP, VB, 1>(p, nrm, grid, tiles, s);
        case 2: return launch_quad_g<RP, VB, 2>(p, nrm, grid, tiles, s);
        case 4: return launch_quad_g<RP, VB, 4>(p, nrm, grid, tiles, s);
        case 8: return launch_quad_g<RP, VB, 8>(p, nrm, grid, tiles, s);
        default: return AMASS_ERR_GEOMETRY;
    }
}

}  // namespace amass

using namespace amass;

extern "C" int amass_quad_score(const amass_quad_score_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->q || !a->mu || !a->mu_scale || !a->v || !a->v_scale || !a->sig2 ||
        !a->block_table || !a->n_sel_hi)
        return AMASS_ERR_NULL;
    if (a->combine == 0 && !a->score) return AMASS_ERR_NULL;
    if (a->combine == 1 && !a->score_h) return AMASS_ERR_NULL;
    if (a->combine != 0 && a->combine != 1) return AMASS_ERR_GEOMETRY;
    if (a->d != 128 || a->n_req < 0 || a->max_pages < 1) return AMASS_ERR_GEOMETRY;
    if (!(a->n_kv >= 1 && (8 % a->n_kv == 0 || a->n_kv % 8 == 0))) return AMASS_ERR_GEOMETRY;
    if (a->v_bits != 8 && a->v_bits != 4) return AMASS_ERR_GEOMETRY;
    if (a->rank != 2 && a->rank != 4 && a->rank != 8) return AMASS_ERR_UNSUPPORTED;
    if (a->n_req == 0) return AMASS_OK;
    QuadParams p;
    p.q = (const uint16_t*)a->q; p.q_st = a->q_st; p.q_hs = a->q_hs;
    p.mu = a->mu; p.mu_sb = a->mu_sb;
    p.mus = (const uint16_t*)a->mu_scale; p.mus_sb = a->mus_sb;
    p.v = a->v; p.v_sb = a->v_sb;
    p.vs = (const uint16_t*)a->v_scale; p.vs_sb = a->vs_sb;
    p.sg = (const uint16_t*)a->sig2; p.sg_sb = a->sg_sb;
    p.bt = a->block_table; p.bt_st = a->bt_st;
    p.nsh = a->n_sel_hi;
    p.score = a->score; p.sc_sr = a->sc_sr; p.sc_sh = a->sc_sh;
    p.score_h = a->score_h; p.sh_sr = a->sh_sr; p.sh_sh = a->sh_sh; p.sh_sg = a->sh_sg;
    p.comb_out = a->comb_out;
    p.scale = a->scale;
    p.n_req = a->n_req; p.n_kv = a->n_kv; p.d = a->d; p.page = a->page;
    p.max_pages = a->max_pages;
    p.hpt = a->n_kv < 8 ? a->n_kv : 8;
    p.ppt = 8 / p.hpt;
    const int hb = a->n_kv / p.hpt;
    const int tiles = (a->max_pages + p.ppt - 1) / p.ppt;
    dim3 grid(1, hb, a->n_req);
    hipStream_t s = (hipStream_t)stream;
    const bool nrm = a->combine == 1;
    if (a->v_bits == 8) {
        switch (a->rank) {
            case 2: return launch_quad_rv<2, 8>(p, a->G, nrm, grid, tiles, s);
            case 4: return launch_quad_rv<4, 8>(p, a->G, nrm, grid, tiles, s);
            case 8: return launch_quad_rv<8, 8>(p, a->G, nrm, grid, tiles, s);
        }
    } else {
        switch (a->rank) {
            case 2: return launch_quad_rv<2, 4>(p, a->G, nrm, grid, tiles, s);
            case 4: return launch_quad_rv<4, 4>(p, a->G, nrm, grid, tiles, s);
            case 8: return launch_quad_rv<8, 4>(p, a->G, nrm, grid, tiles, s);
        }
    }
    return AMASS_ERR_UNSUPPORTED;
}
