// r8 (rank-r int8 low-rank per-key logsumexp) page score for gfx950.
//
// Math per (request r, kv-head h, page p < n_sel_hi[r]) and GQA head g (reference:
// selection/score.py:30-120; int path selection/score_cuda.py:160-448):
//   q~[g,k]  = (Vk_code[:,k] * Vk_scale[k]) . q_g                      k < r
//   tok[g,t] = s * c_scale[t] * (c_code[t,:] . q~[g,:])               t < page, 16p+t < seq_len
//   S_g      = s * (mu_code * mu_scale) . q_g + logsumexp_t tok[g,t]
//   score    = max_g S_g   (kv-union group max)
//
// Front end identical to the quad kernel (8 lanes per (page, kv-head) record, 2-limb
// int8 q, exact int32 v_dot4 sums comb = sum_d qi * code, DPP unit reduction that leaves
// every lane with all G x (r+1) sums).  Tail: lane `sub` of the unit owns tokens 2 sub and
// 2 sub + 1 (one 16-byte load of their int8 code rows), computes the G token logits, and
// the per-g logsumexp over 16 tokens is two 8-lane DPP reductions (max, then sum).
#include "score_common.h"

namespace amass {

constexpr int R8_WAVES = 4;

struct R8Params {
    const uint16_t* q; int64_t q_st, q_hs;
    const int8_t* mu; int64_t mu_sb;
    const uint16_t* mus; int64_t mus_sb;
    const int8_t* vk; int64_t vk_sb;
    const uint16_t* vks; int64_t vks_sb;
    const int8_t* c; int64_t c_sb;
    const uint16_t* cs; int64_t cs_sb;
    const int32_t* bt; int64_t bt_st;
    const int32_t* sl;
    const int32_t* nsh;
    float* score; int64_t sc_sr, sc_sh;
    int32_t* comb_out;
    float scale;
    int n_req, n_kv, d, page, max_pages;
    int hpt, ppt;
};

// sign-extended nibble i of x
__device__ __forceinline__ float nib_f(uint32_t x, int i) {
    return (float)(((int)(x << (28 - 4 * i))) >> 28);
}
__device__ __forceinline__ float byte_f(uint32_t x, int i) {
    return (float)(((int)(x << (24 - 8 * i))) >> 24);
}

template <int RP, int VB, int CB, int G>
__global__ __launch_bounds__(R8_WAVES * WAVE) void r8_score_kernel(const R8Params p) {
    constexpr int RV = RP * VB / 8;
    constexpr int NV4 = RV;
    constexpr int CROW = RP * CB / 8;   // bytes per token row of c
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int req = blockIdx.z;
    const int hb = blockIdx.y;
    const int nsh = p.nsh[req];
    const int sl = p.sl[req];
    const int j = lane >> 3, sub = lane & 7;
    const int h = hb * p.hpt + (j % p.hpt);
    const int poff = j / p.hpt;
    const int npg = (nsh + p.ppt - 1) / p.ppt;
    const int wstride = gridDim.x * R8_WAVES;
    int pg = blockIdx.x * R8_WAVES + wave;
    if (pg >= npg) return;

    uint32_t qh[G][4], ql[G][4];
    float qs[G];
    int qsum[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        quantize_q16(p.q + (int64_t)req * p.q_st + (int64_t)(h * G + g) * p.q_hs + 16 * sub,
                     qh[g], ql[g], qs[g], qsum[g]);
    const int64_t vh_off = (int64_t)h * p.d * RV + (int64_t)sub * 16 * RV;
    const int64_t mh_off = (int64_t)h * p.d + 16 * sub;

    for (; pg < npg; pg += wstride) {
        int page = pg * p.ppt + poff;
        const bool valid = page < nsh;
        if (!valid) page = nsh - 1;
        const int64_t blk = p.bt[(int64_t)req * p.bt_st + page];

        uint32_t raw[4 * NV4];
        const uint4* vsrc = reinterpret_cast<const uint4*>(p.vk + blk * p.vk_sb + vh_off);
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const uint4 u = vsrc[i];
            raw[4 * i] = u.x; raw[4 * i + 1] = u.y; raw[4 * i + 2] = u.z; raw[4 * i + 3] = u.w;
        }
        const uint4 mu4 = *reinterpret_cast<const uint4*>(p.mu + blk * p.mu_sb + mh_off);
        const uint32_t muw[4] = {mu4.x, mu4.y, mu4.z, mu4.w};
        float vsc[RP];
        load_scales<RP>(p.vks + blk * p.vks_sb + (int64_t)h * RP, vsc);
        const float musf = fp16_to_f32(p.mus[blk * p.mus_sb + h]);
        // this lane's two token rows of c (2 * CROW bytes) and their scales
        const int8_t* crow = p.c + blk * p.c_sb + (int64_t)h * p.page * CROW + 2 * sub * CROW;
        uint32_t cw[(2 * CROW + 3) / 4];
        if constexpr (2 * CROW == 16) {
            const uint4 u = *reinterpret_cast<const uint4*>(crow);
            cw[0] = u.x; cw[1] = u.y; cw[2] = u.z; cw[3] = u.w;
        } else if constexpr (2 * CROW == 8) {
            const uint2 u = *reinterpret_cast<const uint2*>(crow);
            cw[0] = u.x; cw[1] = u.y;
        } else {
            cw[0] = *reinterpret_cast<const uint32_t*>(crow);
        }
        const uint32_t csw =
            *reinterpret_cast<const uint32_t*>(p.cs + blk * p.cs_sb + (int64_t)h * p.page + 2 * sub);
        const float cs0 = fp16_to_f32((uint16_t)(csw & 0xFFFF));
        const float cs1 = fp16_to_f32((uint16_t)(csw >> 16));

        uint32_t w[RP][4];
        unpack_v<RP, VB>(raw, w);
        int comb[G][RP + 1];
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int k = 0; k <= RP; ++k) {
                int ah = 0, al = 0;
#pragma unroll
                for (int wi = 0; wi < 4; ++wi) {
                    const uint32_t x = (k < RP) ? w[k < RP ? k : 0][wi] : muw[wi];
                    ah = sdot4(qh[g][wi], x, ah);
                    al = sdot4(ql[g][wi], x, al);
                }
                int cmb = unit8_sum(ah * 128 + al);
                if (VB == 4 && k < RP) cmb -= 8 * qsum[g];
                comb[g][k] = cmb;
            }
        }
        // c codes of the two tokens as floats
        float cf[2][RP];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                if constexpr (CB == 8) {
                    const int byte = t * RP + k;
                    cf[t][k] = byte_f(cw[byte >> 2], byte & 3);
                } else {
                    const int nib = t * RP + k;      // lo nibble = even column
                    cf[t][k] = nib_f(cw[nib >> 3], nib & 7);
                }
            }
        const int tok0 = page * p.page + 2 * sub;
        const bool v0 = tok0 < sl, v1 = tok0 + 1 < sl;
        float Smax = -INFINITY;
        float Sg[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                const float qt = (float)comb[g][k] * qs[g] * vsc[k];
                a0 += cf[0][k] * qt;
                a1 += cf[1][k] * qt;
            }
            const float t0 = v0 ? a0 * p.scale * cs0 : -INFINITY;
            const float t1 = v1 ? a1 * p.scale * cs1 : -INFINITY;
            float m = unit8_maxf(fmaxf(t0, t1));
            const float mm = m == -INFINITY ? 0.f : m;
            float se = __expf(t0 - mm) + __expf(t1 - mm);
            se += dpp_f<DPP_HALF_MIRROR>(se);
            se += dpp_f<DPP_XOR2>(se);
            se += dpp_f<DPP_XOR1>(se);
            const float lse = m + __logf(se);
            const float qmu = (float)comb[g][RP] * qs[g] * musf * p.scale;
            Sg[g] = qmu + lse;
            Smax = fmaxf(Smax, Sg[g]);
        }
        if (valid && sub == 0)
            p.score[(int64_t)req * p.sc_sr + (int64_t)h * p.sc_sh + page] = Smax;
        if (p.comb_out != nullptr && valid && sub == 0) {
            int32_t* co = p.comb_out +
                          (((int64_t)req * p.n_kv + h) * p.max_pages + page) * (G * (RP + 1));
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int k = 0; k <= RP; ++k) co[g * (RP + 1) + k] = comb[g][k];
        }
    }
}

template <int RP, int VB, int CB>
static int launch_r8_b(const R8Params& p, int G, dim3 grid, hipStream_t s) {
    const dim3 blk(R8_WAVES * WAVE);
    switch (G) {
        case 1: hipLaunchKernelGGL((r8_score_kernel<RP, VB, CB, 1>), grid, blk, 0, s, p); break;
        case 2: hipLaunchKernelGGL((r8_score_kernel<RP, VB, CB, 2>), grid, blk, 0, s, p); break;
        case 4: hipLaunchKernelGGL((r8_score_kernel<RP, VB, CB, 4>), grid, blk, 0, s, p); break;
        case 8: hipLaunchKernelGGL((r8_score_kernel<RP, VB, CB, 8>), grid, blk, 0, s, p); break;
        default: return AMASS_ERR_GEOMETRY;
    }
    return check_launch();
}

}  // namespace amass

using namespace amass;

extern "C" int amass_r8_score(const amass_r8_score_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->q || !a->mu || !a->mu_scale || !a->vk || !a->vk_scale || !a->c || !a->c_scale ||
        !a->block_table || !a->seq_lens || !a->n_sel_hi || !a->score)
        return AMASS_ERR_NULL;
    if (a->d != 128 || a->page != 16 || a->n_req < 0 || a->max_pages < 1) return AMASS_ERR_GEOMETRY;
    if (!(a->n_kv >= 1 && (8 % a->n_kv == 0 || a->n_kv % 8 == 0))) return AMASS_ERR_GEOMETRY;
    if ((a->vk_bits != 8 && a->vk_bits != 4) || (a->c_bits != 8 && a->c_bits != 4))
        return AMASS_ERR_GEOMETRY;
    if (a->rank != 8 && a->rank != 4) return AMASS_ERR_UNSUPPORTED;
    if (a->n_req == 0) return AMASS_OK;
    R8Params p;
    p.q = (const uint16_t*)a->q; p.q_st = a->q_st; p.q_hs = a->q_hs;
    p.mu = a->mu; p.mu_sb = a->mu_sb;
    p.mus = (const uint16_t*)a->mu_scale; p.mus_sb = a->mus_sb;
    p.vk = a->vk; p.vk_sb = a->vk_sb;
    p.vks = (const uint16_t*)a->vk_scale; p.vks_sb = a->vks_sb;
    p.c = a->c; p.c_sb = a->c_sb;
    p.cs = (const uint16_t*)a->c_scale; p.cs_sb = a->cs_sb;
    p.bt = a->block_table; p.bt_st = a->bt_st;
    p.sl = a->seq_lens;
    p.nsh = a->n_sel_hi;
    p.score = a->score; p.sc_sr = a->sc_sr; p.sc_sh = a->sc_sh;
    p.comb_out = a->comb_out;
    p.scale = a->scale;
    p.n_req = a->n_req; p.n_kv = a->n_kv; p.d = a->d; p.page = a->page;
    p.max_pages = a->max_pages;
    p.hpt = a->n_kv < 8 ? a->n_kv : 8;
    p.ppt = 8 / p.hpt;
    const int hb = a->n_kv / p.hpt;
    const int tiles = (a->max_pages + p.ppt - 1) / p.ppt;
    const int per = a->n_req * hb;
    int z = (8192 + per * R8_WAVES - 1) / (per * R8_WAVES);
    const int zmax = (tiles + R8_WAVES * 2 - 1) / (R8_WAVES * 2);
    z = z < zmax ? z : zmax;
    z = z < 1 ? 1 : z;
    dim3 grid(z, hb, a->n_req);
    hipStream_t s = (hipStream_t)stream;
    const int key = (a->rank << 8) | (a->vk_bits << 4) | a->c_bits;
    switch (key) {
        case (8 << 8) | (8 << 4) | 8: return launch_r8_b<8, 8, 8>(p, a->G, grid, s);
        case (8 << 8) | (8 << 4) | 4: return launch_r8_b<8, 8, 4>(p, a->G, grid, s);
        case (8 << 8) | (4 << 4) | 8: return launch_r8_b<8, 4, 8>(p, a->G, grid, s);
        case (8 << 8) | (4 << 4) | 4: return launch_r8_b<8, 4, 4>(p, a->G, grid, s);
        case (4 << 8) | (8 << 4) | 8: return launch_r8_b<4, 8, 8>(p, a->G, grid, s);
        case (4 << 8) | (8 << 4) | 4: return launch_r8_b<4, 8, 4>(p, a->G, grid, s);
        case (4 << 8) | (4 << 4) | 8: return launch_r8_b<4, 4, 8>(p, a->G, grid, s);
        case (4 << 8) | (4 << 4) | 4: return launch_r8_b<4, 4, 4>(p, a->G, grid, s);
    }
    return AMASS_ERR_UNSUPPORTED;
}
