// Per-wave sparse paged attention for gfx950, shared by the decode kernels (decode.hip)
// and the per-unit pipeline kernel (unit.hip).  The design notes are at the top of
// decode.hip.
#pragma once
#include "common.h"

namespace amass {

constexpr int DEC_D = 128;
constexpr int DEC_PAGE = 16;
constexpr int DEC_WAVES = 8;      // waves per workgroup

struct PageData {
    uint4 kq[4];          // K[t = l%16][d = 32 i2 + 8 (l/16) .. +8]
    uint4 vq[4];          // V[t = 4 (l/16) + u][d = 8 (l%16) .. +8]
};

struct WaveState {
    f32x4_t acc[8];       // O tile e: rows g = 4 (l/16) + j, column d = 8 (l%16) + e
    float m, l;           // per lane: g = lane % 16
};

template <int VSRC>
__device__ __forceinline__ const uint16_t* v_base(const amass_decode_args& a, int kh, int64_t blk,
                                                  int pt, int sl, int64_t& vst) {
    if constexpr (VSRC == 1) {
        const bool complete = (int64_t)(pt + 1) * DEC_PAGE <= (int64_t)sl;
        const int slot = a.page2slot[(int64_t)kh * a.t_nb + blk];
        const int vb = a.vbo[blk];
        if (complete && slot >= 0) {
            vst = DEC_D;
            return (const uint16_t*)a.hot + ((int64_t)kh * a.t_slots + slot) * (DEC_PAGE * DEC_D);
        }
        if (vb >= 0) {
            vst = a.v_st;
            return (const uint16_t*)a.v + (int64_t)vb * a.v_sb + (int64_t)kh * a.v_sh;
        }
        vst = DEC_D;
        return (const uint16_t*)a.pool +
               (((int64_t)a.t_layer * a.t_nb + blk) * a.n_kv + kh) * (DEC_PAGE * DEC_D);
    }
    vst = a.v_st;
    return (const uint16_t*)a.v + blk * a.v_sb + (int64_t)kh * a.v_sh;
}

// 16-byte load with the non-temporal (streaming) hint: K and V are read once per step.
__device__ __forceinline__ uint4 ld_stream(const uint16_t* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u x = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(x[0], x[1], x[2], x[3]);
}

template <int VSRC>
__device__ __forceinline__ void load_page(const amass_decode_args& a, int kh, int64_t blk, int pt,
                                          int sl, int lane, PageData& pd) {
    const uint16_t* kb = (const uint16_t*)a.k + blk * a.k_sb + (int64_t)kh * a.k_sh +
                         (int64_t)(lane & 15) * a.k_st + 8 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) pd.kq[i] = ld_stream(kb + 32 * i);
    int64_t vst;
    const uint16_t* vb = v_base<VSRC>(a, kh, blk, pt, sl, vst);
    vb += (int64_t)(4 * (lane >> 4)) * vst + 8 * (lane & 15);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        // the mem-v tier's V may sit in host memory: plain loads there
        pd.vq[u] = VSRC == 0 ? ld_stream(vb + (int64_t)u * vst)
                             : *reinterpret_cast<const uint4*>(vb + (int64_t)u * vst);
    }
}

__device__ __forceinline__ uint32_t u4at(const uint4& v, int k) {
    return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}

__device__ __forceinline__ void attend_page(const PageData& pd, const bf16x4_t (&qb)[8],
                                            int valid_t, float scale, int lane, WaveState& st) {
    // ---- S^T = K Q^T -------------------------------------------------------------------
    f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
        const uint32_t lo[2] = {pd.kq[i2].x, pd.kq[i2].y};
        const uint32_t hi[2] = {pd.kq[i2].z, pd.kq[i2].w};
        bf16x4_t k0, k1;
        __builtin_memcpy(&k0, lo, sizeof(k0));
        __builtin_memcpy(&k1, hi, sizeof(k1));
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(k0, qb[2 * i2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(k1, qb[2 * i2 + 1], c, 0, 0, 0);
    }
    const int t0 = 4 * (lane >> 4);
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[j] = c[j] * scale;
        if (t0 + j >= valid_t) s[j] = -INFINITY;
    }
    float ml = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    ml = xor32_maxf(xor16_maxf(ml));
    const float mn = fmaxf(st.m, ml);
    const float alpha = __expf(st.m - mn);
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = __expf(s[j] - mn);
    st.l = st.l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    st.m = mn;
    // rows of the O tiles this lane holds are g = 4 (l/16) + j; rescale only if a max moved
    if (__ballot(alpha != 1.0f)) {
        float ar[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ar[j] = __shfl(alpha, t0 + j, WAVE);
#pragma unroll
        for (int x = 0; x < 8; ++x)
#pragma unroll
            for (int j = 0; j < 4; ++j) st.acc[x][j] *= ar[j];
    }
    // ---- P (A operand, bf16) -------------------------------------------------------------
    bf16x4_t pa;
    {
        const uint32_t ww[2] = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
        __builtin_memcpy(&pa, ww, sizeof(pa));
    }
    // ---- V (B operands) and PV: tile e takes element e of the lane's 8 d of 4 tokens -----
    uint4 vq[4] = {pd.vq[0], pd.vq[1], pd.vq[2], pd.vq[3]};
    if (valid_t < DEC_PAGE) {
        const uint4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (t0 + u >= valid_t) vq[u] = z;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const int k = e >> 1;
        const uint32_t w[2] = {perm(u4at(vq[1], k), u4at(vq[0], k), sel),
                               perm(u4at(vq[3], k), u4at(vq[2], k), sel)};
        bf16x4_t b;
        __builtin_memcpy(&b, w, sizeof(b));
        st.acc[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, b, st.acc[e], 0, 0, 0);
    }
}

// Attend pages j = j0, j0 + step, ... < j1 of unit (r, kh) into st.  Two register
// stages: the steady-state loop issues the next page's loads unconditionally before the
// current page's math (so the wait counts stay exact and the load overlaps), and the last
// one or two pages are peeled.
template <int VSRC, bool DENSE>
__device__ void attend_run(const amass_decode_args& a, int r, int kh, int sl, int j0, int j1,
                           int step, int lane, const bf16x4_t (&qb)[8], WaveState& st) {
    const int32_t* tab = a.page_table + (int64_t)r * a.pt_sr + (int64_t)kh * a.pt_sh;
    const int32_t* bt = a.block_table + (int64_t)r * a.bt_st;
    for (int jb = j0; jb < j1; jb += 64 * step) {
        // page ids / blocks of up to 64 pages, one per lane
        const int jl = jb + lane * step;
        int ptl = 0, blkl = 0;
        if (jl < j1) {
            ptl = DENSE ? jl : tab[jl];
            blkl = bt[ptl];
        }
        const int nloc = min(64, (j1 - jb + step - 1) / step);
        auto pt_at = [&](int i) { return __builtin_amdgcn_readlane(ptl, i); };
        auto blk_at = [&](int i) { return (int64_t)__builtin_amdgcn_readlane(blkl, i); };
        auto vt_at = [&](int i) { return min(DEC_PAGE, sl - pt_at(i) * DEC_PAGE); };
        PageData pa, pb;
        load_page<VSRC>(a, kh, blk_at(0), pt_at(0), sl, lane, pa);
        int i = 0;
        for (; i + 2 < nloc; i += 2) {
            load_page<VSRC>(a, kh, blk_at(i + 1), pt_at(i + 1), sl, lane, pb);
            attend_page(pa, qb, vt_at(i), a.scale, lane, st);
            load_page<VSRC>(a, kh, blk_at(i + 2), pt_at(i + 2), sl, lane, pa);
            attend_page(pb, qb, vt_at(i + 1), a.scale, lane, st);
        }
        if (i + 1 < nloc) {
            load_page<VSRC>(a, kh, blk_at(i + 1), pt_at(i + 1), sl, lane, pb);
            attend_page(pa, qb, vt_at(i), a.scale, lane, st);
            attend_page(pb, qb, vt_at(i + 1), a.scale, lane, st);
        } else {
            attend_page(pa, qb, vt_at(i), a.scale, lane, st);
        }
    }
}

__device__ __forceinline__ void load_q(const amass_decode_args& a, int r, int kh, int lane,
                                       bf16x4_t (&qb)[8]) {
    const int g = lane & 15;
    const uint2 z = {0u, 0u};
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)r * a.q_st +
                           (int64_t)(kh * a.G + g) * a.q_hs + 8 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int off = 32 * (i >> 1) + 4 * (i & 1);
        const uint2 v = (g < a.G) ? *reinterpret_cast<const uint2*>(qrow + off) : z;
        __builtin_memcpy(&qb[i], &v, sizeof(v));
    }
}

__device__ __forceinline__ void init_state(WaveState& st) {
#pragma unroll
    for (int x = 0; x < 8; ++x) st.acc[x] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    st.m = -INFINITY;
    st.l = 0.f;
}

template <bool DENSE>
__device__ __forceinline__ int unit_count(const amass_decode_args& a, int r, int kh, int sl) {
    if (DENSE) return sl > 0 ? (sl + DEC_PAGE - 1) / DEC_PAGE : 0;
    return a.page_cnt[(int64_t)r * a.pc_sr + kh];
}

// The whole layout of one unit (request r, kv head kh, cnt pages): waves w < hw of the
// workgroup attend pages w, w + hw, ... of the unit, merge their (m, l, acc) through LDS
// and write the normalised output (no partials).  hw fixes the fp32 accumulation order,
// so callers with the same hw write the same bits.
struct WholeLds {
    float m[DEC_WAVES][8];
    float l[DEC_WAVES][8];
    float acc[DEC_WAVES][8][DEC_D];
};

template <int VSRC, bool DENSE>
__device__ __forceinline__ void attend_whole(const amass_decode_args& a, int r, int kh, int sl,
                                             int cnt, int hw, WholeLds& L) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    WaveState st;
    init_state(st);
    if (w < hw && w < cnt) {          // waves past hw (a larger workgroup) only merge
        bf16x4_t qb[8];
        load_q(a, r, kh, lane, qb);
        attend_run<VSRC, DENSE>(a, r, kh, sl, w, cnt, hw, lane, qb, st);
    }
    const float lt = xor32_sumf(xor16_sumf(st.l));
    if (lane < a.G) {
        L.m[w][lane] = st.m;
        L.l[w][lane] = lt;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int g = 4 * (lane >> 4) + j;
        if (g < a.G) {
#pragma unroll
            for (int e = 0; e < 8; ++e) L.acc[w][g][8 * (lane & 15) + e] = st.acc[e][j];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < a.G * (DEC_D / 2); idx += blockDim.x) {
        const int g = idx / (DEC_D / 2), d = 2 * (idx % (DEC_D / 2));
        float M = -INFINITY;
        for (int x = 0; x < hw; ++x) M = fmaxf(M, L.m[x][g]);
        float lsum = 0.f, o0 = 0.f, o1 = 0.f;
        for (int x = 0; x < hw; ++x) {
            const float ls = L.l[x][g];
            const float wt = ls > 0.f ? __expf(L.m[x][g] - M) : 0.f;
            lsum += ls * wt;
            o0 += L.acc[x][g][d] * wt;
            o1 += L.acc[x][g][d + 1] * wt;
        }
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        uint32_t* out = reinterpret_cast<uint32_t*>((uint16_t*)a.out + (int64_t)r * a.o_st +
                                                    (int64_t)(kh * a.G + g) * a.o_hs + d);
        *out = pack_bf16x2(o0 * inv, o1 * inv);
    }
}

}  // namespace amass
