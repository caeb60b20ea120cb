// Sparse / dense paged decode attention for gfx950 (Stage B).
//
// Reference math: attention/decode.py:128-241 (split-K online softmax over the selected
// pages) + attention/merge.py:21-50 (LSE merge); the fused single pass of
// attention/decode_cuda.py:508-775.  QK in bf16 with fp32 accumulate, scale after the
// dot, tokens >= seq_len masked to -inf, online (m, l, acc) in fp32, P in bf16 for PV.
//
// One wave attends a run of pages of one (request, kv-head) with two MFMA chains per
// 16-token page (v_mfma_f32_16x16x16_bf16):
//   S^T[t][g] = K[t][:] . Q[g][:]     A = K tile, B = Q^T (hoisted)
//   O[g][d]  += P[g][t] V[t][d]        A = P (the S^T accumulator IS the A layout:
//                                      lane l holds S[g=l%16][t=4(l/16)+j]), B = V
// so no LDS round trip is needed for P.  Every K/V load is 16 bytes: the d order of the
// QK contraction is free, so lane l (token l%16, group gl=l/16) loads K[t][32 i2 + 8 gl ..
// +8] and feeds halves h of it as MFMA k-chunk 2 i2 + h (Q is loaded with the same map);
// for PV lane l (column n=l%16) loads V[4 gl + u][8 n .. 8 n + 8] for its 4 tokens u and
// packs tile e's B operand (d = 8 n + e) with two v_perm_b32.  A page's 4 KB of K and of
// V each arrive as 4 dwordx4 loads per lane, whole 256-byte rows per instruction.  The
// GQA group fills M rows 0..G-1 of 16.  Page/block ids for up to 64 pages come from one
// vector load per wave (broadcast with readlane); the next page's loads are issued before
// the current page is computed; the accumulator rescale is skipped when no row max moved
// (alpha == 1 exactly).
//
// Workgroups.  A unit (request, kv-head) gets S workgroups of 8 waves (S = 1 when the
// units alone fill the GPU, e.g. 32 requests x 8 heads; more for few, long units); wave
// w of workgroup s attends pages s*8 + w, s*8 + w + 8S, ...  The 8 waves merge their
// online-softmax states through LDS.  With S = 1 that is the output (the fused single
// pass).  With S > 1 each workgroup writes one LSE partial (the split-K partial of
// attention/decode.py:146-241) and a second launch, one workgroup per unit, merges the
// S partials (attention/merge.py:21-50); a cross-workgroup ticket in one launch was
// measured slower, its device-scope fences write back and invalidate the XCD's L2.
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

template <int VSRC>
__device__ __forceinline__ void load_page(const amass_decode_args& a, int kh, int64_t blk, int pt,
                                          int sl, int lane, PageData& pd) {
    const uint16_t* kb = (const uint16_t*)a.k + blk * a.k_sb + (int64_t)kh * a.k_sh +
                         (int64_t)(lane & 15) * a.k_st + 8 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) pd.kq[i] = *reinterpret_cast<const uint4*>(kb + 32 * i);
    int64_t vst;
    const uint16_t* vb = v_base<VSRC>(a, kh, blk, pt, sl, vst);
    vb += (int64_t)(4 * (lane >> 4)) * vst + 8 * (lane & 15);
#pragma unroll
    for (int u = 0; u < 4; ++u) pd.vq[u] = *reinterpret_cast<const uint4*>(vb + (int64_t)u * vst);
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
    ml = fmaxf(ml, __shfl_xor(ml, 16, WAVE));
    ml = fmaxf(ml, __shfl_xor(ml, 32, WAVE));
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

// ------------------------------------------------------------------ decode
// Workgroups of a unit that carry pages: at least 8 * pps_min pages each, at most S.
__device__ __forceinline__ int unit_workgroups(int cnt, int S, int pps_min) {
    const int per = DEC_WAVES * pps_min;
    const int want = (cnt + per - 1) / per;
    return max(1, min(S, want));
}

// One workgroup = DEC_WAVES waves over the page stripe j = s*8 + w (mod 8 * S_eff) of
// unit (r = blockIdx.z, kh = blockIdx.y); the waves' online-softmax states merge through
// LDS.  S_eff = 1: normalise and write out.  S_eff > 1: write the workgroup's LSE
// partial for merge_kernel.
template <int VSRC, bool DENSE>
__global__ __launch_bounds__(DEC_WAVES * WAVE) void decode_kernel(const amass_decode_args a) {
    __shared__ float sm_m[DEC_WAVES][8];
    __shared__ float sm_l[DEC_WAVES][8];
    __shared__ float sm_acc[DEC_WAVES][8][DEC_D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int s = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count<DENSE>(a, r, kh, sl);
    const int S = unit_workgroups(cnt, a.split, a.pps_min);
    if (s >= S) return;
    WaveState st;
    init_state(st);
    const int j0 = s * DEC_WAVES + w;
    if (j0 < cnt) {
        bf16x4_t qb[8];
        load_q(a, r, kh, lane, qb);
        attend_run<VSRC, DENSE>(a, r, kh, sl, j0, cnt, DEC_WAVES * S, lane, qb, st);
    }
    float lt = st.l + __shfl_xor(st.l, 16, WAVE);   // sum over lanes g, g+16, g+32, g+48
    lt += __shfl_xor(lt, 32, WAVE);
    if (lane < a.G) {
        sm_m[w][lane] = st.m;
        sm_l[w][lane] = lt;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int g = 4 * (lane >> 4) + j;
        if (g < a.G) {
#pragma unroll
            for (int e = 0; e < 8; ++e) sm_acc[w][g][8 * (lane & 15) + e] = st.acc[e][j];
        }
    }
    __syncthreads();
    // merge the waves: (M, L, sum_w wt acc_w) per (g, d pair)
    const int64_t ubase = ((int64_t)r * a.n_kv + kh) * a.split;   // partial slots of the unit
    const int items = a.G * (DEC_D / 2);
    for (int idx = threadIdx.x; idx < items; idx += blockDim.x) {
        const int g = idx / (DEC_D / 2), d = 2 * (idx % (DEC_D / 2));
        float M = -INFINITY;
#pragma unroll
        for (int x = 0; x < DEC_WAVES; ++x) M = fmaxf(M, sm_m[x][g]);
        float lsum = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int x = 0; x < DEC_WAVES; ++x) {
            const float ls = sm_l[x][g];
            const float wt = ls > 0.f ? __expf(sm_m[x][g] - M) : 0.f;
            lsum += ls * wt;
            o0 += sm_acc[x][g][d] * wt;
            o1 += sm_acc[x][g][d + 1] * wt;
        }
        if (S == 1) {
            const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
            uint32_t* out = reinterpret_cast<uint32_t*>((uint16_t*)a.out + (int64_t)r * a.o_st +
                                                        (int64_t)(kh * a.G + g) * a.o_hs + d);
            *out = pack_bf16x2(o0 * inv, o1 * inv);
        } else {
            const int64_t pg = (ubase + s) * a.G + g;
            *reinterpret_cast<float2*>(a.acc_part + pg * DEC_D + d) = make_float2(o0, o1);
            if (d == 0) {
                a.m_part[pg] = M;
                a.l_part[pg] = lsum;
            }
        }
    }
}

// LSE merge of the split-K partials of unit (kh = blockIdx.x, r = blockIdx.y): m* = max
// m_s over the non-empty partials, w_s = exp(m_s - m*), out = sum w_s acc_s / sum w_s l_s
// (attention/merge.py:21-50).  Units the decode served with one workgroup (S_eff = 1)
// were written directly and are skipped.
__global__ __launch_bounds__(256) void merge_kernel(const amass_decode_args a) {
    const int kh = blockIdx.x, r = blockIdx.y;
    const int sl = a.seq_lens[r];
    const int cnt = a.dense ? (sl > 0 ? (sl + DEC_PAGE - 1) / DEC_PAGE : 0)
                            : a.page_cnt[(int64_t)r * a.pc_sr + kh];
    const int S = unit_workgroups(cnt, a.split, a.pps_min);
    if (S <= 1) return;
    const int64_t ubase = ((int64_t)r * a.n_kv + kh) * a.split;
    for (int idx = threadIdx.x; idx < a.G * (DEC_D / 2); idx += blockDim.x) {
        const int g = idx / (DEC_D / 2), d = 2 * (idx % (DEC_D / 2));
        float M = -INFINITY;
#pragma unroll 4
        for (int x = 0; x < S; ++x) {
            const int64_t pg = (ubase + x) * a.G + g;
            if (a.l_part[pg] > 0.f) M = fmaxf(M, a.m_part[pg]);
        }
        float lsum = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll 4
        for (int x = 0; x < S; ++x) {
            const int64_t pg = (ubase + x) * a.G + g;
            const float ls = a.l_part[pg];
            const float wt = ls > 0.f ? __expf(a.m_part[pg] - M) : 0.f;
            const float2 v = *reinterpret_cast<const float2*>(a.acc_part + pg * DEC_D + d);
            lsum += ls * wt;
            o0 += v.x * wt;
            o1 += v.y * wt;
        }
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        uint32_t* out = reinterpret_cast<uint32_t*>((uint16_t*)a.out + (int64_t)r * a.o_st +
                                                    (int64_t)(kh * a.G + g) * a.o_hs + d);
        *out = pack_bf16x2(o0 * inv, o1 * inv);
    }
}

// Workgroups of the decode kernel resident per CU (queried once per instance).
template <int VSRC, bool DENSE>
static int decode_resident(int& cus) {
    static int per_cu = 0, ncu = 0;
    if (per_cu == 0) {
        int dev = 0, p = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&p, decode_kernel<VSRC, DENSE>,
                                                         DEC_WAVES * WAVE, 0) != hipSuccess ||
            p < 1) {
            cus = 256;
            return 1;
        }
        ncu = n;
        per_cu = p;
    }
    cus = ncu;
    return per_cu;
}

template <int VSRC, bool DENSE>
static int launch_decode(amass_decode_args a, int path, hipStream_t s) {
    int S = 1;
    if (path == 1) {
        S = a.split;
    } else if (path == 0) {
        // one resident round of workgroups over the units
        int cus = 0;
        const int resident = decode_resident<VSRC, DENSE>(cus) * cus;
        const int units = a.n_req * a.n_kv;
        S = (resident + units - 1) / units;
        S = S < a.split ? S : a.split;
        S = S < 1 ? 1 : S;
    }
    if (S > 1 && (!a.m_part || !a.l_part || !a.acc_part)) return AMASS_ERR_NULL;
    a.split = S;
    hipLaunchKernelGGL((decode_kernel<VSRC, DENSE>), dim3(S, a.n_kv, a.n_req),
                       dim3(DEC_WAVES * WAVE), 0, s, a);
    int rc = check_launch();
    if (rc || S == 1) return rc;
    hipLaunchKernelGGL(merge_kernel, dim3(a.n_kv, a.n_req), dim3(256), 0, s, a);
    return check_launch();
}

static int decode_common(const amass_decode_args* ain, int force_dense, int v_src_force,
                         hipStream_t s) {
    if (!ain) return AMASS_ERR_NULL;
    amass_decode_args a = *ain;
    if (force_dense) a.dense = 1;
    if (v_src_force >= 0) a.v_src = v_src_force;
    if (!a.q || !a.k || !a.block_table || !a.seq_lens || !a.out) return AMASS_ERR_NULL;
    if (!a.dense && (!a.page_table || !a.page_cnt)) return AMASS_ERR_NULL;
    if (a.v_src == 0 && !a.v) return AMASS_ERR_NULL;
    if (a.v_src == 1 && (!a.hot || !a.page2slot || !a.vbo || !a.pool)) return AMASS_ERR_NULL;
    if (a.v_src != 0 && a.v_src != 1) return AMASS_ERR_GEOMETRY;
    if (a.dense && a.v_src == 1) return AMASS_ERR_UNSUPPORTED;
    if (a.d != DEC_D || a.page != DEC_PAGE) return AMASS_ERR_GEOMETRY;
    if (a.G < 1 || a.G > 8 || a.n_kv < 1 || a.n_req < 0) return AMASS_ERR_GEOMETRY;
    if (a.path < 0 || a.path > 2) return AMASS_ERR_GEOMETRY;
    if (a.path != 2 && (a.split < 1 || a.pps_min < 1)) return AMASS_ERR_GEOMETRY;
    if (a.path == 2) a.pps_min = a.pps_min < 1 ? 1 : a.pps_min;
    if (a.n_req == 0) return AMASS_OK;
    if (a.dense) return launch_decode<0, true>(a, a.path, s);
    if (a.v_src == 1) return launch_decode<1, false>(a, a.path, s);
    return launch_decode<0, false>(a, a.path, s);
}

}  // namespace amass

using namespace amass;

extern "C" int amass_sparse_decode(const amass_decode_args* a, void* stream) {
    return decode_common(a, 0, -1, (hipStream_t)stream);
}
extern "C" int amass_dense_paged_decode(const amass_decode_args* a, void* stream) {
    return decode_common(a, 1, -1, (hipStream_t)stream);
}
extern "C" int amass_tier_decode(const amass_decode_args* a, void* stream) {
    return decode_common(a, 0, 1, (hipStream_t)stream);
}
