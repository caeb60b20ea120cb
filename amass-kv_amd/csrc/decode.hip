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
#include "common.h"

namespace amass {

constexpr int DEC_D = 128;
constexpr int DEC_PAGE = 16;
constexpr int SPLIT_WAVES = 4;
constexpr int FUSED_WAVES = 8;

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

// ------------------------------------------------------------------ split-K
template <int VSRC, bool DENSE>
__global__ __launch_bounds__(SPLIT_WAVES * WAVE) void decode_split_kernel(const amass_decode_args a) {
    const int lane = threadIdx.x & 63;
    const int sp = blockIdx.x * SPLIT_WAVES + (threadIdx.x >> 6);
    const int kh = blockIdx.y, r = blockIdx.z;
    if (sp >= a.split) return;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count<DENSE>(a, r, kh, sl);
    const int pps = max((cnt + a.split - 1) / a.split, a.pps_min);
    const int j0 = sp * pps;
    if (j0 >= cnt) return;
    const int j1 = min(j0 + pps, cnt);
    bf16x4_t qb[8];
    load_q(a, r, kh, lane, qb);
    WaveState st;
    init_state(st);
    attend_run<VSRC, DENSE>(a, r, kh, sl, j0, j1, 1, lane, qb, st);
    float lt = st.l + __shfl_xor(st.l, 16, WAVE);   // sum over lanes g, g+16, g+32, g+48
    lt += __shfl_xor(lt, 32, WAVE);
    const int64_t base = (((int64_t)r * a.n_kv + kh) * a.split + sp) * a.G;
    if (lane < a.G) {
        a.m_part[base + lane] = st.m;
        a.l_part[base + lane] = lt;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int g = 4 * (lane >> 4) + j;
        if (g < a.G) {
            float* dst = a.acc_part + (base + g) * DEC_D + 8 * (lane & 15);
            *reinterpret_cast<float4*>(dst) =
                make_float4(st.acc[0][j], st.acc[1][j], st.acc[2][j], st.acc[3][j]);
            *reinterpret_cast<float4*>(dst + 4) =
                make_float4(st.acc[4][j], st.acc[5][j], st.acc[6][j], st.acc[7][j]);
        }
    }
}

template <bool DENSE>
__global__ __launch_bounds__(WAVE) void merge_kernel(const amass_decode_args a) {
    const int lane = threadIdx.x;
    const int h = blockIdx.x, r = blockIdx.y;
    const int kh = h / a.G, g = h % a.G;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count<DENSE>(a, r, kh, sl);
    const int pps = max((cnt + a.split - 1) / a.split, a.pps_min);
    const int nact = cnt > 0 ? (cnt + pps - 1) / pps : 0;
    const int64_t base = ((int64_t)r * a.n_kv + kh) * a.split * a.G + g;
    float M = -INFINITY;
    for (int s2 = 0; s2 < nact; ++s2) M = fmaxf(M, a.m_part[base + (int64_t)s2 * a.G]);
    float lt = 0.f, o0 = 0.f, o1 = 0.f;
    for (int s2 = 0; s2 < nact; ++s2) {
        const int64_t idx = base + (int64_t)s2 * a.G;
        const float ls = a.l_part[idx];
        const float w = ls > 0.f ? __expf(a.m_part[idx] - M) : 0.f;
        lt += ls * w;
        const float2 v = *reinterpret_cast<const float2*>(a.acc_part + idx * DEC_D + 2 * lane);
        o0 += v.x * w;
        o1 += v.y * w;
    }
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint32_t* out = reinterpret_cast<uint32_t*>((uint16_t*)a.out + (int64_t)r * a.o_st +
                                                (int64_t)h * a.o_hs + 2 * lane);
    *out = pack_bf16x2(o0 * inv, o1 * inv);
}

// ------------------------------------------------------------------ fused
template <int VSRC, bool DENSE>
__global__ __launch_bounds__(FUSED_WAVES * WAVE) void decode_fused_kernel(const amass_decode_args a) {
    __shared__ float sm_m[FUSED_WAVES][8];
    __shared__ float sm_l[FUSED_WAVES][8];
    __shared__ float sm_acc[FUSED_WAVES][8][DEC_D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kh = blockIdx.x, r = blockIdx.y;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count<DENSE>(a, r, kh, sl);
    WaveState st;
    init_state(st);
    if (w < cnt) {
        bf16x4_t qb[8];
        load_q(a, r, kh, lane, qb);
        attend_run<VSRC, DENSE>(a, r, kh, sl, w, cnt, FUSED_WAVES, lane, qb, st);
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
    for (int idx = threadIdx.x; idx < a.G * (DEC_D / 2); idx += blockDim.x) {
        const int g = idx / (DEC_D / 2), d = 2 * (idx % (DEC_D / 2));
        float M = -INFINITY;
#pragma unroll
        for (int x = 0; x < FUSED_WAVES; ++x) M = fmaxf(M, sm_m[x][g]);
        float lsum = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int x = 0; x < FUSED_WAVES; ++x) {
            const float ls = sm_l[x][g];
            const float wt = ls > 0.f ? __expf(sm_m[x][g] - M) : 0.f;
            lsum += ls * wt;
            o0 += sm_acc[x][g][d] * wt;
            o1 += sm_acc[x][g][d + 1] * wt;
        }
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        uint32_t* out = reinterpret_cast<uint32_t*>((uint16_t*)a.out + (int64_t)r * a.o_st +
                                                    (int64_t)(kh * a.G + g) * a.o_hs + d);
        *out = pack_bf16x2(o0 * inv, o1 * inv);
    }
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
    if (a.G < 1 || a.G > 16 || a.n_kv < 1 || a.n_req < 0) return AMASS_ERR_GEOMETRY;
    if (a.G > 8 && a.path == 2) return AMASS_ERR_GEOMETRY;
    if (a.n_req == 0) return AMASS_OK;
    int path = a.path;
    if (path == 0) path = (a.n_req * a.n_kv >= 128 && a.G <= 8) ? 2 : 1;
    if (path == 1) {
        if (!a.m_part || !a.l_part || !a.acc_part) return AMASS_ERR_NULL;
        if (a.split < 1 || a.pps_min < 1) return AMASS_ERR_GEOMETRY;
        dim3 grid((a.split + SPLIT_WAVES - 1) / SPLIT_WAVES, a.n_kv, a.n_req);
        const dim3 blk(SPLIT_WAVES * WAVE);
        if (a.dense)
            hipLaunchKernelGGL((decode_split_kernel<0, true>), grid, blk, 0, s, a);
        else if (a.v_src == 1)
            hipLaunchKernelGGL((decode_split_kernel<1, false>), grid, blk, 0, s, a);
        else
            hipLaunchKernelGGL((decode_split_kernel<0, false>), grid, blk, 0, s, a);
        int rc = check_launch();
        if (rc) return rc;
        if (a.dense)
            hipLaunchKernelGGL((merge_kernel<true>), dim3(a.n_kv * a.G, a.n_req), dim3(WAVE), 0, s, a);
        else
            hipLaunchKernelGGL((merge_kernel<false>), dim3(a.n_kv * a.G, a.n_req), dim3(WAVE), 0, s, a);
        return check_launch();
    }
    if (path == 2) {
        const dim3 grid(a.n_kv, a.n_req), blk(FUSED_WAVES * WAVE);
        if (a.dense)
            hipLaunchKernelGGL((decode_fused_kernel<0, true>), grid, blk, 0, s, a);
        else if (a.v_src == 1)
            hipLaunchKernelGGL((decode_fused_kernel<1, false>), grid, blk, 0, s, a);
        else
            hipLaunchKernelGGL((decode_fused_kernel<0, false>), grid, blk, 0, s, a);
        return check_launch();
    }
    return AMASS_ERR_GEOMETRY;
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
