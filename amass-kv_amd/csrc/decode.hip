// Sparse / dense paged decode attention for gfx950 (Stage B).
//
// Reference math: attention/decode.py:128-241 (split-K online softmax over the selected
// pages) + attention/merge.py:21-50 (LSE merge); the fused single pass of
// attention/decode_cuda.py:508-775.  QK in bf16 with fp32 accumulate, scale after the
// dot, tokens >= seq_len masked to -inf, online (m, l, acc) in fp32, P in bf16 for PV.
//
// One wave attends a run of pages of one (request, kv-head) with two MFMA chains per
// 16-token page (v_mfma_f32_16x16x16_bf16):
//   S^T[t][g] = K[t][:] . Q[g][:]     A = K tile (lane: token l%16, 4 d), B = Q^T (hoisted)
//   O[g][d]  += P[g][t] V[t][d]        A = P (the S^T accumulator IS the A layout:
//                                      lane l holds S[g=l%16][t=4(l/16)+j]), B = V
// so no LDS round trip is needed for P.  V's B operand needs 4 consecutive tokens per
// lane: each lane loads dwords (2 d) of 4 token rows and packs them with v_perm_b32; the
// d -> MFMA column map is d = 32 i + 2 n + e (tile (i, e), column n).  The GQA group fills
// M rows 0..G-1 of 16.  Page ids / block ids for up to 64 pages are fetched by one vector
// load per wave and broadcast with readlane, and the K/V loads of page j+1 are issued
// before page j is computed (two register stages).
#include "common.h"

namespace amass {

constexpr int DEC_D = 128;
constexpr int DEC_PAGE = 16;
constexpr int SPLIT_WAVES = 4;
constexpr int FUSED_WAVES = 8;

struct PageData {
    uint2 kf[8];          // K[t = l%16][d = 16 i + 4 (l/16) .. +4]
    uint32_t vr[4][4];    // V[t = 4 (l/16) + u][d = 32 i + 2 (l%16) .. +2]
};

struct WaveState {
    f32x4_t acc[8];       // O tiles (i, e) -> index 2 i + e
    float m, l;           // per lane: g = lane % 16
};

__device__ __forceinline__ const uint16_t* v_base(const amass_decode_args& a, int kh, int64_t blk,
                                                  int pt, int sl, int64_t& vst) {
    if (a.v_src == 1) {
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

__device__ __forceinline__ void load_page(const amass_decode_args& a, int kh, int64_t blk, int pt,
                                          int sl, int lane, PageData& pd) {
    const uint16_t* kb = (const uint16_t*)a.k + blk * a.k_sb + (int64_t)kh * a.k_sh +
                         (int64_t)(lane & 15) * a.k_st + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) pd.kf[i] = *reinterpret_cast<const uint2*>(kb + 16 * i);
    int64_t vst;
    const uint16_t* vb = v_base(a, kh, blk, pt, sl, vst);
    vb += (int64_t)(4 * (lane >> 4)) * vst + 2 * (lane & 15);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            pd.vr[u][i] = *reinterpret_cast<const uint32_t*>(vb + (int64_t)u * vst + 32 * i);
}

__device__ __forceinline__ void attend_page(const PageData& pd_in, const bf16x4_t (&qb)[8],
                                            int valid_t, float scale, int lane, WaveState& st) {
    // ---- S^T = K Q^T -------------------------------------------------------------------
    f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        bf16x4_t ka;
        __builtin_memcpy(&ka, &pd_in.kf[i], sizeof(ka));
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ka, qb[i], c, 0, 0, 0);
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
    // rows of the O tiles this lane holds: g = 4 (l/16) + j
    float ar[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ar[j] = __shfl(alpha, t0 + j, WAVE);
#pragma unroll
    for (int x = 0; x < 8; ++x)
#pragma unroll
        for (int j = 0; j < 4; ++j) st.acc[x][j] *= ar[j];
    // ---- P (A operand, bf16) -------------------------------------------------------------
    bf16x4_t pa;
    {
        const uint32_t w0 = pack_bf16x2(p[0], p[1]);
        const uint32_t w1 = pack_bf16x2(p[2], p[3]);
        const uint32_t ww[2] = {w0, w1};
        __builtin_memcpy(&pa, ww, sizeof(pa));
    }
    // ---- V (B operands) and PV ------------------------------------------------------------
    uint32_t vr[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) vr[u][i] = pd_in.vr[u][i];
    if (valid_t < DEC_PAGE) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (t0 + u >= valid_t)
#pragma unroll
                for (int i = 0; i < 4; ++i) vr[u][i] = 0u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t e0[2] = {perm(vr[1][i], vr[0][i], 0x05040100u),
                                perm(vr[3][i], vr[2][i], 0x05040100u)};
        const uint32_t e1[2] = {perm(vr[1][i], vr[0][i], 0x07060302u),
                                perm(vr[3][i], vr[2][i], 0x07060302u)};
        bf16x4_t b0, b1;
        __builtin_memcpy(&b0, e0, sizeof(b0));
        __builtin_memcpy(&b1, e1, sizeof(b1));
        st.acc[2 * i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, b0, st.acc[2 * i], 0, 0, 0);
        st.acc[2 * i + 1] =
            __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, b1, st.acc[2 * i + 1], 0, 0, 0);
    }
}

// Attend pages j = j0, j0 + step, ... < j1 of unit (r, kh) into st.
__device__ void attend_run(const amass_decode_args& a, int r, int kh, int sl, int j0, int j1,
                           int step, int lane, const bf16x4_t (&qb)[8], WaveState& st) {
    const int32_t* tab = a.page_table + (int64_t)r * a.pt_sr + (int64_t)kh * a.pt_sh;
    const int32_t* bt = a.block_table + (int64_t)r * a.bt_st;
    for (int jb = j0; jb < j1; jb += 64 * step) {
        // page ids / blocks of up to 64 pages, one per lane
        const int jl = jb + lane * step;
        int ptl = 0, blkl = 0;
        if (jl < j1) {
            ptl = a.dense ? jl : tab[jl];
            blkl = bt[ptl];
        }
        const int nloc = min(64, (j1 - jb + step - 1) / step);
        PageData pa, pb;
        int pt_a = __builtin_amdgcn_readlane(ptl, 0);
        load_page(a, kh, (int64_t)__builtin_amdgcn_readlane(blkl, 0), pt_a, sl, lane, pa);
        for (int i = 0; i < nloc; i += 2) {
            int pt_b = 0;
            if (i + 1 < nloc) {
                pt_b = __builtin_amdgcn_readlane(ptl, i + 1);
                load_page(a, kh, (int64_t)__builtin_amdgcn_readlane(blkl, i + 1), pt_b, sl, lane, pb);
            }
            attend_page(pa, qb, min(DEC_PAGE, sl - pt_a * DEC_PAGE), a.scale, lane, st);
            if (i + 1 >= nloc) break;
            if (i + 2 < nloc) {
                pt_a = __builtin_amdgcn_readlane(ptl, i + 2);
                load_page(a, kh, (int64_t)__builtin_amdgcn_readlane(blkl, i + 2), pt_a, sl, lane, pa);
            }
            attend_page(pb, qb, min(DEC_PAGE, sl - pt_b * DEC_PAGE), a.scale, lane, st);
        }
    }
}

__device__ __forceinline__ void load_q(const amass_decode_args& a, int r, int kh, int lane,
                                       bf16x4_t (&qb)[8]) {
    const int g = lane & 15;
    const uint2 z = {0u, 0u};
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)r * a.q_st +
                           (int64_t)(kh * a.G + g) * a.q_hs + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint2 v = (g < a.G) ? *reinterpret_cast<const uint2*>(qrow + 16 * i) : z;
        __builtin_memcpy(&qb[i], &v, sizeof(v));
    }
}

__device__ __forceinline__ void init_state(WaveState& st) {
#pragma unroll
    for (int x = 0; x < 8; ++x) st.acc[x] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    st.m = -INFINITY;
    st.l = 0.f;
}

__device__ __forceinline__ int unit_count(const amass_decode_args& a, int r, int kh, int sl) {
    if (a.dense) return sl > 0 ? (sl + DEC_PAGE - 1) / DEC_PAGE : 0;
    return a.page_cnt[(int64_t)r * a.pc_sr + kh];
}

// ------------------------------------------------------------------ split-K
__global__ __launch_bounds__(SPLIT_WAVES * WAVE) void decode_split_kernel(const amass_decode_args a) {
    const int lane = threadIdx.x & 63;
    const int sp = blockIdx.x * SPLIT_WAVES + (threadIdx.x >> 6);
    const int kh = blockIdx.y, r = blockIdx.z;
    if (sp >= a.split) return;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count(a, r, kh, sl);
    const int pps = max((cnt + a.split - 1) / a.split, a.pps_min);
    const int j0 = sp * pps;
    if (j0 >= cnt) return;
    const int j1 = min(j0 + pps, cnt);
    bf16x4_t qb[8];
    load_q(a, r, kh, lane, qb);
    WaveState st;
    init_state(st);
    attend_run(a, r, kh, sl, j0, j1, 1, lane, qb, st);
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
            float* dst = a.acc_part + (base + g) * DEC_D + 2 * (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<float2*>(dst + 32 * i) =
                    make_float2(st.acc[2 * i][j], st.acc[2 * i + 1][j]);
        }
    }
}

__global__ __launch_bounds__(WAVE) void merge_kernel(const amass_decode_args a) {
    const int lane = threadIdx.x;
    const int h = blockIdx.x, r = blockIdx.y;
    const int kh = h / a.G, g = h % a.G;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count(a, r, kh, sl);
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
__global__ __launch_bounds__(FUSED_WAVES * WAVE) void decode_fused_kernel(const amass_decode_args a) {
    __shared__ float sm_m[FUSED_WAVES][8];
    __shared__ float sm_l[FUSED_WAVES][8];
    __shared__ float sm_acc[FUSED_WAVES][8][DEC_D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kh = blockIdx.x, r = blockIdx.y;
    const int sl = a.seq_lens[r];
    const int cnt = unit_count(a, r, kh, sl);
    WaveState st;
    init_state(st);
    if (w < cnt) {
        bf16x4_t qb[8];
        load_q(a, r, kh, lane, qb);
        attend_run(a, r, kh, sl, w, cnt, FUSED_WAVES, lane, qb, st);
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
            for (int i = 0; i < 4; ++i) {
                sm_acc[w][g][32 * i + 2 * (lane & 15)] = st.acc[2 * i][j];
                sm_acc[w][g][32 * i + 2 * (lane & 15) + 1] = st.acc[2 * i + 1][j];
            }
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
        hipLaunchKernelGGL(decode_split_kernel, grid, dim3(SPLIT_WAVES * WAVE), 0, s, a);
        int rc = check_launch();
        if (rc) return rc;
        hipLaunchKernelGGL(merge_kernel, dim3(a.n_kv * a.G, a.n_req), dim3(WAVE), 0, s, a);
        return check_launch();
    }
    if (path == 2) {
        hipLaunchKernelGGL(decode_fused_kernel, dim3(a.n_kv, a.n_req), dim3(FUSED_WAVES * WAVE),
                           0, s, a);
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
