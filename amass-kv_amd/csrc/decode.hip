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
// Workgroups.  A workgroup is (request, split s) and holds one wave per kv head (up to
// 8): wave h attends pages s, s + S, s + 2S, ... of head h's selection.  The waves of a
// workgroup therefore read the slices of different heads (often of the same blocks)
// together, which is the access mix that lets the non-temporal K/V loads stream at
// ~7 TB/s; eight waves of ONE head at the same offset of eight blocks measured 6.0 TB/s
// with or without the hint.  A head served by one split (S_eff = 1) normalises and
// writes its output (the fused single pass); otherwise every split writes an LSE
// partial (the split-K partial of attention/decode.py:146-241) and a second launch, one
// workgroup per unit, merges them (attention/merge.py:21-50); a cross-workgroup ticket
// in one launch was measured slower, its device-scope fences write back and invalidate
// the XCD's L2.
#include <mutex>

#include "attend.h"

namespace amass {

// ------------------------------------------------------------------ split plan
// A workgroup serves one head group (hw = min(n_kv, 8) kv heads) of one request, in one of
// two layouts chosen per launch.  Request r's work W_r is the most pages any head of the
// group attends.
//   whole (one head per workgroup): the group's nh heads get a workgroup each, whose
//     waves split the head's pages and merge through LDS into the output (no partials).
//     Path 2 (the fused single pass), and path 0 when the batch is latency-bound (on
//     average <= DEC_WHOLE_PPS pages per resident workgroup) and its longest unit over
//     the workgroup's waves takes at most two page steps more than a split would: the
//     merge launch it saves costs more than the streaming it loses.
//   split (one wave per head): S_r = min(smax, max(1, ceil(W_r / tpw))) workgroups, split
//     s taking pages s, s + S_r, ... of every head; S_r > 1 writes LSE partials.  The
//     waves of a workgroup read the slices of different heads of (often) the same blocks,
//     which keeps the non-temporal loads streaming.
// Balanced plan (path 0, split): tpw is the smallest value >= max(pps_min, ceil(sum W /
// target)) whose split total fits `target` resident workgroups (a binary search, skipped
// when the first value fits); path 1: tpw = pps_min, smax = S.  Workgroup x walks the
// requests' workgroup counts in order.  Every wave computes the plan on the device (no
// host knowledge of the lengths, so the launch stays capturable).
constexpr int DEC_WHOLE_PPS = 16;

struct SplitPlan {
    int req, s, S;
};

__device__ __forceinline__ int req_work(const amass_decode_args& a, int r, int kh0, int hw) {
    if (a.dense) {
        const int sl = a.seq_lens[r];
        return sl > 0 ? (sl + DEC_PAGE - 1) / DEC_PAGE : 0;
    }
    const int32_t* pc = a.page_cnt + (int64_t)r * a.pc_sr + kh0;
    const int n = min(hw, a.n_kv - kh0);
    int c[DEC_WAVES];
#pragma unroll
    for (int h = 0; h < DEC_WAVES; ++h) c[h] = h < n ? pc[h] : 0;   // all loads issued first
    int m = 0;
#pragma unroll
    for (int h = 0; h < DEC_WAVES; ++h) m = max(m, c[h]);
    return m;
}

__device__ __forceinline__ int req_splits(int W, int tpw, int smax) {
    return W <= 0 ? 1 : min(smax, (W + tpw - 1) / tpw);
}
// workgroups of a request
__device__ __forceinline__ int req_units(int W, bool whole, int tpw, int smax, int nh) {
    return whole ? nh : req_splits(W, tpw, smax);
}

// W of requests base + lane (0 past the batch)
__device__ __forceinline__ int lane_work(const amass_decode_args& a, int base, int kh0, int hw) {
    const int r = base + (threadIdx.x & 63);
    return r < a.n_req ? req_work(a, r, kh0, hw) : 0;
}

// Workgroups the whole batch takes at `tpw` (every lane gets the sum).  w0 = lane_work(0).
// Splits the whole batch takes at `tpw` (every lane gets the sum).  w0 = lane_work(0).
__device__ __forceinline__ int plan_total(const amass_decode_args& a, int w0, int kh0, int hw,
                                          int tpw, int smax) {
    const int lane = threadIdx.x & 63;
    int tot = wave_sum_uniform(lane < a.n_req ? req_splits(w0, tpw, smax) : 0);
    for (int base = WAVE; base < a.n_req; base += WAVE)
        tot += wave_sum_uniform(base + lane < a.n_req
                                    ? req_splits(lane_work(a, base, kh0, hw), tpw, smax) : 0);
    return tot;
}

// The launch's layout (whole) and pages per split (tpw).
__device__ __forceinline__ void plan_setup(const amass_decode_args& a, int w0, int kh0, int hw,
                                           int plan, int target, int smax, bool& whole,
                                           int& tpw) {
    whole = plan == 2;
    tpw = a.pps_min;
    if (plan != 0) return;
    int total = wave_sum_uniform(w0), wmax = wave_max_uniform(w0);
    for (int base = WAVE; base < a.n_req; base += WAVE) {
        const int w = lane_work(a, base, kh0, hw);
        total += wave_sum_uniform(w);
        wmax = max(wmax, wave_max_uniform(w));
    }
    int lo = max(a.pps_min, (total + target - 1) / target);
    // whole: a batch that cannot fill the resident workgroups, unless its longest unit
    // spread over one workgroup's waves takes more page steps than a split (lo pages)
    // plus the merge would -- few units with many pages (e.g. one request's dense
    // decode) stream faster split
    if (total <= DEC_WHOLE_PPS * target && (wmax + hw - 1) / hw <= lo + 2) {
        whole = true;
        return;
    }
    if (plan_total(a, w0, kh0, hw, lo, smax) <= target) {   // uniform batches
        tpw = lo;
        return;
    }
    int hi = max(lo, wmax);                  // at hi every request takes one split
    ++lo;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (plan_total(a, w0, kh0, hw, mid, smax) <= target) hi = mid;
        else lo = mid + 1;
    }
    tpw = lo;
}

__device__ __forceinline__ bool split_walk(const amass_decode_args& a, int w0, int kh0, int hw,
                                           int nh, bool whole, int tpw, int smax, int x,
                                           SplitPlan& p) {
    const int lane = threadIdx.x & 63;
    int before = 0;                                     // workgroups of earlier batches
    for (int base = 0; base < a.n_req; base += WAVE) {
        const int r = base + lane;
        const int w = base == 0 ? w0 : lane_work(a, base, kh0, hw);
        const int n = r < a.n_req ? req_units(w, whole, tpw, smax, nh) : 0;
        const int incl = wave_incl_scan(n);
        const int in_batch = __builtin_amdgcn_readlane(incl, WAVE - 1);
        if (x < before + in_batch) {
            const unsigned long long hit = __ballot(before + incl > x);
            const int src = __ffsll((long long)hit) - 1;
            p.req = base + src;
            p.S = __builtin_amdgcn_readlane(n, src);
            p.s = x - before - __builtin_amdgcn_readlane(incl - n, src);
            return true;
        }
        before += in_batch;
    }
    return false;
}

// The last partial slot of a unit holds its split count (int32) for merge_kernel.
__device__ __forceinline__ int* split_count_slot(const amass_decode_args& a, int r, int kh) {
    return reinterpret_cast<int*>(a.m_part) +
           (((int64_t)r * a.n_kv + kh) * a.split + (a.split - 1)) * a.G;
}

// Workgroup x = blockIdx.x of head group blockIdx.y, request p.req:
//   whole: head kh0 + p.s; wave w attends pages w, w + waves, ...; LDS merge; output.
//   split: split p.s; wave w attends pages s, s + S_r, ... of head kh0 + w.  S_r = 1:
//     normalise and write out; S_r > 1: write the split's LSE partial (slot s).
// `sarg` is the plan's target (path 0) or its fixed S (path 1).
template <int VSRC, bool DENSE>
__global__ __launch_bounds__(DEC_WAVES * WAVE) void decode_kernel(const amass_decode_args a,
                                                                  int plan, int sarg) {
    __shared__ WholeLds wl;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int hw = blockDim.x >> 6;
    const int kh0 = blockIdx.y * hw;
    const int nh = min(hw, a.n_kv - kh0);
    const int cap = plan == 2 ? 1 : a.split - 1;     // partial slots besides the count slot
    const int smax = plan == 1 ? min(sarg, cap) : cap;
    const int w0 = lane_work(a, 0, kh0, hw);
    bool whole;
    int tpw;
    plan_setup(a, w0, kh0, hw, plan, sarg, smax, whole, tpw);
    SplitPlan pl;
    if (!split_walk(a, w0, kh0, hw, nh, whole, tpw, smax, blockIdx.x, pl)) return;
    const int r = pl.req;
    const int sl = a.seq_lens[r];
    WaveState st;
    init_state(st);

    if (whole) {
        // ---- one head, the workgroup's waves split its pages, LDS merge ---------------
        const int kh = kh0 + pl.s;
        if (plan != 2 && threadIdx.x == 0) *split_count_slot(a, r, kh) = 1;
        attend_whole<VSRC, DENSE>(a, r, kh, sl, unit_count<DENSE>(a, r, kh, sl), hw, wl);
        return;
    }

    // ---- split layout: one wave per head --------------------------------------------------
    const int kh = kh0 + w;
    if (kh >= a.n_kv) return;
    const int s = pl.s, S = pl.S;
    const int cnt = unit_count<DENSE>(a, r, kh, sl);
    if (s < cnt) {
        bf16x4_t qb[8];
        load_q(a, r, kh, lane, qb);
        attend_run<VSRC, DENSE>(a, r, kh, sl, s, cnt, S, lane, qb, st);
    }
    if (plan != 2 && s == 0 && lane == 0) *split_count_slot(a, r, kh) = S;
    const float lt = xor32_sumf(xor16_sumf(st.l));   // sum over lanes g, g+16, g+32, g+48
    // this lane holds rows g = 4 (l/16) + j, columns d = 8 (l%16) .. +8 of the O tiles
    const int d0 = 8 * (lane & 15);
    if (S == 1) {
        // rows of 8 bf16 are 16-byte aligned for the usual contiguous (T, H, d) output
        const bool out16 = ((((uintptr_t)a.out) | (uintptr_t)(a.o_st * 2) |
                             (uintptr_t)(a.o_hs * 2)) & 15) == 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int g = 4 * (lane >> 4) + j;
            const float lg = __shfl(lt, g, WAVE);
            if (g < a.G) {
                const float inv = lg > 0.f ? 1.f / lg : 0.f;
                const uint4 o = {pack_bf16x2(st.acc[0][j] * inv, st.acc[1][j] * inv),
                                 pack_bf16x2(st.acc[2][j] * inv, st.acc[3][j] * inv),
                                 pack_bf16x2(st.acc[4][j] * inv, st.acc[5][j] * inv),
                                 pack_bf16x2(st.acc[6][j] * inv, st.acc[7][j] * inv)};
                uint16_t* dst = (uint16_t*)a.out + (int64_t)r * a.o_st +
                                (int64_t)(kh * a.G + g) * a.o_hs + d0;
                if (out16) {
                    *reinterpret_cast<uint4*>(dst) = o;
                } else {
                    uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
                    d32[0] = o.x; d32[1] = o.y; d32[2] = o.z; d32[3] = o.w;
                }
            }
        }
    } else {
        const int64_t pg0 = (((int64_t)r * a.n_kv + kh) * a.split + s) * a.G;   // slot s
        if (lane < a.G) {
            a.m_part[pg0 + lane] = st.m;
            a.l_part[pg0 + lane] = lt;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int g = 4 * (lane >> 4) + j;
            if (g < a.G) {
                float4* dst = reinterpret_cast<float4*>(a.acc_part + (pg0 + g) * DEC_D + d0);
                dst[0] = make_float4(st.acc[0][j], st.acc[1][j], st.acc[2][j], st.acc[3][j]);
                dst[1] = make_float4(st.acc[4][j], st.acc[5][j], st.acc[6][j], st.acc[7][j]);
            }
        }
    }
}

// LSE merge of the split-K partials of head g = blockIdx.z of unit (kh = blockIdx.x,
// r = blockIdx.y): m* = max m_s over the non-empty partials, w_s = exp(m_s - m*),
// out = sum w_s acc_s / sum w_s l_s (attention/merge.py:21-50).  The unit's split count
// comes from its count slot; units written directly (count 1) are skipped.  Each of the
// four waves merges every fourth partial (lane = a pair of d) with a running maximum, so
// all of a thread's loads are independent of the others' results; the four (m, l, acc)
// then combine through LDS the same way.
constexpr int MG_WAVES = 4;

__global__ __launch_bounds__(MG_WAVES * WAVE) void merge_kernel(const amass_decode_args a) {
    const int kh = blockIdx.x, r = blockIdx.y, g = blockIdx.z;
    const int S = *split_count_slot(a, r, kh);
    if (S <= 1) return;
    const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
    const int64_t ubase = ((int64_t)r * a.n_kv + kh) * a.split;
    __shared__ float sh_m[MG_WAVES], sh_l[MG_WAVES];
    __shared__ float2 sh_o[MG_WAVES][WAVE];
    float m = -INFINITY, lsum = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll 4
    for (int x = grp; x < S; x += MG_WAVES) {
        const int64_t pg = (ubase + x) * a.G + g;
        const float ls = a.l_part[pg], ms = a.m_part[pg];
        const float2 v = *reinterpret_cast<const float2*>(a.acc_part + pg * DEC_D + 2 * lane);
        if (ls > 0.f) {                                 // empty partials carry no weight
            const float mn = fmaxf(m, ms);
            const float al = __expf(m - mn), be = __expf(ms - mn);
            lsum = lsum * al + ls * be;
            o0 = o0 * al + v.x * be;
            o1 = o1 * al + v.y * be;
            m = mn;
        }
    }
    sh_o[grp][lane] = make_float2(o0, o1);
    if (lane == 0) {
        sh_m[grp] = m;
        sh_l[grp] = lsum;
    }
    __syncthreads();
    if (grp != 0) return;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < MG_WAVES; ++w)
        if (sh_l[w] > 0.f) M = fmaxf(M, sh_m[w]);
    float l = 0.f;
    o0 = 0.f;
    o1 = 0.f;
#pragma unroll
    for (int w = 0; w < MG_WAVES; ++w) {
        const float wt = sh_l[w] > 0.f ? __expf(sh_m[w] - M) : 0.f;
        l += sh_l[w] * wt;
        o0 += sh_o[w][lane].x * wt;
        o1 += sh_o[w][lane].y * wt;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint32_t* out = reinterpret_cast<uint32_t*>((uint16_t*)a.out + (int64_t)r * a.o_st +
                                                (int64_t)(kh * a.G + g) * a.o_hs + 2 * lane);
    *out = pack_bf16x2(o0 * inv, o1 * inv);
}


// Workgroups of the decode kernel resident per CU (queried once per instance).
// Resident workgroups of `waves` waves per CU (cached per wave count) and the CU count.
template <int VSRC, bool DENSE>
static int decode_resident(int waves, int& cus) {
    static int per_cu[DEC_WAVES + 1] = {0};
    static int ncu = 0;
    if (per_cu[waves] == 0) {
        int dev = 0, p = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&p, decode_kernel<VSRC, DENSE>,
                                                         waves * WAVE, 0) != hipSuccess ||
            p < 1) {
            cus = 256;
            return 1;
        }
        ncu = n;
        per_cu[waves] = p;
    }
    cus = ncu;
    return per_cu[waves];
}

template <int VSRC, bool DENSE>
static int launch_decode(amass_decode_args a, int path, hipStream_t s) {
    const int hw = a.n_kv < DEC_WAVES ? a.n_kv : DEC_WAVES;     // heads (waves) per workgroup
    const int hg = (a.n_kv + hw - 1) / hw;                       // head groups
    // paths 0, 1 keep the last partial slot of a unit for its split count: splitting
    // needs at least 3 slots, otherwise the fused single pass serves every head
    const int plan = (path != 2 && a.split < 3) ? 2 : path;
    int sarg = 1, grid = a.n_req * hw;
    if (plan == 0) {
        // balanced plan over one resident round of workgroups per head group
        int cus = 0;
        const int resident = decode_resident<VSRC, DENSE>(hw, cus) * cus;
        sarg = (resident + hg - 1) / hg;
        grid = sarg > grid ? sarg : grid;   // >= the plan's total (<= target, or n_req * hw)
    } else if (plan == 1) {
        sarg = a.split - 1;
        grid = a.n_req * sarg;
    }
    if (plan != 2 && (!a.m_part || !a.l_part || !a.acc_part)) return AMASS_ERR_NULL;
    hipLaunchKernelGGL((decode_kernel<VSRC, DENSE>), dim3(grid, hg), dim3(hw * WAVE), 0, s, a,
                       plan, sarg);
    int rc = check_launch();
    if (rc || plan == 2) return rc;
    hipLaunchKernelGGL(merge_kernel, dim3(a.n_kv, a.n_req, a.G), dim3(MG_WAVES * WAVE), 0, s, a);
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
    // K and V rows are read as 16-byte (8-element) loads, q as 8-byte loads, out written
    // at least 4 bytes at a time
    const auto off = [](const void* p, uintptr_t align) { return ((uintptr_t)p & (align - 1)) != 0; };
    if (off(a.k, 16) || ((a.k_sb | a.k_st | a.k_sh) & 7)) return AMASS_ERR_GEOMETRY;
    if (a.v && (off(a.v, 16) || ((a.v_sb | a.v_st | a.v_sh) & 7))) return AMASS_ERR_GEOMETRY;
    if (a.v_src == 1 && (off(a.hot, 16) || off(a.pool, 16))) return AMASS_ERR_GEOMETRY;
    if (off(a.q, 8) || ((a.q_st | a.q_hs) & 3)) return AMASS_ERR_GEOMETRY;
    if (off(a.out, 4) || ((a.o_st | a.o_hs) & 1)) return AMASS_ERR_GEOMETRY;
    if (a.n_req == 0) return AMASS_OK;
    if (a.dense) return launch_decode<0, true>(a, a.path, s);
    if (a.v_src == 1) return launch_decode<1, false>(a, a.path, s);
    return launch_decode<0, false>(a, a.path, s);
}

// ------------------------------------------------------------------ allocation-free variant
// The split-K partials live in one file-scope device array (each GPU holds its own copy
// for the life of the process).  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in symbol): the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current and kept.
constexpr int64_t DEC_SCRATCH_BYTES = AMASS_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[DEC_SCRATCH_BYTES / sizeof(float)];

constexpr int DEC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[DEC_MAX_DEVICES] = {nullptr};

static int scratch_address(float** out) {
    int dev = 0;
    int rc = record_hip(hipGetDevice(&dev));
    if (rc) return rc;
    if (dev < 0 || dev >= DEC_MAX_DEVICES) return AMASS_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        rc = record_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (rc) return rc;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return AMASS_OK;
}

// Bytes of partials a launch of `a` uses: m and l (R, n_kv, split, G) each, then acc
// (R, n_kv, split, G, d) at a 256-byte boundary; 0 when only the fused pass runs.
static int64_t decode_partial_bytes(const amass_decode_args& a, int64_t& acc_off) {
    acc_off = 0;
    if (a.path == 2 || a.split < 3) return 0;
    const int64_t slots = (int64_t)a.n_req * a.n_kv * a.split * a.G;
    acc_off = ((2 * slots * (int64_t)sizeof(float)) + 255) & ~(int64_t)255;
    return acc_off + slots * DEC_D * (int64_t)sizeof(float);
}

static int decode_noalloc(const amass_decode_args* ain, hipStream_t s) {
    if (!ain) return AMASS_ERR_NULL;
    amass_decode_args a = *ain;
    if (a.n_req < 0 || a.n_kv < 1 || a.G < 1 || a.G > 8 || a.d != DEC_D) return AMASS_ERR_GEOMETRY;
    if (a.path != 2 && a.split < 1) return AMASS_ERR_GEOMETRY;
    if (a.path != 2 && a.split >= 3 && a.n_req > 0) {
        // partial slots per unit: at most what the array holds (alignment pad < 256 B);
        // the device plan never splits a unit into more than split - 1 parts
        const int64_t per_slot = (int64_t)a.n_req * a.n_kv * a.G * (2 + DEC_D) * (int64_t)sizeof(float);
        const int64_t fit = (DEC_SCRATCH_BYTES - 256) / per_slot;
        if (fit < 3) return AMASS_ERR_CAPACITY;
        if (fit < a.split) a.split = (int)fit;
    }
    int64_t acc_off = 0;
    const int64_t need = decode_partial_bytes(a, acc_off);
    if (need > DEC_SCRATCH_BYTES) return AMASS_ERR_CAPACITY;
    float* base = nullptr;
    const int rc = scratch_address(&base);
    if (rc) return rc;
    const int64_t slots = (int64_t)a.n_req * a.n_kv * (a.split > 0 ? a.split : 1) * a.G;
    a.m_part = base;
    a.l_part = base + slots;
    a.acc_part = base + acc_off / (int64_t)sizeof(float);
    return decode_common(&a, 0, -1, s);
}

}  // namespace amass

using namespace amass;

extern "C" int amass_sparse_decode(const amass_decode_args* a, void* stream) {
    return decode_common(a, 0, -1, (hipStream_t)stream);
}
extern "C" int amass_sparse_decode_noalloc(const amass_decode_args* a, void* stream) {
    return decode_noalloc(a, (hipStream_t)stream);
}
extern "C" int amass_dense_paged_decode(const amass_decode_args* a, void* stream) {
    return decode_common(a, 1, -1, (hipStream_t)stream);
}
extern "C" int amass_tier_decode(const amass_decode_args* a, void* stream) {
    return decode_common(a, 0, 1, (hipStream_t)stream);
}
