// Stage-A selection for gfx950: derive params, nrm combine, top-b / coverage nucleus.
//
// One workgroup (512 or 1024 threads) per (request, kv-head), the unit's pages held in
// registers.  The b-th largest score is found by an MSD digit search over order-preserving
// uint32 keys (2048-bin LDS histograms of 11 key bits; in coverage mode each bin also
// accumulates the 2^-32 fixed-point page mass with 64-bit LDS atomics, so the cut is
// found by mass instead of by count), usually one histogram followed by an exact ranking
// of the chosen bin's keys by one wave.  The keep test and the ascending compaction rank
// ties at tau by page index.
//
// Semantics follow selection/select.py:60-101 (_topb_select_kernel): keep =
// (selectable & chosen) | p < sink | p >= n_sel_hi | (n_sel_hi - sink <= 1), compaction
// ascending with -1 padding, page_cnt.  tie_mode 0 keeps exactly b pages (ties at the
// b-th score -> lower page index); tie_mode 1 is the reference threshold rule score >= tau.
#include "select_unit.h"

namespace amass {

constexpr int SEL_THREADS = 512;
constexpr int SEL_WAVES = SEL_THREADS / WAVE;
constexpr int SEL_MAXP = 16384;   // pages per request: 32 per thread of the selection

// ------------------------------------------------------------------ derive params
__global__ void derive_kernel(const int32_t* __restrict__ sl, int32_t* __restrict__ npg,
                              int32_t* __restrict__ nsh, int32_t* __restrict__ bfix,
                              double budget, int n_req, int page, int win, int sink) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n_req) return;
    const int s = sl[r];
    const int np = (s + page - 1) / page;
    const int nh = np - win;
    const int S = nh - sink;
    const double bf = ceil((double)S * budget);
    int b = (int)bf;
    b = b > 1 ? b : 1;
    const int smax = S > 1 ? S : 1;
    b = b < smax ? b : smax;
    npg[r] = np;
    nsh[r] = nh;
    bfix[r] = b;
}

// ------------------------------------------------------------------ nrm combine
// Per-head maxima m[0..G) of the block: wave reductions, one LDS exchange, one barrier.
__device__ __forceinline__ void head_max(float* m, int G, float (*red)[SEL_WAVES]) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G) {
            const float x = wave_maxf_uniform(m[g]);
            if ((threadIdx.x & 63) == 0) red[g][w] = x;
        }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G) {
            float x = red[g][0];
#pragma unroll
            for (int i = 1; i < SEL_WAVES; ++i) x = fmaxf(x, red[g][i]);
            m[g] = x;
        }
}

struct NoTrack {
    __device__ void operator()(int, float) const {}
};

// V consecutive floats src[p..p+V): one vector load when the run is whole, else guarded
// scalar loads (`fill` past n).  Vector runs need src 16-byte aligned and p % V == 0.
template <int V>
__device__ __forceinline__ void ld_run(const float* __restrict__ src, int p, int n, float fill,
                                       float* o) {
    if (p + V <= n) {
        if constexpr (V == 4) {
            const float4 x = *reinterpret_cast<const float4*>(src + p);
            o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
        } else if constexpr (V == 2) {
            const float2 x = *reinterpret_cast<const float2*>(src + p);
            o[0] = x.x; o[1] = x.y;
        } else {
            o[0] = src[p];
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = p + i < n ? src[p + i] : fill;
    }
}
template <int V>
__device__ __forceinline__ void st_run(float* __restrict__ dst, int p, int n, const float* v) {
    if (p + V <= n) {
        if constexpr (V == 4) {
            *reinterpret_cast<float4*>(dst + p) = make_float4(v[0], v[1], v[2], v[3]);
        } else if constexpr (V == 2) {
            *reinterpret_cast<float2*>(dst + p) = make_float2(v[0], v[1]);
        } else {
            dst[p] = v[0];
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i)
            if (p + i < n) dst[p + i] = v[i];
    }
}

// nrm combine of one (request, kv-head) over pages [0, n):
//   hmax_g = max_p sh[g][p];  score[p] = sum_{g ascending} exp(sh[g][p] - hmax_g)
// written to `gs` (global) and `lds` (if non-null); track(p, score) sees every page.
// Thread t takes runs of V pages at V*t + k*V*SEL_THREADS; all NB runs x G heads of a batch
// are loaded before any is used.  REG: the whole unit fits one batch (n <= V*NB*threads)
// and stays in registers between the max and the sum, otherwise the sum pass reloads.
template <int V, int NB, bool REG, typename Track>
__device__ void nrm_run(const float* __restrict__ sh, int64_t sg, int G, int n, float* lds,
                        float* __restrict__ gs, float (*red)[SEL_WAVES], Track& track) {
    constexpr int RUN = V * SEL_THREADS;
    constexpr int STEP = RUN * NB;
    const int tid = threadIdx.x;
    float m[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) m[g] = -INFINITY;
    float v[NB][8][V];
    auto load = [&](int p0, float fill) {
#pragma unroll
        for (int k = 0; k < NB; ++k)
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                if (g < G) {
                    ld_run<V>(sh + g * sg, p0 + k * RUN, n, fill, v[k][g]);
                } else {
#pragma unroll
                    for (int i = 0; i < V; ++i) v[k][g][i] = fill;
                }
            }
    };
    auto combine = [&](int p0) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int p = p0 + k * RUN;
            if (p < n) {
                float acc[V];
#pragma unroll
                for (int i = 0; i < V; ++i) acc[i] = 0.f;
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    if (g < G)
#pragma unroll
                        for (int i = 0; i < V; ++i) acc[i] += nrm_exp(v[k][g][i] - m[g]);
                st_run<V>(gs, p, n, acc);
#pragma unroll
                for (int i = 0; i < V; ++i)
                    if (p + i < n) {
                        if (lds) lds[p + i] = acc[i];
                        track(p + i, acc[i]);
                    }
            }
        }
    };
    auto fold_max = [&]() {
#pragma unroll
        for (int k = 0; k < NB; ++k)
#pragma unroll
            for (int g = 0; g < 8; ++g)
#pragma unroll
                for (int i = 0; i < V; ++i) m[g] = fmaxf(m[g], v[k][g][i]);
    };
    if (REG) {
        load(tid * V, -INFINITY);
        fold_max();
        head_max(m, G, red);
        combine(tid * V);
        return;
    }
    for (int p0 = tid * V; p0 < n; p0 += STEP) {
        load(p0, -INFINITY);
        fold_max();
    }
    head_max(m, G, red);
    for (int p0 = tid * V; p0 < n; p0 += STEP) {
        load(p0, 0.f);
        combine(p0);
    }
}

template <typename Track>
__device__ void nrm_stage(const float* __restrict__ sh, int64_t sg, int G, int n, float* lds,
                          float* __restrict__ gs, float (*red)[SEL_WAVES], Track& track) {
    const bool al = ((((uintptr_t)sh) | ((uintptr_t)gs)) & 15) == 0 && (sg & 3) == 0;
    if (n <= 2 * SEL_THREADS) {
        if (al) nrm_run<2, 1, true>(sh, sg, G, n, lds, gs, red, track);
        else nrm_run<1, 2, true>(sh, sg, G, n, lds, gs, red, track);
    } else {
        if (al) nrm_run<4, 2, false>(sh, sg, G, n, lds, gs, red, track);
        else nrm_run<1, 4, false>(sh, sg, G, n, lds, gs, red, track);
    }
}

// plain scores: gs[0, n) -> lds, track(p, score)
template <int V, int NB, typename Track>
__device__ void copy_run(const float* __restrict__ gs, int n, float* lds, Track& track) {
    constexpr int RUN = V * SEL_THREADS;
    for (int p0 = threadIdx.x * V; p0 < n; p0 += RUN * NB) {
        float v[NB][V];
#pragma unroll
        for (int k = 0; k < NB; ++k) ld_run<V>(gs, p0 + k * RUN, n, 0.f, v[k]);
#pragma unroll
        for (int k = 0; k < NB; ++k)
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const int p = p0 + k * RUN + i;
                if (p < n) {
                    lds[p] = v[k][i];
                    track(p, v[k][i]);
                }
            }
    }
}

// ------------------------------------------------------------------ nrm standalone
__global__ __launch_bounds__(SEL_THREADS) void nrm_kernel(const amass_nrm_args a) {
    __shared__ float red[8][SEL_WAVES];
    const int kh = blockIdx.x, r = blockIdx.y;
    const int nsh = min(a.n_sel_hi[r], a.max_pages);
    if (nsh <= 0) return;
    const float* sh = a.score_h + (int64_t)r * a.sh_sr + (int64_t)kh * a.sh_sh;
    float* out = a.score + (int64_t)r * a.sc_sr + (int64_t)kh * a.sc_sh;
    NoTrack nt;
    nrm_stage(sh, a.sh_sg, a.G, nsh, nullptr, out, red, nt);
}

// the nrm pages of a unit: min(n_sel_hi, n_pages, max_pages), >= 0
__device__ __forceinline__ int scored_pages(const amass_select_args& a, int r) {
    const int np = min(a.n_pages[r], a.max_pages);
    const int ns = min(a.n_sel_hi[r], np);
    return ns > 0 ? ns : 0;
}

// Per-head maxima over the block: wave reductions, one LDS exchange, one barrier.
template <int WAVES, int CAP>
__device__ __forceinline__ void block_head_max(float* m, int G, float (*red)[CAP]) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G) {
            const float x = wave_maxf_uniform(m[g]);
            if ((threadIdx.x & 63) == 0) red[g][w] = x;
        }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G) {
            float x = red[g][0];
#pragma unroll
            for (int i = 1; i < WAVES; ++i) x = fmaxf(x, red[g][i]);
            m[g] = x;
        }
}

// The nrm combine of NP_PAGES pages of one unit (workgroup (kv-head, request, chunk)):
// score[p] = sum_{g ascending} exp(score_h[g][p] - hmax_g), hmax_g = the maximum of the
// unit's per-tile maxima (the same maxima and sums as the fused staging).  The score_h
// loads are issued before the maxima are read and reduced.
__global__ __launch_bounds__(NP_THREADS) void nrm_pass_kernel(const amass_select_args a) {
    constexpr int TPT = (SEL_MAXP / XS_TILE) / NP_THREADS;   // tile maxima per thread
    __shared__ float red[8][NP_THREADS / WAVE];
    // chunk is the slowest grid dimension: workgroups are dealt to the 8 XCDs round-robin
    // in grid order, so (with n_kv * n_req a multiple of 8) a unit's chunks share one XCD
    // and its L2 -- the unit's tile maxima, which every chunk reads, come from HBM once
    // per unit, and the selection launch after (grid (n_kv, n_req)) finds the unit's
    // combined scores in the same XCD's L2
    const int kh = blockIdx.x, r = blockIdx.y, chunk = blockIdx.z;
    const int tid = threadIdx.x, G = a.G, MP = a.max_pages;
    const int p0 = chunk * NP_PAGES;
    const float* sh = a.score_h + (int64_t)r * a.sh_sr + (int64_t)kh * a.sh_sh;
    const float* tm = a.tile_max + (int64_t)r * a.tm_sr + (int64_t)kh * a.tm_sh;
    float* gs = a.score + (int64_t)r * a.sc_sr + (int64_t)kh * a.sc_sh;
    const bool vec = ((((uintptr_t)sh) | ((uintptr_t)gs)) & 15) == 0 && (a.sh_sg & 3) == 0;
    // loads first: the row's pages and tile maxima are in bounds (rows are MP wide)
    float v[8][4];                              // [head][page]: pages p0 + 4 tid + {0..3}
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G) ld_pages<4>(sh + g * a.sh_sg, p0 + 4 * tid, MP, vec, -INFINITY, v[g]);
    const int ntm = (MP + XS_TILE - 1) / XS_TILE;
    float tv[8][TPT];
#pragma unroll
    for (int g = 0; g < 8; ++g)
#pragma unroll
        for (int k = 0; k < TPT; ++k) {
            const int t = tid + k * NP_THREADS;
            tv[g][k] = (g < G && t < ntm) ? tm[g * a.tm_sg + t] : -INFINITY;
        }
    const int n = scored_pages(a, r);
    if (p0 >= n) return;                        // uniform over the workgroup
    const int nt = (n + XS_TILE - 1) / XS_TILE;
    float m[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        m[g] = -INFINITY;
#pragma unroll
        for (int k = 0; k < TPT; ++k)
            if (tid + k * NP_THREADS < nt) m[g] = fmaxf(m[g], tv[g][k]);
    }
    block_head_max<NP_THREADS / WAVE, NP_THREADS / WAVE>(m, G, red);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += nrm_exp(v[g][i] - m[g]);
    st_pages<4>(gs, p0 + 4 * tid, n, vec, acc);
}

template <int NT, int PPT, bool NRM>
__global__ __launch_bounds__(NT) void select_kernel(const amass_select_args a) {
    __shared__ XSel s;
    select_unit<NT, PPT, NRM>(a, blockIdx.y, blockIdx.x, s);
}

template <int NT, int PPT>
static void launch_select(const amass_select_args& k, bool fused, hipStream_t st) {
    if constexpr (NT == XS_THREADS && PPT <= 8) {
        if (fused) {
            hipLaunchKernelGGL((select_kernel<NT, PPT, true>), dim3(k.n_kv, k.n_req), dim3(NT),
                               0, st, k);
            return;
        }
    }
    hipLaunchKernelGGL((select_kernel<NT, PPT, false>), dim3(k.n_kv, k.n_req), dim3(NT), 0,
                       st, k);
}

}  // namespace amass

using namespace amass;

extern "C" int amass_derive_params(const amass_derive_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->seq_lens || !a->n_pages || !a->n_sel_hi || !a->b_fix) return AMASS_ERR_NULL;
    if (a->page < 1 || a->window_pages < 1 || a->sink_pages < 0 || a->n_req < 0)
        return AMASS_ERR_GEOMETRY;
    if (!(a->budget > 0.0 && a->budget <= 1.0)) return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    const int blk = 256;
    hipLaunchKernelGGL(derive_kernel, dim3((a->n_req + blk - 1) / blk), dim3(blk), 0,
                       (hipStream_t)stream, a->seq_lens, a->n_pages, a->n_sel_hi, a->b_fix,
                       a->budget, a->n_req, a->page, a->window_pages, a->sink_pages);
    return check_launch();
}

extern "C" int amass_nrm_combine(const amass_nrm_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->score_h || !a->score || !a->n_sel_hi) return AMASS_ERR_NULL;
    if (a->G < 1 || a->G > 8 || a->n_kv < 1 || a->max_pages < 1) return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    hipLaunchKernelGGL(nrm_kernel, dim3(a->n_kv, a->n_req), dim3(SEL_THREADS), 0,
                       (hipStream_t)stream, *a);
    return check_launch();
}

static int select_common(const amass_select_args* a, int mode, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->score || !a->n_pages || !a->n_sel_hi || !a->page_table || !a->page_cnt)
        return AMASS_ERR_NULL;
    if (mode == 0 && !a->b_fix) return AMASS_ERR_NULL;
    if (a->n_kv < 1 || a->max_pages < 1 || a->sink_pages < 0) return AMASS_ERR_GEOMETRY;
    if (a->score_h && (a->G < 1 || a->G > 8)) return AMASS_ERR_GEOMETRY;
    if (a->tile_max && !a->score_h) return AMASS_ERR_GEOMETRY;
    if (a->max_pages > SEL_MAXP) return AMASS_ERR_CAPACITY;
    if (a->tie_mode != 0 && a->tie_mode != 1) return AMASS_ERR_GEOMETRY;
    if (a->score_kind != 0 && a->score_kind != 1) return AMASS_ERR_GEOMETRY;
    if (mode == 1 && !(a->coverage > 0.0 && a->coverage <= 1.0)) return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    amass_select_args k = *a;
    k.mode = mode;
    hipStream_t st = (hipStream_t)stream;
    int ppt = 1;
    while (ppt * XS_THREADS < k.max_pages) ppt *= 2;           // <= 32 (SEL_MAXP)
    bool fused = false;
    if (k.score_h) {
        fused = k.tile_max && ppt <= 8 && ppt * k.G <= XS_FUSED;
        if (!fused) {
            // the combined scores first (many workgroups with the per-tile maxima, else
            // the standalone two-pass combine), then the selection over st.score
            if (k.tile_max) {
                const int chunks = (k.max_pages + NP_PAGES - 1) / NP_PAGES;
                hipLaunchKernelGGL(nrm_pass_kernel, dim3(k.n_kv, k.n_req, chunks),
                                   dim3(NP_THREADS), 0, st, k);
            } else {
                amass_nrm_args na;
                na.score_h = k.score_h; na.sh_sr = k.sh_sr; na.sh_sh = k.sh_sh; na.sh_sg = k.sh_sg;
                na.score = k.score; na.sc_sr = k.sc_sr; na.sc_sh = k.sc_sh;
                na.n_sel_hi = k.n_sel_hi;
                na.n_req = k.n_req; na.n_kv = k.n_kv; na.G = k.G; na.max_pages = k.max_pages;
                hipLaunchKernelGGL(nrm_kernel, dim3(k.n_kv, k.n_req), dim3(SEL_THREADS), 0, st, na);
            }
            const int rc = check_launch();
            if (rc) return rc;
        }
    }
    // 512 threads up to 4096 pages (1..8 per thread) and beyond 8192 (32), 1024 threads
    // for 4097 .. 8192 pages (8 per thread)
    switch (ppt) {
        case 1: launch_select<XS_THREADS, 1>(k, fused, st); break;
        case 2: launch_select<XS_THREADS, 2>(k, fused, st); break;
        case 4: launch_select<XS_THREADS, 4>(k, fused, st); break;
        case 8: launch_select<XS_THREADS, 8>(k, fused, st); break;
        case 16: launch_select<XS_THREADS_L, 8>(k, fused, st); break;
        default: launch_select<XS_THREADS, 32>(k, fused, st); break;
    }
    return check_launch();
}

extern "C" int amass_topb_select(const amass_select_args* a, void* stream) {
    return select_common(a, 0, stream);
}
extern "C" int amass_coverage_select(const amass_select_args* a, void* stream) {
    return select_common(a, 1, stream);
}
