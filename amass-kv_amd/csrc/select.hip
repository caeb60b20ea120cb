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
#include "common.h"

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

// ------------------------------------------------------------------ wave helpers
// number of set bits of `m` below this lane
__device__ __forceinline__ int lanes_below(unsigned long long m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// ------------------------------------------------------------------ nrm combine
// The nrm combine's exp (every combine site uses this one, so the standalone, fused and
// pre-pass combines agree bit for bit): the hardware exp2 of x log2(e), ~1e-7 relative.
__device__ __forceinline__ float nrm_exp(float x) { return __expf(x); }

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

// ------------------------------------------------------------------ selection
// One workgroup of NT threads per (request, kv-head) (512; 1024 for units of 4097 to 8192
// pages); thread t holds pages c * V * NT + V t + i (chunk c < NC, i < V, V * NC = PPT) in
// registers from the first load to the page-table write, so every phase reads registers
// and LDS carries only the histogram and small exchanges.  Phases:
//   stage    plain scores, or the fused nrm combine over score_h with the per-head maxima
//            that every wave reduces itself from the score launch's per-tile maxima; the
//            loads cover the row's MP pages and are issued before n_sel_hi arrives (the
//            rows are MP wide); from then on each thread holds its pages' order keys;
//   search   tau = the b-th largest key (count) or the key where the mass from the top
//            reaches `need` (coverage): 2048-bin histograms of the key relative to the
//            unit's smallest selectable key, 11 bits at a time from its highest set bit,
//            each searched by one wave in two levels (xs_find); a chosen bin of <= 64
//            keys is ranked by one wave, exactly;
//   compact  per-chunk wave scans of packed keep / tie counts, one exchange, then every
//            thread writes its kept pages at their ranks (ascending page ids).
// Every cross-lane reduction and scan uses DPP row steps and readlane (no LDS permutes).
// Large nrm units (MP G beyond the fused staging's registers) get a pre-pass over many
// workgroups (nrm_pass_kernel) that writes the combined scores; the selection then reads
// those.  Without per-tile maxima the standalone two-pass nrm_kernel does that.
constexpr int XS_THREADS = 512;              // units up to 4096 pages (and above 8192)
constexpr int XS_THREADS_L = 1024;            // units of 4097 .. 8192 pages
constexpr int XS_WAVES = XS_THREADS_L / WAVE; // exchange arrays sized for the larger block
constexpr int XS_BITS = 11;                   // key bits per histogram digit
constexpr int XS_BINS = 1 << XS_BITS;         // 64 groups of 32 for the two-level search
constexpr int XS_PBINS_M = XS_BINS + XS_BINS / 16;  // mass slots: 2 unused after every 32 bins
constexpr int XS_PBINS_C = XS_BINS + XS_BINS / 8;   // count slots: 4 unused after every 32
constexpr int XS_CAND = WAVE;                 // a bin this small is ranked by one wave
constexpr int XS_TILE = 16;                   // pages per per-tile maximum of score_h
constexpr int XS_FUSED = 64;                  // PPT * G floats of the fused nrm staging
constexpr int XS_MAXNC = 8;                   // chunks per thread at PPT = 32
constexpr int NP_THREADS = 256;               // nrm pre-pass workgroup
constexpr int NP_PAGES = 4 * NP_THREADS;      // pages per pre-pass workgroup

// Histogram slots: each group of 32 bins starts on a 16-byte boundary followed by 16
// unused bytes (mass group g at slot 34 g, count group g at slot 36 g), so the 64 lanes
// that each read one group with 16-byte loads spread evenly over the LDS banks.
__device__ __forceinline__ unsigned int xs_pad_m(unsigned int b) { return b + 2 * (b >> 5); }
__device__ __forceinline__ unsigned int xs_pad_c(unsigned int b) { return b + 4 * (b >> 5); }

struct __align__(16) XSel {
    unsigned long long hmass[XS_PBINS_M];     // histogram: 2^-32 fixed-point masses
    unsigned int hcnt[XS_PBINS_C];            //            and counts (bin b at xs_pad_*(b))
    unsigned int ckey[XS_CAND];               // candidates: relative keys
    unsigned long long ured[2][XS_WAVES];     // total / sink mass
    float fred[XS_WAVES];                     // score max
    unsigned int kred[2][XS_WAVES];           // selectable key min / max
    int cpk[XS_MAXNC][XS_WAVES];              // compaction: packed tie / sure counts per wave
    int ncand;
    unsigned int prefix, bin, bin_cnt;        // digit search: rel >> shift of the chosen bin
    int cnt_above;                            // keys / mass strictly above the chosen bin
    unsigned long long mass_above;
    unsigned int f_key;                       // candidate finish: tau's relative key,
    int f_cab, f_ceq;                         // the keys above it, its tie count,
    unsigned long long f_mab;                 // the mass above it
};

// V consecutive floats of src from page p: one vector load when the run is whole and
// `vec` (16-byte aligned base, stride a multiple of 4 floats), else guarded scalar loads.
template <int V>
__device__ __forceinline__ void ld_pages(const float* __restrict__ src, int p, int n, bool vec,
                                         float fill, float* o) {
    if (vec && p + V <= n) {
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
__device__ __forceinline__ void st_pages(float* __restrict__ dst, int p, int n, bool vec,
                                         const float* v) {
    if (vec && p + V <= n) {
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

// The nrm combine of NP_PAGES pages of one unit (workgroup (chunk, kv-head, request)):
// score[p] = sum_{g ascending} exp(score_h[g][p] - hmax_g), hmax_g = the maximum of the
// unit's per-tile maxima (the same maxima and sums as the fused staging).  The score_h
// loads are issued before the maxima are read and reduced.
__global__ __launch_bounds__(NP_THREADS) void nrm_pass_kernel(const amass_select_args a) {
    constexpr int TPT = (SEL_MAXP / XS_TILE) / NP_THREADS;   // tile maxima per thread
    __shared__ float red[8][NP_THREADS / WAVE];
    const int chunk = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
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

// The histogram search from the highest bin down: the bin where the cumulative weight
// (mass in coverage mode, else count) from the top, after what earlier digits put above,
// reaches `target`.  Wave 0 alone: lane i sums the 32 bins of group 63 - i (bins
// XS_BINS-1-32i down, 16-byte loads), one wave scan finds the group and a second one, over
// its 32 bins, the bin; the finding lane appends the bin to the prefix (digit bits
// [shift, top)) and adds the weight above it to the running total.  One barrier.
__device__ void xs_find(XSel& s, bool by_mass, unsigned long long target, int shift, int top) {
    if (threadIdx.x < WAVE) {
        const int lane = threadIdx.x;
        const int g = WAVE - 1 - lane;                      // bins 32 g .. 32 g + 31
        unsigned long long sum = 0;
        if (by_mass) {
            const ulonglong2* h = reinterpret_cast<const ulonglong2*>(s.hmass + 34 * g);
            ulonglong2 x[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) x[j] = h[j];
#pragma unroll
            for (int j = 0; j < 16; ++j) sum += x[j].x + x[j].y;
        } else {
            const uint4* h = reinterpret_cast<const uint4*>(s.hcnt + 36 * g);
            uint4 x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = h[j];
            unsigned int c = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) c += (x[j].x + x[j].y) + (x[j].z + x[j].w);
            sum = c;
        }
        const unsigned long long above0 =
            by_mass ? s.mass_above : (unsigned long long)s.cnt_above;
        const unsigned long long incl = wave_incl_scan_u64(sum);
        const unsigned long long hit = __ballot(above0 + incl >= target);
        const int L = hit ? __ffsll((long long)hit) - 1 : WAVE - 1;
        const unsigned long long base = above0 + readlane_u64(incl - sum, L);
        const int hL = XS_BINS - 1 - 32 * L;                // group L's highest bin
        const int gl = WAVE - 1 - L, bl = 31 - lane;         // its bins from the top
        const unsigned long long m =
            lane < 32 ? (by_mass ? s.hmass[34 * gl + bl] : (unsigned long long)s.hcnt[36 * gl + bl])
                      : 0ull;
        const unsigned long long incl2 = wave_incl_scan_u64(m);
        const unsigned long long hit2 = __ballot(lane < 32 && base + incl2 >= target);
        const int j = hit2 ? __ffsll((long long)hit2) - 1 : 31;
        if (lane == j) {
            const unsigned int bin = (unsigned int)(hL - j);
            const unsigned long long wabove = base + incl2 - m;
            s.bin = bin;
            s.bin_cnt = by_mass ? 0u : (unsigned int)m;
            if (by_mass) s.mass_above = wabove;
            else s.cnt_above = (int)wabove;
            s.prefix = (s.prefix << (top - shift)) | bin;
        }
    }
    __syncthreads();
}

template <int NT, int PPT, bool NRM>
__global__ __launch_bounds__(NT) void select_kernel(const amass_select_args a) {
    constexpr int NW = NT / WAVE;
    constexpr int V = PPT < 4 ? PPT : 4;        // pages per run
    constexpr int NC = PPT / V;                 // runs (chunks) per thread
    constexpr int CSTEP = V * NT;               // pages per chunk
    __shared__ XSel s;
    const int kh = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int MP = a.max_pages;
    float* gscore = a.score + (int64_t)r * a.sc_sr + (int64_t)kh * a.sc_sh;
    auto page_of = [&](int c, int i) { return c * CSTEP + V * tid + i; };

    // ---- stage: loads first (the row's MP pages), then the unit's geometry ---------------
    float v[PPT];
    float hv[NRM ? 8 : 1][NRM ? PPT : 1];
    float m[8];
    if constexpr (NRM) {
        const float* sh = a.score_h + (int64_t)r * a.sh_sr + (int64_t)kh * a.sh_sh;
        const bool vec = ((((uintptr_t)sh) | ((uintptr_t)gscore)) & 15) == 0 &&
                         (a.sh_sg & 3) == 0;
#pragma unroll
        for (int g = 0; g < 8; ++g)
            if (g < a.G) {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    ld_pages<V>(sh + g * a.sh_sg, page_of(c, 0), MP, vec, -INFINITY,
                                &hv[g][c * V]);
            }
    } else {
        const bool vec = (((uintptr_t)gscore) & 15) == 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) ld_pages<V>(gscore, page_of(c, 0), MP, vec, 0.f, &v[c * V]);
    }
    // fused: every wave loads all of the row's tile maxima (lane l: tiles l + 64 i, in
    // bounds: tiles < ceil(MP / 16) <= PPT NT / 16) and reduces them itself, masked below,
    // so the per-head maxima need no exchange between the waves
    constexpr int TL = NRM ? (PPT * NT / XS_TILE + WAVE - 1) / WAVE : 1;
    float tv[NRM ? 8 : 1][TL];
    if constexpr (NRM) {
        const float* tm = a.tile_max + (int64_t)r * a.tm_sr + (int64_t)kh * a.tm_sh;
        const int ntm = (MP + XS_TILE - 1) / XS_TILE;
#pragma unroll
        for (int g = 0; g < 8; ++g)
#pragma unroll
            for (int i = 0; i < TL; ++i) {
                const int t = lane + WAVE * i;
                tv[g][i] = (g < a.G && t < ntm) ? tm[g * a.tm_sg + t] : -INFINITY;
            }
    }
    const int np = min(a.n_pages[r], MP);       // a row never exceeds its table width
    const int nsh = min(a.n_sel_hi[r], np);
    const int bfix = a.mode == 0 ? a.b_fix[r] : 0;
    const int sink = a.sink_pages;
    const int nsc = nsh > 0 ? nsh : 0;          // scored pages [0, nsc)
    const int S = nsh - sink;
    const bool keep_all = S <= 1;
    const int lo = sink, hi = nsh;              // selectable [lo, hi) when !keep_all
    int32_t* tab = a.page_table + (int64_t)r * a.pt_sr + (int64_t)kh * a.pt_sh;

    for (int i = tid; i < XS_PBINS_C; i += NT) {
        s.hcnt[i] = 0;
        if (i < XS_PBINS_M) s.hmass[i] = 0;
    }
    if (tid == 0) {
        s.prefix = 0;
        s.bin = 0;
        s.bin_cnt = 0;
        s.cnt_above = 0;
        s.mass_above = 0;
        s.ncand = 0;
    }
    if constexpr (NRM) {
        const int nt = (nsc + XS_TILE - 1) / XS_TILE;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            float x = -INFINITY;
#pragma unroll
            for (int i = 0; i < TL; ++i)
                if (lane + WAVE * i < nt) x = fmaxf(x, tv[g][i]);
            m[g] = g < a.G ? wave_maxf_uniform(x) : -INFINITY;
        }
        const bool vec = (((uintptr_t)gscore) & 15) == 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int i = 0; i < V; ++i) {
                float acc = 0.f;
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    if (g < a.G) acc += nrm_exp(hv[g][c * V + i] - m[g]);
                v[c * V + i] = acc;
            }
            st_pages<V>(gscore, page_of(c, 0), nsc, vec, &v[c * V]);
        }
    }

    // ---- order keys, the score max and the selectable key range --------------------------
    // From here on every thread holds its pages' order keys (u2f gives the score back).
    uint32_t key[PPT];
    {
        float pmax = -INFINITY;
        unsigned int kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int p = page_of(k / V, k % V);
            key[k] = f2u(v[k]);
            if (p < nsc) {
                pmax = fmaxf(pmax, v[k]);
                if (p >= lo && p < hi) {
                    kmin = min(kmin, key[k]);
                    kmax = max(kmax, key[k]);
                }
            }
        }
        pmax = wave_maxf_uniform(pmax);
        kmin = wave_minu_uniform(kmin);
        kmax = wave_maxu_uniform(kmax);
        if (lane == 0) { s.fred[wv] = pmax; s.kred[0][wv] = kmin; s.kred[1][wv] = kmax; }
    }
    __syncthreads();
    float bmax = s.fred[0];
    unsigned int kmin = s.kred[0][0], kmax = s.kred[1][0];
#pragma unroll
    for (int i = 1; i < NW; ++i) {
        bmax = fmaxf(bmax, s.fred[i]);
        kmin = min(kmin, s.kred[0][i]);
        kmax = max(kmax, s.kred[1][i]);
    }

    // digits are taken of rel = key - kmin (order-preserving on [lo, hi)) from its
    // highest set bit down, so the first histogram already spreads the unit over the bins
    const unsigned int range = kmax - kmin;
    const int nb = range ? 32 - __clz(range) : 1;

    bool coverage = a.mode == 1;
    int b = 0;
    unsigned long long need = 0;
    const float smax = coverage ? (a.score_kind == 0 ? bmax : -INFINITY) : 0.f;
    unsigned int tau = 0;
    int take = 0;

    if (!coverage) b = bfix < 1 ? 1 : (bfix > S ? S : bfix);
    if (!keep_all) {
        const int shift = nb > XS_BITS ? nb - XS_BITS : 0;
        // ---- first digit's histogram (and, in coverage mode, the total / sink mass) ----
        // (top-b builds the count histogram; coverage its mass histogram and totals)
        {
            unsigned long long tot = 0, snk = 0;
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                const int p = page_of(k / V, k % V);
                if (p < nsc) {
                    const bool sel = p >= lo && p < hi;
                    if (coverage) {
                        const unsigned long long w = mass_q(u2f(key[k]), smax, a.score_kind);
                        tot += w;
                        if (p < sink) snk += w;
                        if (sel) atomicAdd(&s.hmass[xs_pad_m((key[k] - kmin) >> shift)], w);
                    } else if (sel && b != 1) {
                        atomicAdd(&s.hcnt[xs_pad_c((key[k] - kmin) >> shift)], 1u);
                    }
                }
            }
            if (coverage) {
                tot = wave_sum_u64_uniform(tot);
                snk = wave_sum_u64_uniform(snk);
                if (lane == 0) { s.ured[0][wv] = tot; s.ured[1][wv] = snk; }
            }
        }
        __syncthreads();
        if (coverage) {
            unsigned long long tot = 0, snk = 0;
#pragma unroll
            for (int i = 0; i < NW; ++i) { tot += s.ured[0][i]; snk += s.ured[1][i]; }
            const double nd = ceil(a.coverage * (double)tot);
            const long long needs = (long long)nd - (long long)snk;
            if (needs <= 0) {          // sinks already cover: one selectable page
                coverage = false;
                b = 1;
            } else {
                need = (unsigned long long)needs;
            }
        }
    }
    if (!keep_all && !coverage && b == 1) {
        // one page: tau = the largest selectable key, its lowest-index tie (or, for the
        // threshold rule, all of them) -- no histogram needed
        tau = kmax;
        take = a.tie_mode == 1 ? 0x7FFFFFFF : 1;
    } else if (!keep_all) {
        int top = nb;
        int shift = top > XS_BITS ? top - XS_BITS : 0;

        // ---- digit search --------------------------------------------------------------
        // After each scan the chosen bin's keys are gathered (the first XS_CAND kept, all
        // counted); a bin of more keys takes the next 11 bits.  Top-b knows the bin's count
        // from its histogram and skips the gather of a large bin.
        for (;;) {
            xs_find(s, coverage, coverage ? need : (unsigned long long)b, shift, top);
            const bool gather = shift == 0 || coverage || s.bin_cnt <= XS_CAND;
            if (gather) {
                const unsigned int pre = s.prefix;
#pragma unroll
                for (int k = 0; k < PPT; ++k) {
                    const int p = page_of(k / V, k % V);
                    const unsigned int rel = key[k] - kmin;
                    const bool in = p >= lo && p < hi && (rel >> shift) == pre;
                    const unsigned long long bal = __ballot(in);
                    if (bal) {
                        int base = 0;
                        if (lane == 0) base = atomicAdd(&s.ncand, __popcll(bal));
                        base = __builtin_amdgcn_readlane(base, 0);
                        if (in) {
                            const int idx = base + lanes_below(bal);
                            if (idx < XS_CAND) s.ckey[idx] = rel;
                        }
                    }
                }
                __syncthreads();
                if (shift == 0 || s.ncand <= XS_CAND) break;
            }
            // the next 11 bits of the keys inside the chosen bin
            for (int i = tid; i < XS_PBINS_C; i += NT) {
                s.hcnt[i] = 0;
                if (i < XS_PBINS_M) s.hmass[i] = 0;
            }
            __syncthreads();
            if (tid == 0) s.ncand = 0;          // every thread read it before the barrier
            top = shift;
            shift = top > XS_BITS ? top - XS_BITS : 0;
            const unsigned int pre = s.prefix;
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                const int p = page_of(k / V, k % V);
                const unsigned int rel = key[k] - kmin;
                if (p >= lo && p < hi && (rel >> top) == pre) {
                    const unsigned int bin = (rel >> shift) & (XS_BINS - 1);
                    // an opaque copy keeps the compiler from computing every page's mass
                    // ahead of the digit loop (only pages of the chosen bin need one)
                    uint32_t kk = key[k];
                    asm volatile("" : "+v"(kk));
                    if (coverage)
                        atomicAdd(&s.hmass[xs_pad_m(bin)], mass_q(u2f(kk), smax, a.score_kind));
                    else atomicAdd(&s.hcnt[xs_pad_c(bin)], 1u);
                }
            }
            __syncthreads();
        }
        unsigned int tau_rel;
        int count_eq, cab;                      // cab: keys above tau (top-b only)
        unsigned long long mab;
        if (shift > 0) {
            // ---- the <= 64 candidates ranked exactly by wave 0 (register broadcasts) ------
            if (wv == 0) {
                const int c = min(s.ncand, XS_CAND);
                const unsigned int kt = lane < c ? s.ckey[lane] : 0u;
                // the candidates' masses (only they need one: computed here, not per page)
                const unsigned long long mt =
                    lane < c && coverage ? mass_q(u2f(kt + kmin), smax, a.score_kind) : 0ull;
                const uint32_t mlo = (uint32_t)mt, mhi = (uint32_t)(mt >> 32);
                unsigned int ab = 0, eq = 0;
                unsigned long long am = 0, em = 0;
                for (int j = 0; j < c; ++j) {
                    // readlane returns int: widen through uint32_t (no sign extension)
                    const unsigned int kj = (uint32_t)__builtin_amdgcn_readlane((int)kt, j);
                    const unsigned long long mj =
                        ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)mhi, j)
                         << 32) |
                        (unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)mlo, j);
                    ab += kj > kt;
                    eq += kj == kt;
                    am += kj > kt ? mj : 0ull;
                    em += kj == kt ? mj : 0ull;
                }
                // kt is tau iff the target falls inside its tie class (keys above < target
                // <= keys above + its ties), counted by mass or by count
                const unsigned long long above =
                    coverage ? s.mass_above + am : (unsigned long long)(s.cnt_above + (int)ab);
                const unsigned long long own = coverage ? em : (unsigned long long)eq;
                const unsigned long long target = coverage ? need : (unsigned long long)b;
                const bool win = lane < c && above < target && target <= above + own;
                const unsigned long long wb = __ballot(win);
                const int src = wb ? __ffsll((long long)wb) - 1 : 0;   // ties of kt agree
                const unsigned int fk = readlane_u(kt, src);
                const int feq = __builtin_amdgcn_readlane((int)eq, src);
                const int fab = __builtin_amdgcn_readlane((int)ab, src);
                const unsigned long long fam = readlane_u64(am, src);
                if (lane == 0) {
                    s.f_key = wb ? fk : s.prefix << shift;
                    s.f_cab = s.cnt_above + (wb ? fab : 0);
                    s.f_mab = s.mass_above + (wb ? fam : 0ull);
                    s.f_ceq = wb ? feq : 0;
                }
            }
            __syncthreads();
            tau_rel = s.f_key;
            count_eq = s.f_ceq;
            cab = s.f_cab;
            mab = s.f_mab;
        } else {
            tau_rel = s.prefix;                 // every bit resolved: one tie class
            count_eq = s.ncand;
            cab = s.cnt_above;
            mab = s.mass_above;
        }
        tau = tau_rel + kmin;
        if (coverage) {
            // ties needed: ceil(rem / wq) clamped to [1, count_eq], from a double estimate
            // (off by at most one below 2^15) corrected with exact 64-bit products
            const unsigned long long rem = need - mab;
            const unsigned long long wq = mass_q(u2f(tau), smax, a.score_kind);
            int t = count_eq;
            if (wq) {
                const double e = ceil((double)rem / (double)wq);
                t = e < (double)count_eq ? (int)e : count_eq;
                while (t > 1 && (unsigned long long)(t - 1) * wq >= rem) --t;
                while (t < count_eq && (unsigned long long)t * wq < rem) ++t;
            }
            take = count_eq >= 1 && t < 1 ? 1 : t;
        } else {
            take = b - cab;
        }
        if (a.tie_mode == 1) take = count_eq;
    }

    // ---- keep + ascending compaction --------------------------------------------------
    // A page is a sure keep (outside the selectable region, key > tau, or for the
    // threshold rule score >= tau) or a tie (key == tau, index rule); ties are kept in page
    // order while their rank is < take, so a kept page goes to position sure(<p) +
    // min(ties(<p), take).  Page order is (chunk, thread, slot): per chunk a wave scan of
    // the threads' packed (ties << 16 | sures) counts, one exchange of the waves' totals,
    // which every wave scans again.  Packed sums stay below 2^15 per field.
    const float ftau = u2f(tau);
    uint32_t sure_m = 0, tie_m = 0;              // bit k: page slot k
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        const int p = page_of(k / V, k % V);
        bool su = false, ti = false;
        if (p < np) {
            if (keep_all || p < lo || p >= hi) {
                su = true;
            } else if (a.tie_mode == 1) {
                su = u2f(key[k]) >= ftau;
            } else {
                su = key[k] > tau;
                ti = key[k] == tau;
            }
        }
        sure_m |= (uint32_t)su << k;
        tie_m |= (uint32_t)ti << k;
    }
    constexpr uint32_t VM = (1u << V) - 1u;
    int excl[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int own = __popc((sure_m >> (c * V)) & VM) + (__popc((tie_m >> (c * V)) & VM) << 16);
        const int incl = wave_incl_scan(own);
        excl[c] = incl - own;
        if (lane == WAVE - 1) s.cpk[c][wv] = incl;
    }
    __syncthreads();
    int before = 0;                              // packed counts of the pages before a chunk
    int base[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int wincl = wave_incl_scan(lane < NW ? s.cpk[c][lane] : 0);
        const int wprev = wv > 0 ? __builtin_amdgcn_readlane(wincl, wv > 0 ? wv - 1 : 0) : 0;
        base[c] = before + wprev + excl[c];
        before += __builtin_amdgcn_readlane(wincl, NW - 1);
    }
    const int cnt = (before & 0xFFFF) + min(before >> 16, take);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int sb = base[c] & 0xFFFF, tb = base[c] >> 16;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const bool su = (sure_m >> (c * V + i)) & 1u, ti = (tie_m >> (c * V + i)) & 1u;
            if (su || (ti && tb < take)) tab[sb + min(tb, take)] = page_of(c, i);
            sb += su;
            tb += ti;
        }
    }
    for (int p = cnt + tid; p < MP; p += NT) tab[p] = -1;
    if (tid == 0) {
        a.page_cnt[(int64_t)r * a.pc_sr + kh] = cnt;
        // selectable pages kept: every page outside [lo, hi) of the row is kept
        if (a.n_sel_out)
            a.n_sel_out[(int64_t)r * a.n_kv + kh] = keep_all ? (S > 0 ? S : 0) : cnt - (np - S);
    }
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
                hipLaunchKernelGGL(nrm_pass_kernel, dim3(chunks, k.n_kv, k.n_req),
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
