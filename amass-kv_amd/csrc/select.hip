// Stage-A selection for gfx950: derive params, nrm combine, top-b / coverage nucleus.
//
// One workgroup (512 threads, 8 waves) per (request, kv-head).  The unit's scores are
// staged once in LDS (fp32, up to MAXP pages), optionally produced there by the fused nrm
// combine.  The b-th largest score is found by a 4-pass MSD radix select over
// order-preserving uint32 keys (256-bin LDS histograms; in coverage mode each bin also
// accumulates the 2^-32 fixed-point page mass with 64-bit LDS atomics, so the cut is
// found by mass instead of by count).  Bin scans are wave-parallel prefix sums.  The
// final keep test and the ascending compaction are two chunked block scans in page order
// (the second also ranks ties at tau by page index).
//
// Semantics follow selection/select.py:60-101 (_topb_select_kernel): keep =
// (selectable & chosen) | p < sink | p >= n_sel_hi | (n_sel_hi - sink <= 1), compaction
// ascending with -1 padding, page_cnt.  tie_mode 0 keeps exactly b pages (ties at the
// b-th score -> lower page index); tie_mode 1 is the reference threshold rule score >= tau.
#include "common.h"

namespace amass {

constexpr int SEL_THREADS = 512;
constexpr int SEL_WAVES = SEL_THREADS / WAVE;
constexpr int SEL_MAXP = 16384;   // 64 KB of fp32 scores in LDS

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
__device__ __forceinline__ unsigned int wave_minu(unsigned int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, (unsigned int)__shfl_xor((int)v, o, WAVE));
    return v;
}
__device__ __forceinline__ unsigned int wave_maxu(unsigned int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, (unsigned int)__shfl_xor((int)v, o, WAVE));
    return v;
}
// number of set bits of `m` below this lane
__device__ __forceinline__ int lanes_below(unsigned long long m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// ------------------------------------------------------------------ nrm combine
// Per-head maxima m[0..G) of the block: wave reductions, one LDS exchange, one barrier.
__device__ __forceinline__ void head_max(float* m, int G, float (*red)[SEL_WAVES]) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int g = 0; g < 8; ++g)
        if (g < G) {
            const float x = wave_maxf(m[g]);
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
                        for (int i = 0; i < V; ++i) acc[i] += expf(v[k][g][i] - m[g]);
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
// A radix pass whose chosen bin holds <= SEL_CAND keys ends the radix search: those keys
// are gathered and ranked against each other exactly (all pairs), which replaces the
// remaining passes.
constexpr int SEL_CAND = 256;

struct __align__(16) SelShared {
    unsigned int hcnt[2][256];           // double-buffered radix histograms
    unsigned long long hmass[2][256];
    unsigned int ckey[SEL_CAND];         // candidates: rel keys and masses
    unsigned long long cmass[SEL_CAND];
    int ncand;
    unsigned int f_prefix;               // candidate finish result
    int f_cab, f_ceq;
    unsigned long long f_mab;
    float hred[8][SEL_WAVES];            // nrm per-head maxima
    float fred[SEL_WAVES];               // score max
    unsigned int kred[2][SEL_WAVES];     // selectable key min / max
    unsigned long long ured[2][SEL_WAVES];  // total / sink mass
    int wred[2][SEL_WAVES];              // per-wave sure-keep / tie counts
    unsigned int prefix, bin;            // radix state (written by the scanning lane)
    int cnt_above;
    unsigned long long mass_above;
};

// Wave 0 scans the 256 bins of histogram `buf` from high to low and finds the bin holding
// the target.  Count mode: first bin where cnt_above + cumulative count >= target; mass
// mode likewise on mass.  The scanning lane appends the bin to the prefix (at `shift`) and
// adds the bins strictly above to the running totals.
__device__ void scan_bins(SelShared& s, int buf, bool by_mass, unsigned long long target,
                          int shift) {
    const int lane = threadIdx.x & 63;
    // lane L owns bins 255-4L .. 252-4L (descending)
    unsigned long long v[4];
    unsigned int c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int bin = 255 - 4 * lane - i;
        c[i] = s.hcnt[buf][bin];
        v[i] = by_mass ? s.hmass[buf][bin] : (unsigned long long)c[i];
    }
    unsigned long long own = v[0] + v[1] + v[2] + v[3];
    unsigned int ownc = c[0] + c[1] + c[2] + c[3];
    unsigned long long incl = own;
    unsigned int inclc = ownc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(incl, o, WAVE);
        const unsigned int yc = __shfl_up(inclc, o, WAVE);
        if (lane >= o) { incl += y; inclc += yc; }
    }
    const unsigned long long excl = incl - own;
    const unsigned int exclc = inclc - ownc;
    const unsigned long long base = by_mass ? s.mass_above : (unsigned long long)s.cnt_above;
    // first lane whose inclusive sum reaches the target
    const bool hit = base + incl >= target;
    const unsigned long long bal = __ballot(hit);
    const int L = bal ? (__ffsll((long long)bal) - 1) : 63;
    if (lane == L) {
        unsigned long long cum = base + excl;
        unsigned long long mab = s.mass_above + (by_mass ? excl : 0ull);
        unsigned int cab = (unsigned int)s.cnt_above + exclc;
        int pick = 3;
        for (int i = 0; i < 4; ++i) {
            if (cum + v[i] >= target || i == 3) { pick = i; break; }
            cum += v[i];
            cab += c[i];
            mab += by_mass ? v[i] : 0ull;
        }
        // mass of bins above in count mode is not tracked (not needed)
        const unsigned int bin = (unsigned int)(255 - 4 * L - pick);
        s.bin = bin;
        s.prefix |= bin << shift;
        s.cnt_above = (int)cab;
        s.mass_above = mab;
    }
}

// sc[p4..p4+4) from LDS in one 128-bit read (p4 % 4 == 0; the LDS array is padded to a
// multiple of 4 floats)
__device__ __forceinline__ void ld4(const float* sc, int p4, float* v) {
    const float4 x = *reinterpret_cast<const float4*>(sc + p4);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
}

struct SelTrack {
    int lo, hi;
    float pmax;
    unsigned int kmin, kmax;
    __device__ void operator()(int p, float v) {
        pmax = fmaxf(pmax, v);
        if (p >= lo && p < hi) {
            const unsigned int k = f2u(v);
            kmin = min(kmin, k);
            kmax = max(kmax, k);
        }
    }
};

__global__ __launch_bounds__(SEL_THREADS) void select_kernel(const amass_select_args a) {
    extern __shared__ __align__(16) float sc[];   // scores of this unit, [round4(max_pages)]
    __shared__ SelShared s;
    const int kh = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int MP = a.max_pages;
    const int np = min(a.n_pages[r], MP);       // a row never exceeds its table width
    const int nsh = min(a.n_sel_hi[r], np);
    const int bfix = a.mode == 0 ? a.b_fix[r] : 0;
    const int sink = a.sink_pages;
    int32_t* tab = a.page_table + (int64_t)r * a.pt_sr + (int64_t)kh * a.pt_sh;
    float* gscore = a.score + (int64_t)r * a.sc_sr + (int64_t)kh * a.sc_sh;
    const int nsc = nsh > 0 ? nsh : 0;          // scored pages [0, nsc)

    const int S = nsh - sink;
    const bool keep_all = S <= 1;
    const int lo = sink, hi = nsh;        // selectable [lo, hi) when !keep_all

    for (int i = tid; i < 2 * 256; i += SEL_THREADS) {
        (&s.hcnt[0][0])[i] = 0;
        (&s.hmass[0][0])[i] = 0;
    }
    if (tid == 0) { s.prefix = 0; s.cnt_above = 0; s.mass_above = 0; s.ncand = 0; }

    // ---- stage scores in LDS; track the score max and the selectable key range ---------
    SelTrack tr{lo, hi, -INFINITY, 0xFFFFFFFFu, 0u};
    if (a.score_h != nullptr) {
        const float* sh = a.score_h + (int64_t)r * a.sh_sr + (int64_t)kh * a.sh_sh;
        nrm_stage(sh, a.sh_sg, a.G, nsc, sc, gscore, s.hred, tr);
    } else if ((((uintptr_t)gscore) & 15) == 0) {
        copy_run<4, 2>(gscore, nsc, sc, tr);
    } else {
        copy_run<1, 4>(gscore, nsc, sc, tr);
    }
    {
        const float m = wave_maxf(tr.pmax);
        const unsigned int k0 = wave_minu(tr.kmin), k1 = wave_maxu(tr.kmax);
        if (lane == 0) { s.fred[wv] = m; s.kred[0][wv] = k0; s.kred[1][wv] = k1; }
    }
    __syncthreads();
    float bmax = s.fred[0];
    unsigned int kmin = s.kred[0][0], kmax = s.kred[1][0];
#pragma unroll
    for (int i = 1; i < SEL_WAVES; ++i) {
        bmax = fmaxf(bmax, s.fred[i]);
        kmin = min(kmin, s.kred[0][i]);
        kmax = max(kmax, s.kred[1][i]);
    }

    // Radix digits are taken of rel = key - kmin (order-preserving on [lo, hi)), from its
    // highest set bit down, so the first pass already spreads the unit over the bins.
    const unsigned int range = kmax - kmin;
    const int nb = range ? 32 - __clz(range) : 1;
    const int passes = (nb + 7) >> 3;

    bool coverage = a.mode == 1;
    int b = 0;
    unsigned long long need = 0;
    const float smax = coverage ? (a.score_kind == 0 ? bmax : -INFINITY) : 0.f;
    unsigned int tau = 0;
    int take = 0;

    if (!keep_all) {
        // ---- pass-0 histogram (and, in coverage mode, the total / sink mass) ------------
        const int sh0 = nb > 8 ? nb - 8 : 0;
        if (coverage) {
            unsigned long long tot = 0, snk = 0;
            for (int p4 = 4 * tid; p4 < nsc; p4 += 4 * SEL_THREADS) {
                float v[4];
                ld4(sc, p4, v);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int p = p4 + j;
                    if (p < nsc) {
                        const unsigned long long w = mass_q(v[j], smax, a.score_kind);
                        tot += w;
                        if (p < sink) snk += w;
                        if (p >= lo && p < hi) {
                            const unsigned int bin = ((f2u(v[j]) - kmin) >> sh0) & 255u;
                            atomicAdd(&s.hcnt[0][bin], 1u);
                            atomicAdd(&s.hmass[0][bin], w);
                        }
                    }
                }
            }
            tot = wave_sum_u64(tot);
            snk = wave_sum_u64(snk);
            if (lane == 0) { s.ured[0][wv] = tot; s.ured[1][wv] = snk; }
        } else {
            for (int p4 = (lo & ~3) + 4 * tid; p4 < hi; p4 += 4 * SEL_THREADS) {
                float v[4];
                ld4(sc, p4, v);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int p = p4 + j;
                    if (p >= lo && p < hi)
                        atomicAdd(&s.hcnt[0][((f2u(v[j]) - kmin) >> sh0) & 255u], 1u);
                }
            }
        }
        __syncthreads();
        if (coverage) {
            unsigned long long tot = 0, snk = 0;
#pragma unroll
            for (int i = 0; i < SEL_WAVES; ++i) { tot += s.ured[0][i]; snk += s.ured[1][i]; }
            const double nd = ceil(a.coverage * (double)tot);
            const long long needs = (long long)nd - (long long)snk;
            if (needs <= 0) {          // sinks already cover: one selectable page
                coverage = false;
                b = 1;
            } else {
                need = (unsigned long long)needs;
            }
        } else {
            b = bfix < 1 ? 1 : (bfix > S ? S : bfix);
        }

        // ---- radix select of tau: scan, then the next digit's histogram ----------------
        int fshift = -1;                // >= 0: finish by candidates below this bit
        for (int pass = 0; pass < passes; ++pass) {
            const int top = nb - 8 * pass;             // digit = rel bits [shift, top)
            const int shift = top > 8 ? top - 8 : 0;
            const int buf = pass & 1;
            if (pass > 0) {
                const unsigned int pre = s.prefix;
                const unsigned int pm = 0xFFFFFFFFu << top;   // top < 32 after pass 0
                for (int p4 = (lo & ~3) + 4 * tid; p4 < hi; p4 += 4 * SEL_THREADS) {
                    float v[4];
                    ld4(sc, p4, v);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int p = p4 + j;
                        const unsigned int rel = f2u(v[j]) - kmin;
                        if (p >= lo && p < hi && (rel & pm) == pre) {
                            const unsigned int bin = (rel >> shift) & 255u;
                            atomicAdd(&s.hcnt[buf][bin], 1u);
                            if (coverage)
                                atomicAdd(&s.hmass[buf][bin], mass_q(v[j], smax, a.score_kind));
                        }
                    }
                }
                __syncthreads();
            }
            if (tid < WAVE) {
                scan_bins(s, buf, coverage, coverage ? need : (unsigned long long)b, shift);
            } else if (pass + 1 < passes && pass > 0) {
                for (int i = tid - WAVE; i < 256; i += SEL_THREADS - WAVE) {
                    s.hcnt[buf ^ 1][i] = 0;
                    s.hmass[buf ^ 1][i] = 0;
                }
            }
            __syncthreads();
            if (pass + 1 < passes && (int)s.hcnt[buf][s.bin] <= SEL_CAND) {
                fshift = shift;
                break;
            }
        }
        unsigned int tau_rel;
        int count_eq, cab;
        unsigned long long mab;
        if (fshift >= 0) {
            // ---- candidate finish: the keys of the chosen bin, ranked all-pairs ----------
            const unsigned int pre = s.prefix;
            const unsigned int pm = 0xFFFFFFFFu << fshift;
            if (tid == 0) {            // defaults (replaced by the winner below)
                s.f_prefix = pre;
                s.f_cab = s.cnt_above;
                s.f_mab = s.mass_above;
                s.f_ceq = 0;
            }
            for (int p4 = (lo & ~3) + 4 * tid; p4 < hi; p4 += 4 * SEL_THREADS) {
                float v[4];
                ld4(sc, p4, v);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int p = p4 + j;
                    const unsigned int rel = f2u(v[j]) - kmin;
                    const bool in = p >= lo && p < hi && (rel & pm) == pre;
                    const unsigned long long bal = __ballot(in);
                    if (bal) {
                        int base = 0;
                        if (lane == 0) base = atomicAdd(&s.ncand, __popcll(bal));
                        base = __shfl(base, 0, WAVE);
                        if (in) {
                            const int idx = base + lanes_below(bal);
                            s.ckey[idx] = rel;
                            s.cmass[idx] = coverage ? mass_q(v[j], smax, a.score_kind) : 0ull;
                        }
                    }
                }
            }
            __syncthreads();
            const int c = s.ncand;
            if (tid < c) {
                const unsigned int kt = s.ckey[tid];
                unsigned int ab = 0, eq = 0;
                unsigned long long am = 0, em = 0;
                int j = 0;
                for (; j + 4 <= c; j += 4) {
                    const uint4 k4 = *reinterpret_cast<const uint4*>(&s.ckey[j]);
                    const ulonglong2 m0 = *reinterpret_cast<const ulonglong2*>(&s.cmass[j]);
                    const ulonglong2 m1 = *reinterpret_cast<const ulonglong2*>(&s.cmass[j + 2]);
                    const unsigned int kk[4] = {k4.x, k4.y, k4.z, k4.w};
                    const unsigned long long mm[4] = {m0.x, m0.y, m1.x, m1.y};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        ab += kk[i] > kt;
                        eq += kk[i] == kt;
                        am += kk[i] > kt ? mm[i] : 0ull;
                        em += kk[i] == kt ? mm[i] : 0ull;
                    }
                }
                for (; j < c; ++j) {
                    const unsigned int kj = s.ckey[j];
                    const unsigned long long mj = s.cmass[j];
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
                if (above < target && target <= above + own) {   // all ties of kt agree
                    s.f_prefix = kt;
                    s.f_cab = s.cnt_above + (int)ab;
                    s.f_mab = s.mass_above + am;
                    s.f_ceq = (int)eq;
                }
            }
            __syncthreads();
            tau_rel = s.f_prefix;
            count_eq = s.f_ceq;
            cab = s.f_cab;
            mab = s.f_mab;
        } else {
            tau_rel = s.prefix;
            count_eq = (int)s.hcnt[(passes - 1) & 1][s.bin];
            cab = s.cnt_above;
            mab = s.mass_above;
        }
        tau = tau_rel + kmin;
        if (coverage) {
            const unsigned long long rem = need - mab;
            const unsigned long long wq = mass_q(u2f(tau), smax, a.score_kind);
            long long t = wq ? (long long)((rem + wq - 1) / wq) : (long long)count_eq;
            if (t < 1) t = 1;
            if (t > count_eq) t = count_eq;
            take = (int)t;
            b = cab + take;
        } else {
            take = b - cab;
        }
        if (a.tie_mode == 1) take = count_eq;
    }

    // ---- keep + ascending compaction --------------------------------------------------
    // A page is a sure keep (outside the selectable region, key > tau, or for the
    // threshold rule score >= tau) or a tie (key == tau, index rule); ties are kept in page
    // order while their rank is < take, so pages kept before p = sure(<p) + min(ties(<p),
    // take).  Wave w owns a run of 256-page blocks; lane l takes pages 4l..4l+3 of a block,
    // and ballots per slot j give each lane the counts of the lanes below it.
    const int n = np > 0 ? np : 0;
    const int per = (((n + SEL_WAVES - 1) / SEL_WAVES) + 255) & ~255;
    const int w0 = wv * per, w1 = min(n, w0 + per);
    const float ftau = u2f(tau);
    auto classify = [&](int p4, bool* sure, bool* tie) {
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (p4 < w1) ld4(sc, p4, v);           // w1 <= n <= max_pages: inside the array
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int p = p4 + j;
            sure[j] = false;
            tie[j] = false;
            if (p >= w1) continue;
            if (keep_all || p < lo || p >= hi) {
                sure[j] = true;
            } else if (a.tie_mode == 1) {
                sure[j] = v[j] >= ftau;
            } else {
                const unsigned int k = f2u(v[j]);
                sure[j] = k > tau;
                tie[j] = k == tau;
            }
        }
    };
    int sure_c = 0, tie_c = 0;
    for (int b0 = w0; b0 < w1; b0 += 4 * WAVE) {
        bool sure[4], tie[4];
        classify(b0 + 4 * lane, sure, tie);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sure_c += __popcll(__ballot(sure[j]));
            tie_c += __popcll(__ballot(tie[j]));
        }
    }
    if (lane == 0) { s.wred[0][wv] = sure_c; s.wred[1][wv] = tie_c; }
    __syncthreads();
    int sure_base = 0, tie_base = 0, sure_tot = 0, tie_tot = 0;
#pragma unroll
    for (int i = 0; i < SEL_WAVES; ++i) {
        const int x = s.wred[0][i], t = s.wred[1][i];
        if (i < wv) { sure_base += x; tie_base += t; }
        sure_tot += x;
        tie_tot += t;
    }
    const int cnt = sure_tot + min(tie_tot, take);
    int kp = sure_base + min(tie_base, take);
    int rt = tie_base;
    for (int b0 = w0; b0 < w1; b0 += 4 * WAVE) {
        bool sure[4], tie[4], keep[4];
        const int p4 = b0 + 4 * lane;
        classify(p4, sure, tie);
        int rk = rt, t_all = 0;                  // tie rank of this lane's next tie
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned long long bt = __ballot(tie[j]);
            rk += lanes_below(bt);
            t_all += __popcll(bt);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {            // lane-local ties in slot order
            keep[j] = sure[j] || (tie[j] && rk < take);
            rk += tie[j];
        }
        int pos = kp, k_all = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned long long bk = __ballot(keep[j]);
            pos += lanes_below(bk);
            k_all += __popcll(bk);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (keep[j]) tab[pos++] = p4 + j;
        rt += t_all;
        kp += k_all;
    }
    for (int p = cnt + tid; p < MP; p += SEL_THREADS) tab[p] = -1;
    if (tid == 0) {
        a.page_cnt[(int64_t)r * a.pc_sr + kh] = cnt;
        if (a.n_sel_out)
            a.n_sel_out[(int64_t)r * a.n_kv + kh] =
                keep_all ? (S > 0 ? S : 0) : (a.tie_mode == 1 ? cnt - (n - S) : b);
    }
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
    if (a->max_pages > SEL_MAXP) return AMASS_ERR_CAPACITY;
    if (a->tie_mode != 0 && a->tie_mode != 1) return AMASS_ERR_GEOMETRY;
    if (a->score_kind != 0 && a->score_kind != 1) return AMASS_ERR_GEOMETRY;
    if (mode == 1 && !(a->coverage > 0.0 && a->coverage <= 1.0)) return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    amass_select_args k = *a;
    k.mode = mode;
    const size_t lds = (size_t)((a->max_pages + 3) & ~3) * sizeof(float);
    hipLaunchKernelGGL(select_kernel, dim3(a->n_kv, a->n_req), dim3(SEL_THREADS), lds,
                       (hipStream_t)stream, k);
    return check_launch();
}

extern "C" int amass_topb_select(const amass_select_args* a, void* stream) {
    return select_common(a, 0, stream);
}
extern "C" int amass_coverage_select(const amass_select_args* a, void* stream) {
    return select_common(a, 1, stream);
}
