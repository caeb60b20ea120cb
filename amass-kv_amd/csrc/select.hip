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

// ------------------------------------------------------------------ block helpers
__device__ __forceinline__ float block_maxf(float v, float* red) {
    v = wave_maxf(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < SEL_WAVES; ++i) r = fmaxf(r, red[i]);
    return r;
}
__device__ __forceinline__ unsigned long long block_sum_u64(unsigned long long v,
                                                            unsigned long long* red) {
    v = wave_sum_u64(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    unsigned long long r = 0;
#pragma unroll
    for (int i = 0; i < SEL_WAVES; ++i) r += red[i];
    return r;
}
// exclusive prefix over threads of a per-thread count; returns the total in `total`
__device__ __forceinline__ int block_excl_scan(int v, int* red, int& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, WAVE);
        if (lane >= o) x += y;
    }
    __syncthreads();
    if (lane == 63) red[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < SEL_WAVES; ++i) {
        const int t = red[i];
        if (i < w) base += t;
        tot += t;
    }
    total = tot;
    return base + x - v;
}

// nrm combine of one (request, kv-head) into LDS (and global `score`)
__device__ void nrm_into(const float* __restrict__ sh, int64_t sh_sg, int G, int nsh,
                         float* sc, float* gscore, float* red, float* hmax_s) {
    for (int g = 0; g < G; ++g) {
        float m = -INFINITY;
        for (int p = threadIdx.x; p < nsh; p += blockDim.x) m = fmaxf(m, sh[g * sh_sg + p]);
        m = block_maxf(m, red);
        if (threadIdx.x == 0) hmax_s[g] = m;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < nsh; p += blockDim.x) {
        float acc = 0.f;
        for (int g = 0; g < G; ++g) acc += expf(sh[g * sh_sg + p] - hmax_s[g]);
        sc[p] = acc;
        if (gscore) gscore[p] = acc;
    }
    __syncthreads();
}

// ------------------------------------------------------------------ nrm standalone
__global__ __launch_bounds__(SEL_THREADS) void nrm_kernel(const amass_nrm_args a) {
    __shared__ float red[SEL_WAVES];
    __shared__ float hmax_s[8];
    const int kh = blockIdx.x, r = blockIdx.y;
    const int nsh = a.n_sel_hi[r];
    if (nsh <= 0) return;
    const float* sh = a.score_h + (int64_t)r * a.sh_sr + (int64_t)kh * a.sh_sh;
    float* out = a.score + (int64_t)r * a.sc_sr + (int64_t)kh * a.sc_sh;
    for (int g = 0; g < a.G; ++g) {
        float m = -INFINITY;
        for (int p = threadIdx.x; p < nsh; p += blockDim.x) m = fmaxf(m, sh[g * a.sh_sg + p]);
        m = block_maxf(m, red);
        if (threadIdx.x == 0) hmax_s[g] = m;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < nsh; p += blockDim.x) {
        float acc = 0.f;
        for (int g = 0; g < a.G; ++g) acc += expf(sh[g * a.sh_sg + p] - hmax_s[g]);
        out[p] = acc;
    }
}

// ------------------------------------------------------------------ selection
struct SelShared {
    unsigned int hcnt[256];
    unsigned long long hmass[256];
    int ired[SEL_WAVES];
    float fred[SEL_WAVES];
    unsigned long long ured[SEL_WAVES];
    float hmax[8];
    // radix state broadcast
    unsigned int prefix, pmask, bin;
    int cnt_above;
    unsigned long long mass_above;
};

// Wave 0 scans the 256 bins from high to low and finds the bin holding the target.
// Count mode: first bin where cnt_above + cum_count >= target.  Mass mode likewise on
// mass.  Updates the running above-totals with the bins strictly above.
__device__ void scan_bins(SelShared& s, bool by_mass, unsigned long long target) {
    const int lane = threadIdx.x & 63;
    // lane L owns bins 255-4L .. 252-4L (descending)
    unsigned long long v[4];
    unsigned int c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int bin = 255 - 4 * lane - i;
        c[i] = s.hcnt[bin];
        v[i] = by_mass ? s.hmass[bin] : (unsigned long long)c[i];
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
    int L = bal ? (__ffsll((long long)bal) - 1) : 63;
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
        s.bin = (unsigned int)(255 - 4 * L - pick);
        s.cnt_above = (int)cab;
        s.mass_above = mab;
    }
}

__global__ __launch_bounds__(SEL_THREADS) void select_kernel(const amass_select_args a) {
    extern __shared__ float sc[];      // [max(nsh,0)] scores of this unit
    __shared__ SelShared s;
    const int kh = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x;
    const int MPc = a.max_pages;
    const int np = min(a.n_pages[r], MPc);      // a row never exceeds its table width
    const int nsh = min(a.n_sel_hi[r], np);
    const int sink = a.sink_pages;
    const int MP = a.max_pages;
    int32_t* tab = a.page_table + (int64_t)r * a.pt_sr + (int64_t)kh * a.pt_sh;
    float* gscore = a.score + (int64_t)r * a.sc_sr + (int64_t)kh * a.sc_sh;
    const int nsc = nsh < np ? (nsh > 0 ? nsh : 0) : np;   // scored pages [0, nsc)

    // ---- stage scores -------------------------------------------------------------
    if (a.score_h != nullptr) {
        const float* sh = a.score_h + (int64_t)r * a.sh_sr + (int64_t)kh * a.sh_sh;
        nrm_into(sh, a.sh_sg, a.G, nsc, sc, gscore, s.fred, s.hmax);
    } else {
        for (int p = tid; p < nsc; p += SEL_THREADS) sc[p] = gscore[p];
        __syncthreads();
    }

    const int S = nsh - sink;
    const bool keep_all = S <= 1;
    const int lo = sink, hi = nsh;        // selectable [lo, hi) when !keep_all
    bool coverage = a.mode == 1;
    int b = 0;
    unsigned long long need = 0;
    float smax = 0.f;

    if (!keep_all && np > 0) {
        if (coverage) {
            float m = -INFINITY;
            if (a.score_kind == 0)
                for (int p = tid; p < nsc; p += SEL_THREADS) m = fmaxf(m, sc[p]);
            smax = block_maxf(m, s.fred);
            unsigned long long tot = 0, snk = 0;
            for (int p = tid; p < nsc; p += SEL_THREADS) {
                const unsigned long long w = mass_q(sc[p], smax, a.score_kind);
                tot += w;
                if (p < sink) snk += w;
            }
            tot = block_sum_u64(tot, s.ured);
            snk = block_sum_u64(snk, s.ured);
            const double nd = ceil(a.coverage * (double)tot);
            const long long needs = (long long)nd - (long long)snk;
            if (needs <= 0) {          // sinks already cover: one selectable page
                coverage = false;
                b = 1;
            } else {
                need = (unsigned long long)needs;
            }
        } else {
            b = a.b_fix[r];
            b = b < 1 ? 1 : (b > S ? S : b);
        }
    }

    // ---- radix select of tau --------------------------------------------------------
    unsigned int tau = 0;
    int take = 0;
    if (!keep_all && np > 0) {
        if (tid == 0) { s.prefix = 0; s.pmask = 0; s.cnt_above = 0; s.mass_above = 0; }
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;
            for (int i = tid; i < 256; i += SEL_THREADS) { s.hcnt[i] = 0; s.hmass[i] = 0; }
            __syncthreads();
            const unsigned int pre = s.prefix, pm = s.pmask;
            for (int p = lo + tid; p < hi; p += SEL_THREADS) {
                const unsigned int k = f2u(sc[p]);
                if ((k & pm) == pre) {
                    const unsigned int bin = (k >> shift) & 255u;
                    atomicAdd(&s.hcnt[bin], 1u);
                    if (coverage) atomicAdd(&s.hmass[bin], mass_q(sc[p], smax, a.score_kind));
                }
            }
            __syncthreads();
            if (tid < WAVE) scan_bins(s, coverage, coverage ? need : (unsigned long long)b);
            __syncthreads();
            if (tid == 0) {
                s.prefix |= s.bin << shift;
                s.pmask |= 255u << shift;
            }
            __syncthreads();
        }
        tau = s.prefix;
        const int count_eq = (int)s.hcnt[s.bin];
        const int cab = s.cnt_above;
        if (coverage) {
            const unsigned long long rem = need - s.mass_above;
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

    // ---- keep + ascending compaction (chunked scans in page order) ---------------------
    const int n = np > 0 ? np : 0;
    const int chunk = (n + SEL_THREADS - 1) / SEL_THREADS;
    const int c0 = tid * chunk;
    const int c1 = min(c0 + chunk, n);
    const float ftau = u2f(tau);
    int tie_local = 0;
    if (!keep_all && a.tie_mode == 0)
        for (int p = max(c0, lo); p < min(c1, hi); ++p) tie_local += (f2u(sc[p]) == tau);
    int ties_total;
    int tie_base = block_excl_scan(tie_local, s.ired, ties_total);
    int keep_local = 0;
    for (int p = c0; p < c1; ++p) {
        bool keep;
        if (keep_all || p < lo || p >= hi) {
            keep = true;
        } else {
            const float v = sc[p];
            if (a.tie_mode == 1) {
                keep = v >= ftau;
            } else {
                const unsigned int k = f2u(v);
                keep = k > tau || (k == tau && tie_base++ < take);
            }
        }
        keep_local += keep;
    }
    int cnt;
    int pos = block_excl_scan(keep_local, s.ired, cnt);
    tie_base = block_excl_scan(tie_local, s.ired, ties_total);
    for (int p = c0; p < c1; ++p) {
        bool keep;
        if (keep_all || p < lo || p >= hi) {
            keep = true;
        } else {
            const float v = sc[p];
            if (a.tie_mode == 1) {
                keep = v >= ftau;
            } else {
                const unsigned int k = f2u(v);
                keep = k > tau || (k == tau && tie_base++ < take);
            }
        }
        if (keep) tab[pos++] = p;
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
    const size_t lds = (size_t)a->max_pages * sizeof(float);
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
