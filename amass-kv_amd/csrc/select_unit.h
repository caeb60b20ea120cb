// Stage-A selection of one (request, kv head) unit by one workgroup, shared by the
// selection kernel (select.hip) and the per-unit pipeline kernel (unit.hip).  The design
// notes are at the top of select.hip.
#pragma once
#include "common.h"

namespace amass {

// ------------------------------------------------------------------ wave helpers
// number of set bits of `m` below this lane
__device__ __forceinline__ int lanes_below(unsigned long long m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// The nrm combine's exp (every combine site uses this one, so the standalone, fused and
// pre-pass combines agree bit for bit): the hardware exp2 of x log2(e), ~1e-7 relative.
__device__ __forceinline__ float nrm_exp(float x) { return __expf(x); }

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

// The selection of unit (request r, kv head kh) by a workgroup of NT threads (the body of
// select_kernel; the per-unit pipeline kernel calls it after scoring the unit).  Returns
// the unit's page count (uniform over the workgroup).
template <int NT, int PPT, bool NRM>
__device__ __forceinline__ int select_unit(const amass_select_args& a, int r, int kh, XSel& s) {
    constexpr int NW = NT / WAVE;
    constexpr int V = PPT < 4 ? PPT : 4;        // pages per run
    constexpr int NC = PPT / V;                 // runs (chunks) per thread
    constexpr int CSTEP = V * NT;               // pages per chunk
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
        // plain scores: only the row's scored pages (a ragged batch's short rows would
        // otherwise stream their whole MP-wide rows; config 2: 1.36x the algorithmic bytes).
        // The n_sel_hi load goes first; at these launches' latency it measured no slower
        // (config 2 10.4 us either way), where the fused staging above, whose rows the
        // latency-bound single-request and config-1 launches read whole, lost ~0.1-0.2 us.
        const int lb = min(max(a.n_sel_hi[r], 0), MP);
        const bool vec = (((uintptr_t)gscore) & 15) == 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) ld_pages<V>(gscore, page_of(c, 0), lb, vec, 0.f, &v[c * V]);
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
    return cnt;
}

}  // namespace amass
