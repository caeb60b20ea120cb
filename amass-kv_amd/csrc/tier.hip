// mem-v tier residency for gfx950: gather plan (hits / misses / exact-LRU victims) and
// the flat miss fetch from the pinned, device-mapped host pool into the HBM hot buffer.
//
// Semantics of tier/residency.py:45-139 (_miss_diff_kernel, _select_victims_kernel) and
// :196-248 (_fetch_flat_kernel).  The reference picks victims one miss at a time per
// kv-head (an argmin over all S slots per miss).  Because a slot chosen as a victim gets
// clock = now and so leaves the candidate set, that sequential rule is the same as: sort
// the slots not touched this step by (lru clock, slot index) and give the k-th DISTINCT
// new miss (in request, position order) the k-th slot.  The victim kernel does exactly
// that with one workgroup per kv-head: a dedup pass (atomicMin of the first flat position
// per physical block), a block scan that ranks the first occurrences, an ordering of the
// untouched slots by (clock, slot) -- a histogram cut plus a rank count
// over the slots the new misses need, or a stable radix sort of all of them -- and a
// parallel apply.  No serial per-miss loop remains.  The step's clock is clock[0] + 1; the
// victims launch's last workgroup stores it (no separate clock launch).
#include "common.h"

namespace amass {

constexpr int TP_THREADS = 1024;
constexpr int TP_WAVES = TP_THREADS / WAVE;
constexpr int TP_MAXS = 8192;
constexpr int TP_MAXREQ = 1024;
constexpr int MD_THREADS = 1024;              // miss diff: a unit's pages in one pass (<= 1024)


template <int NT>
__device__ __forceinline__ int blk_excl_scan(int v, int* red, int& total) {
    constexpr int NW = NT / WAVE;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int x = wave_incl_scan(v);                  // DPP row steps + readlane
    __syncthreads();
    if (lane == 63) red[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int t = red[i];
        if (i < w) base += t;
        tot += t;
    }
    total = tot;
    return base + x - v;
}

// ---- hits touch the LRU clock; misses are compacted in selection order ----------------
__global__ __launch_bounds__(MD_THREADS) void miss_diff_kernel(const amass_tier_plan_args a) {
    __shared__ int red[MD_THREADS / WAVE];
    const int kv = blockIdx.x, r = blockIdx.y;
    const int32_t* tab = a.page_table + (int64_t)r * a.pt_sr + (int64_t)kv * a.pt_sh;
    // the first page ids are loaded with the count (rows are max_pages wide), so the
    // block lookups wait for one round trip less
    const int pt0 = (int)threadIdx.x < a.max_pages ? tab[threadIdx.x] : 0;
    const int n = a.page_cnt[(int64_t)r * a.pc_sr + kv];
    const int sl = a.seq_lens[r];
    const int clk = a.clock[0] + 1;                    // this step's clock
    if (kv == 0 && r == 0 && threadIdx.x == 0) a.fetch_cnt[0] = 0;
    const int32_t* bt = a.block_table + (int64_t)r * a.bt_st;
    int32_t* mp = a.miss_pages + ((int64_t)r * a.n_kv + kv) * a.max_pages;
    int nmiss = 0;
    for (int off = 0; off < n; off += MD_THREADS) {
        const int idx = off + threadIdx.x;
        int is_miss = 0, blk = 0;
        if (idx < n) {
            const int pt = off == 0 ? pt0 : tab[idx];
            blk = bt[pt];
            const bool complete = (int64_t)(pt + 1) * a.page <= (int64_t)sl;
            const int slot = a.page2slot[(int64_t)kv * a.nb + blk];
            if (complete && slot >= 0) a.lru_clock[(int64_t)kv * a.slots + slot] = clk;
            is_miss = (complete && slot < 0) ? 1 : 0;
        }
        int tot;
        const int pos = blk_excl_scan<MD_THREADS>(is_miss, red, tot);
        if (is_miss) mp[nmiss + pos] = blk;
        nmiss += tot;
    }
    if (threadIdx.x == 0) a.miss_cnt[(int64_t)r * a.n_kv + kv] = nmiss;
}

__device__ __forceinline__ int load_agent(const int32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- per kv-head: dedup, rank new misses, sort untouched slots, apply ------------------
__global__ __launch_bounds__(TP_THREADS) void victims_kernel(const amass_tier_plan_args a) {
    __shared__ int off[TP_MAXREQ + 1];
    __shared__ uint16_t sb[2][TP_MAXS];
    __shared__ int red[TP_WAVES], red2[TP_WAVES];
    __shared__ int smax_s[TP_WAVES], smin_s[TP_WAVES];
    __shared__ __align__(16) int hist[256];
    __shared__ uint32_t cand[TP_THREADS];
    __shared__ int sel_bin, sel_quota, fbase;
    __shared__ int sclk[TP_MAXS];                      // the slots' clocks (load transpose)
    const int kv = blockIdx.x, tid = threadIdx.x;
    const int clk = a.clock[0] + 1;                    // this step's clock
    if (a.n_req == 0 && kv == 0 && tid == 0) a.fetch_cnt[0] = 0;   // (else: miss_diff's)
    const int S = a.slots;
    const int64_t mbase_kv = (int64_t)kv * a.max_pages;
    int32_t* fp = a.first_pos + (int64_t)kv * a.nb;
    int32_t* p2s = a.page2slot + (int64_t)kv * a.nb;
    int32_t* s2p = a.slot2page + (int64_t)kv * S;
    int32_t* lru = a.lru_clock + (int64_t)kv * S;

    // 1. flat offsets of every request's miss list.  The slots' clocks are loaded right
    // after the counts (nothing in this launch writes them before the apply), coalesced
    // (slot tid + TP_THREADS i), and pass through LDS to each thread's run of CS
    // consecutive slots, so their latency hides under the miss bookkeeping; INT_MAX marks
    // a position past the buffer (never below the step's clock: not a candidate).
    constexpr int SPT = TP_MAXS / TP_THREADS;          // slots per thread (S <= TP_MAXS)
    int mc = tid < a.n_req ? a.miss_cnt[(int64_t)tid * a.n_kv + kv] : 0;
    int lv[SPT];
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        const int sidx = tid + TP_THREADS * i;
        lv[i] = sidx < S ? lru[sidx] : 0x7FFFFFFF;
    }
    int M;
    const int o = blk_excl_scan<TP_THREADS>(mc, red, M);
    if (tid < a.n_req) off[tid] = o;
    if (tid == 0) off[a.n_req] = M;
#pragma unroll
    for (int i = 0; i < SPT; ++i) sclk[tid + TP_THREADS * i] = lv[i];
    __syncthreads();
    const int CS = (S + TP_THREADS - 1) / TP_THREADS;
    const int s0 = min(tid * CS, S), s1 = min(s0 + CS, S);
    int cl[SPT];
#pragma unroll
    for (int i = 0; i < SPT; ++i) cl[i] = (i < CS && s0 + i < s1) ? sclk[s0 + i] : 0x7FFFFFFF;
    if (M > 0) {                                       // uniform

    const int C = (M + TP_THREADS - 1) / TP_THREADS;
    const int f0 = min(tid * C, M), f1 = min(f0 + C, M);
    auto locate = [&](int f, int& r) {      // r: request owning flat position f
        while (off[r + 1] <= f) ++r;
    };
    auto miss_at = [&](int r, int f) -> int32_t* {
        return a.miss_pages + (int64_t)r * a.n_kv * a.max_pages + mbase_kv + (f - off[r]);
    };
    int r0 = 0;
    {   // first request of this chunk (binary search)
        int lo = 0, hi = a.n_req - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (off[mid] <= f0) lo = mid; else hi = mid - 1;
        }
        r0 = lo;
    }

    // 2. first occurrence of each physical block among this step's misses (the block of
    // the thread's first position stays in a register for the passes below: with at most
    // TP_THREADS misses per kv head it is the thread's only one)
    int mb0 = 0;
    {
        int r = r0;
        for (int f = f0; f < f1; ++f) {
            locate(f, r);
            const int b = *miss_at(r, f);
            if (f == f0) mb0 = b;
            atomicMin(&fp[b], f);
        }
    }
    auto block_at = [&](int r, int f) -> int { return f == f0 ? mb0 : *miss_at(r, f); };
    // the atomics act at L2 and the agent-scope loads below read L2; the barrier's release
    // waits for this workgroup's atomics, so no device-scope fence is needed (one cost
    // ~4 us here: it writes back and invalidates the XCD's L2)
    __syncthreads();

    // 3. rank the distinct new misses in flat order
    int nfirst = 0;
    {
        int r = r0;
        for (int f = f0; f < f1; ++f) {
            locate(f, r);
            nfirst += (load_agent(&fp[block_at(r, f)]) == f);
        }
    }

    // 4. the order of the untouched slots by (clock, slot).  Only the first Mnew are
    // used: when they all lie within 255 clock values of the oldest untouched clock and
    // Mnew <= TP_THREADS, a 256-bin histogram of clock - cmin finds the bin B holding the
    // Mnew-th slot, the slots of the bins below B and the first ones of bin B (slot order)
    // are gathered as (clock - cmin) << 13 | slot keys, and each is placed by counting the
    // smaller keys.  Otherwise (wide clock ranges, more new misses than threads, or fewer
    // untouched slots than new misses) all untouched slots are sorted: a stable 1-bit LSD
    // radix sort by clock over the bits the clocks use.
    int nun = 0, kmax = 0, kmin = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        if (cl[i] < clk) {
            ++nun;
            kmax = max(kmax, cl[i]);
            kmin = min(kmin, cl[i]);
        }
    }
    // one exchange for both block scans (distinct new misses, untouched slots) and the
    // clock range (clocks are >= 0: their unsigned order is their order); every thread
    // read the last scan's totals before the barriers since, so `red` is free
    int Mnew, U, rank0, upos;
    {
        const int lane = tid & 63, w = tid >> 6;
        const int xf = wave_incl_scan(nfirst), xu = wave_incl_scan(nun);
        const int km = (int)wave_maxu_uniform((uint32_t)kmax);
        const int kn = (int)wave_minu_uniform((uint32_t)kmin);
        if (lane == 63) {
            red[w] = xf;
            red2[w] = xu;
            smax_s[w] = km;
            smin_s[w] = kn;
        }
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        int bf = 0, bu = 0, tf = 0, tu = 0;
#pragma unroll
        for (int i = 0; i < TP_WAVES; ++i) {
            const int f = red[i], u = red2[i];
            if (i < w) { bf += f; bu += u; }
            tf += f;
            tu += u;
        }
        Mnew = tf;
        U = tu;
        rank0 = bf + xf - nfirst;
        upos = bu + xu - nun;
    }
    // one fetch-list reservation per kv head for its min(Mnew, U) fetches (the k-th new
    // miss takes entry fbase + k), issued by wave 1 while wave 0 searches the histogram
    if (tid == WAVE) fbase = atomicAdd(a.fetch_cnt, min(Mnew, U));
    int kall = 0, cmin = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < TP_WAVES; ++i) {
        kall = max(kall, smax_s[i]);
        cmin = min(cmin, smin_s[i]);
    }
    const uint16_t* sorted = sb[0];
    bool fast = U >= Mnew && Mnew <= TP_THREADS;
    if (fast) {
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            // a wave whose 64 lanes share a bin adds once (a cold buffer puts every slot
            // in bin 0)
            const int bin = cl[i] < clk ? min(cl[i] - cmin, 255) : -1;
            const int b0 = __builtin_amdgcn_readfirstlane(bin);
            if (__ballot(bin == b0) == ~0ull) {
                if (b0 >= 0 && (tid & 63) == 0) atomicAdd(&hist[b0], WAVE);
            } else if (bin >= 0) {
                atomicAdd(&hist[bin], 1);
            }
        }
        __syncthreads();
        // B = the first bin whose running count reaches Mnew (>= 1: M > 0 has a first
        // occurrence) and the quota taken from it: wave 0 alone, lane l summing bins
        // 4l .. 4l + 3 (every untouched slot has a bin, so the total U >= Mnew is reached)
        if (tid < WAVE) {
            const int4 h = reinterpret_cast<const int4*>(hist)[tid];
            const int sum = (h.x + h.y) + (h.z + h.w);
            const int incl = wave_incl_scan(sum);
            const unsigned long long hit = __ballot(incl >= Mnew);
            if (tid == __ffsll((long long)hit) - 1) {
                int c = incl - sum, b = 4 * tid;
                if (c + h.x < Mnew) {
                    c += h.x; ++b;
                    if (c + h.y < Mnew) {
                        c += h.y; ++b;
                        if (c + h.z < Mnew) { c += h.z; ++b; }
                    }
                }
                sel_bin = b;
                sel_quota = Mnew - c;
            }
        }
        __syncthreads();
        const int B = sel_bin, quota = sel_quota;
        fast = B < 255;                               // uniform
        if (fast) {
            // one scan of packed (bin-B slots << 16 | slots below bin B) counts: a thread's
            // first taken slot goes to (below-B slots before it) + min(bin-B slots before
            // it, quota), its bin-B slots taken in slot order while their rank < quota
            int nl = 0, nb = 0;
#pragma unroll
            for (int i = 0; i < SPT; ++i)
                if (cl[i] < clk) {
                    nl += cl[i] - cmin < B ? 1 : 0;
                    nb += cl[i] - cmin == B ? 1 : 0;
                }
            int tpk;
            const int pk = blk_excl_scan<TP_THREADS>(nl | (nb << 16), red, tpk);
            int rb = pk >> 16;
            int cp = (pk & 0xFFFF) + min(rb, quota);
            bool take[SPT];
#pragma unroll
            for (int i = 0; i < SPT; ++i) {
                const int rel = cl[i] - cmin;
                take[i] = false;
                if (cl[i] < clk) {
                    if (rel < B) take[i] = true;
                    else if (rel == B) take[i] = rb++ < quota;
                }
            }
            if (B == 0) {
                // every candidate lies in the oldest bin: their order is the slot order,
                // which is the order of the scan (the usual case once the buffer has aged
                // in whole steps: the oldest clock holds many slots)
#pragma unroll
                for (int i = 0; i < SPT; ++i)
                    if (take[i]) sb[0][cp++] = (uint16_t)(s0 + i);
                __syncthreads();
            } else {
#pragma unroll
                for (int i = 0; i < SPT; ++i)
                    if (take[i])
                        cand[cp++] = ((uint32_t)(cl[i] - cmin) << 13) | (uint32_t)(s0 + i);
                __syncthreads();
                if (tid < Mnew) {
                    const uint32_t key = cand[tid];
                    int rank = 0;
                    for (int j = 0; j < Mnew; ++j) rank += cand[j] < key ? 1 : 0;
                    sb[0][rank] = (uint16_t)(key & 0x1FFFu);
                }
                __syncthreads();
            }
        }
    }
    if (!fast) {
        for (int i = 0; i < SPT; ++i) {
            const int sidx = s0 + i;
            if (cl[i] < clk) sb[0][upos++] = (uint16_t)sidx;
        }
        __syncthreads();
        const int nbits = kall > 0 ? 32 - __clz(kall) : 0;
        const int CU = (U + TP_THREADS - 1) / TP_THREADS;
        const int u0 = min(tid * CU, U), u1 = min(u0 + CU, U);
        for (int b = 0; b < nbits; ++b) {
            const uint16_t* cur = sb[b & 1];
            uint16_t* nxt = sb[(b + 1) & 1];
            int nz = 0;
            for (int i = u0; i < u1; ++i) nz += ((lru[cur[i]] >> b) & 1) == 0;
            int Z;
            int zb = blk_excl_scan<TP_THREADS>(nz, red, Z);
            for (int i = u0; i < u1; ++i) {
                const uint16_t sv = cur[i];
                if (((lru[sv] >> b) & 1) == 0) nxt[zb++] = sv;
                else nxt[Z + (i - zb)] = sv;
            }
            __syncthreads();
        }
        sorted = sb[nbits & 1];
    }

    // 5. apply: the k-th new miss takes sorted[k]; duplicates and overflow get -1
    {
        int r = r0, rank = rank0;
        for (int f = f0; f < f1; ++f) {
            locate(f, r);
            const int32_t blk = block_at(r, f);
            int32_t* vict = a.victim_slots + (int64_t)r * a.n_kv * a.max_pages + mbase_kv +
                            (f - off[r]);
            if (load_agent(&fp[blk]) != f) {
                *vict = -1;
                continue;
            }
            const int k = rank++;
            if (k >= U) {
                *vict = -1;
                a.overflow[0] = 1;
                continue;
            }
            const int s = sorted[k];
            const int old = s2p[s];
            if (old >= 0) p2s[old] = -1;
            p2s[blk] = s;
            s2p[s] = blk;
            lru[s] = clk;
            *vict = s;
            const int fi = fbase + k;
            if (fi < a.fcap) {
                a.fetch_list[3 * (int64_t)fi + 0] = kv;
                a.fetch_list[3 * (int64_t)fi + 1] = blk;
                a.fetch_list[3 * (int64_t)fi + 2] = s;
            }
        }
    }
    __syncthreads();
    // 6. restore the dedup scratch
    {
        int r = r0;
        for (int f = f0; f < f1; ++f) {
            locate(f, r);
            fp[block_at(r, f)] = 0x7FFFFFFF;
        }
    }
    }
    // the last workgroup to finish advances the clock and clears the arrival count for the
    // next call.  Relaxed: a workgroup that uses the clock has consumed its load (the slot
    // comparisons) before it arrives, so no later store can be the value it read; the
    // tables this launch wrote reach the next launches at the kernel boundary (an acq_rel
    // RMW would write back and invalidate the XCD's L2 on every workgroup)
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(&a.clock[1], 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        if (old == (int)gridDim.x - 1) {
            __hip_atomic_store(&a.clock[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.clock[0], clk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---- flat fetch: one 4 KB page per workgroup iteration, 16 B per thread -----------------
__global__ __launch_bounds__(256) void fetch_kernel(const amass_tier_fetch_args a) {
    const int n = min(a.fetch_cnt[0], a.fcap);
    const int tid = threadIdx.x;
    const int tok = tid >> 4, ch = tid & 15;   // 16 tokens x 16 chunks of 8 elements
    const int64_t pe = (int64_t)a.page * a.d;  // elements per page
    for (int i = blockIdx.x; i < n; i += gridDim.x) {
        const int kv = a.fetch_list[3 * (int64_t)i + 0];
        const int blk = a.fetch_list[3 * (int64_t)i + 1];
        const int slot = a.fetch_list[3 * (int64_t)i + 2];
        uint16_t* hot = (uint16_t*)a.hot + ((int64_t)kv * a.slots + slot) * pe;
        uint16_t* pool = (uint16_t*)a.pool + (((int64_t)a.t_layer * a.nb + blk) * a.n_kv + kv) * pe;
        const int64_t e = (int64_t)tok * a.d + 8 * ch;
        const int8_t vld = a.pool_valid[(int64_t)kv * a.nb + blk];
        const int vb = a.vbo ? a.vbo[blk] : -1;
        if (vld == 0 && vb >= 0) {
            const uint16_t* st = (const uint16_t*)a.vpool + (int64_t)vb * a.v_sb +
                                 (int64_t)kv * a.v_sh + (int64_t)tok * a.v_st + 8 * ch;
            const uint4 x = *reinterpret_cast<const uint4*>(st);
            *reinterpret_cast<uint4*>(hot + e) = x;
            *reinterpret_cast<uint4*>(pool + e) = x;
            __syncthreads();
            if (tid == 0) a.pool_valid[(int64_t)kv * a.nb + blk] = 1;
        } else {
            *reinterpret_cast<uint4*>(hot + e) = *reinterpret_cast<const uint4*>(pool + e);
        }
    }
}

}  // namespace amass

using namespace amass;

extern "C" int amass_tier_gather_plan(const amass_tier_plan_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->page_table || !a->page_cnt || !a->block_table || !a->seq_lens || !a->page2slot ||
        !a->slot2page || !a->lru_clock || !a->clock || !a->miss_pages || !a->miss_cnt ||
        !a->victim_slots || !a->overflow || !a->fetch_list || !a->fetch_cnt || !a->first_pos)
        return AMASS_ERR_NULL;
    if (a->n_req < 0 || a->n_kv < 1 || a->nb < 1 || a->slots < 1 || a->max_pages < 1 ||
        a->page < 1 || a->fcap < 1)
        return AMASS_ERR_GEOMETRY;
    if (a->slots > TP_MAXS || a->n_req > TP_MAXREQ) return AMASS_ERR_CAPACITY;
    hipStream_t s = (hipStream_t)stream;
    int rc = check_launch();
    if (rc) return rc;
    if (a->n_req > 0) {          // (with no requests the victims launch alone advances the clock)
        hipLaunchKernelGGL(miss_diff_kernel, dim3(a->n_kv, a->n_req), dim3(MD_THREADS), 0, s, *a);
        rc = check_launch();
        if (rc) return rc;
    }
    hipLaunchKernelGGL(victims_kernel, dim3(a->n_kv), dim3(TP_THREADS), 0, s, *a);
    return check_launch();
}

extern "C" int amass_tier_fetch(const amass_tier_fetch_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->fetch_list || !a->fetch_cnt || !a->hot || !a->pool || !a->pool_valid)
        return AMASS_ERR_NULL;
    if (a->page * a->d != 16 * 128 || a->n_kv < 1 || a->nb < 1 || a->slots < 1 || a->fcap < 1 ||
        a->grid < 1)
        return AMASS_ERR_GEOMETRY;
    if (a->vbo && !a->vpool) return AMASS_ERR_NULL;
    hipLaunchKernelGGL(fetch_kernel, dim3(a->grid), dim3(256), 0, (hipStream_t)stream, *a);
    return check_launch();
}
