// mem-v write path for gfx950: residency invalidation, the per-step staging lifecycle
// (flushed-bit clear, flush collect, flush copy to the pinned pool, staging-block alloc,
// token slots) and the per-layer V scatter.
//
// Semantics of tier/residency.py:251-278 (_invalidate_kernel) and tier/staging.py:51-232
// (_scatter_kv, _vflush_clear, _flush_collect, _flush_copy, _valloc, _vslot kernels),
// taken in (request, page) order.  The reference serialises collect and alloc in one
// program (grid (1,)) because they share the flush index and the free-stack top; here
// they are one 1024-thread workgroup each that ranks a whole chunk of pages at once with
// block scans, and visits only the 256-page chunks a parallel mark pass found holding a
// staged block (a decode step completes about one page per request every 16 tokens, so
// almost every chunk is skipped).  Shared blocks count once (the first occurrence in
// order), as the reference's atomic claims make them.
#include "common.h"

namespace amass {

constexpr int ST_CHUNK = 256;      // pages per mark chunk
constexpr int ST_THREADS = 1024;   // collect / alloc workgroup
constexpr int ST_WAVES = ST_THREADS / WAVE;

// exclusive prefix over the workgroup's threads of v; total in `total` (two barriers)
__device__ __forceinline__ int st_excl_scan(int v, int* red, int& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int x = wave_incl_scan(v);                  // DPP row steps + readlane
    __syncthreads();
    if (lane == 63) red[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
    for (int i = 0; i < nw; ++i) {
        const int t = red[i];
        if (i < w) base += t;
        tot += t;
    }
    total = tot;
    return base + x - v;
}

struct ReqRange {
    bool active;      // sl > 0 and ql > 0
    int ctx;          // settled tokens sl - ql
    int p0, p1;       // written pages
};
__device__ __forceinline__ ReqRange req_range(const int32_t* sl_, const int32_t* qsl, int r,
                                              int page) {
    ReqRange x;
    const int sl = sl_[r];
    const int ql = qsl[r + 1] - qsl[r];
    x.active = sl > 0 && ql > 0 && ql <= sl;
    x.ctx = sl - ql;
    x.p0 = x.ctx >= 0 ? x.ctx / page : 0;
    x.p1 = sl > 0 ? (sl - 1) / page : -1;
    return x;
}

// ------------------------------------------------------------------ invalidate
// grid (n_req, L): every (written page, kv head) of request r in layer l
__global__ __launch_bounds__(256) void invalidate_kernel(const amass_invalidate_args a) {
    const int r = blockIdx.x, l = blockIdx.y;
    const int sl = a.seq_lens[r];
    if (sl <= 0) return;
    const int ql = a.query_start_loc[r + 1] - a.query_start_loc[r];
    const int ctx = sl - ql > 0 ? sl - ql : 0;
    const int p0 = ctx / a.page;
    const int p1 = min((sl - 1) / a.page, a.max_pages - 1);
    const int npg = p1 - p0 + 1;
    const int32_t* bt = a.block_table + (int64_t)r * a.bt_st;
    for (int i = threadIdx.x; i < npg * a.n_kv; i += blockDim.x) {
        const int p = p0 + i / a.n_kv, kv = i % a.n_kv;
        const int blk = bt[p];
        if (blk < 0 || blk >= a.nb) continue;
        const int64_t lk = (int64_t)l * a.n_kv + kv;
        const int64_t row = lk * a.nb + blk;
        a.pool_valid[row] = 0;
        const int slot = a.page2slot[row];
        if (slot >= 0 && slot < a.slots) {
            a.page2slot[row] = -1;
            a.slot2page[lk * a.slots + slot] = -1;
        }
    }
}

// ------------------------------------------------------------------ begin_step 1: mark
// grid (n_chunks, n_req): workgroup (c, r) counts the staged complete pages of chunk c of
// request r into mark[r][c]; chunk 0 also clears v_flushed of r's written pages.
__global__ __launch_bounds__(ST_CHUNK) void stage_mark_kernel(const amass_stage_args a,
                                                              int n_chunks) {
    __shared__ int red[ST_CHUNK / WAVE];
    const int c = blockIdx.x, r = blockIdx.y;
    const ReqRange q = req_range(a.seq_lens, a.query_start_loc, r, a.page);
    const int32_t* bt = a.block_table + (int64_t)r * a.bt_st;
    if (q.active && c == 0) {
        for (int p = q.p0 + (int)threadIdx.x; p <= q.p1 && p < a.max_pages; p += blockDim.x) {
            const int blk = bt[p];
            if (blk >= 0 && blk < a.nb) a.v_flushed[blk] = 0;
        }
    }
    const int np = q.active ? min(q.ctx / a.page, a.max_pages) : 0;
    const int p = c * ST_CHUNK + threadIdx.x;
    int cand = 0;
    if (p < np) {
        const int blk = bt[p];
        cand = (blk >= 0 && blk < a.nb && a.vbo[blk] >= 0) ? 1 : 0;
    }
    int tot;
    st_excl_scan(cand, red, tot);
    if (threadIdx.x == 0) a.mark[(int64_t)r * n_chunks + c] = tot;
}

// ------------------------------------------------------------------ begin_step 2: collect
// One workgroup.  Nonzero mark chunks in (request, chunk) order; per chunk one page per
// thread: new claims (not flushed) take flush-list slots while there is room, every
// staged page not left over is freed onto the stack.
__global__ __launch_bounds__(ST_THREADS) void stage_collect_kernel(const amass_stage_args a,
                                                                   int n_chunks) {
    __shared__ int red[ST_WAVES];
    __shared__ int list[ST_THREADS];
    __shared__ int s_fcnt, s_top;
    const int tid = threadIdx.x;
    if (tid == 0) {
        s_fcnt = 0;
        s_top = *a.free_top;
    }
    __syncthreads();
    const int T = a.n_req * n_chunks;
    for (int w0 = 0; w0 < T; w0 += ST_THREADS) {
        const int e = w0 + tid;
        const int nz = (e < T && a.mark[e] > 0) ? 1 : 0;
        int nlist;
        const int pos = st_excl_scan(nz, red, nlist);
        if (nz) list[pos] = e;
        __syncthreads();
        for (int k = 0; k < nlist; ++k) {
            const int ch = list[k];
            const int r = ch / n_chunks, c = ch % n_chunks;
            const ReqRange q = req_range(a.seq_lens, a.query_start_loc, r, a.page);
            const int np = q.active ? min(q.ctx / a.page, a.max_pages) : 0;
            const int p = c * ST_CHUNK + tid;
            int blk = -1, vb = -1;
            bool cand = false, fresh = false;
            if (tid < ST_CHUNK && p < np) {
                blk = a.block_table[(int64_t)r * a.bt_st + p];
                if (blk >= 0 && blk < a.nb) {
                    vb = a.vbo[blk];
                    cand = vb >= 0 && vb < a.nv;
                    fresh = cand && a.v_flushed[blk] == 0;
                }
            }
            const int fc = s_fcnt, top = s_top;
            int nfresh;
            const int rn = st_excl_scan(fresh ? 1 : 0, red, nfresh);
            const int i = fc + rn;
            const bool ok = fresh && i < a.maxf;
            const bool over = fresh && i >= a.maxf;
            const bool fr = cand && !over;
            int nfree;
            const int rf = st_excl_scan(fr ? 1 : 0, red, nfree);
            if (ok) {
                a.flush_list[2 * i] = blk;
                a.flush_list[2 * i + 1] = vb;
                a.v_flushed[blk] = 1;
            }
            if (fr) {
                a.vbo[blk] = -1;
                a.free_stack[top + rf] = vb;
            }
            __syncthreads();
            if (tid == 0) {
                s_fcnt = min(fc + nfresh, max(fc, a.maxf));
                s_top = top + nfree;
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        *a.flush_cnt = s_fcnt;
        *a.free_top = s_top;
    }
}

// ------------------------------------------------------------------ begin_step 3: copy
// grid (maxf, L): list entry i of layer l: v_pool[l, vb] (page, n_kv, d) -> pinned pool
// [l, blk, kv] (page, d) for every kv head, 16-byte copies; then pool_valid = 1.
__global__ __launch_bounds__(256) void stage_flush_copy_kernel(const amass_stage_args a) {
    const int i = blockIdx.x, l = blockIdx.y;
    if (i >= *a.flush_cnt) return;
    const int blk = a.flush_list[2 * i], vb = a.flush_list[2 * i + 1];
    const int cpr = a.d / 8;                           // 16-byte chunks per row
    const int total = a.n_kv * a.page * cpr;
    const uint16_t* src = (const uint16_t*)a.v_pool + (int64_t)l * a.vp_sl + (int64_t)vb * a.vp_sb;
    uint16_t* dst = (uint16_t*)a.pool + (((int64_t)l * a.nb + blk) * a.n_kv) * a.page * a.d;
    for (int x = threadIdx.x; x < total; x += blockDim.x) {
        const int ch = x % cpr, t = (x / cpr) % a.page, kv = x / (cpr * a.page);
        const uint4 v = *reinterpret_cast<const uint4*>(src + (int64_t)t * a.vp_st +
                                                        (int64_t)kv * a.vp_sh + 8 * ch);
        *reinterpret_cast<uint4*>(dst + ((int64_t)kv * a.page + t) * a.d + 8 * ch) = v;
    }
    for (int kv = threadIdx.x; kv < a.n_kv; kv += blockDim.x)
        a.pool_valid[((int64_t)l * a.n_kv + kv) * a.nb + blk] = 1;
}

// ------------------------------------------------------------------ begin_step 4: alloc
// One workgroup.  The written pages of all active requests, flattened in (request, page)
// order, in chunks of 1024: a page whose block has no staging block pops the stack;
// duplicates of a block inside a chunk defer to the first (atomicMin on `first`).
__global__ __launch_bounds__(ST_THREADS) void stage_alloc_kernel(const amass_stage_args a) {
    __shared__ int red[ST_WAVES];
    __shared__ int woff[ST_THREADS];
    __shared__ int s_top, s_ovf;
    const int tid = threadIdx.x;
    if (tid == 0) {
        s_top = *a.free_top;
        s_ovf = 0;
    }
    __syncthreads();
    for (int rb = 0; rb < a.n_req; rb += ST_THREADS) {
        const int nr = min(ST_THREADS, a.n_req - rb);
        int nw = 0;
        if (tid < nr) {
            const ReqRange q = req_range(a.seq_lens, a.query_start_loc, rb + tid, a.page);
            if (q.active) nw = max(0, min(q.p1, a.max_pages - 1) - q.p0 + 1);
        }
        int tot;
        const int off = st_excl_scan(nw, red, tot);
        woff[tid] = off;
        __syncthreads();
        for (int e0 = 0; e0 < tot; e0 += ST_THREADS) {
            const int e = e0 + tid;
            int blk = -1;
            bool need = false;
            if (e < tot) {
                int lo = 0, hi = nr - 1;                 // last request with woff <= e
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (woff[mid] <= e) lo = mid;
                    else hi = mid - 1;
                }
                const int r = rb + lo;
                const ReqRange q = req_range(a.seq_lens, a.query_start_loc, r, a.page);
                blk = a.block_table[(int64_t)r * a.bt_st + q.p0 + (e - woff[lo])];
                need = blk >= 0 && blk < a.nb && a.vbo[blk] < 0;
            }
            if (need) atomicMin(&a.first[blk], e);
            __syncthreads();
            const bool lead = need && atomicAdd(&a.first[blk], 0) == e;
            int nlead;
            const int rk = st_excl_scan(lead ? 1 : 0, red, nlead);
            const int top = s_top;
            if (lead) {
                if (rk < top) a.vbo[blk] = a.free_stack[top - 1 - rk];
                else s_ovf = 1;
            }
            __syncthreads();
            if (need) atomicExch(&a.first[blk], 0x7FFFFFFF);   // scratch back at rest
            if (tid == 0) s_top = max(top - nlead, 0);
            __syncthreads();
        }
    }
    if (tid == 0) {
        *a.free_top = s_top;
        if (s_ovf) *a.overflow = 1;
    }
}

// ------------------------------------------------------------------ begin_step 5: slots
__global__ __launch_bounds__(256) void stage_vslot_kernel(const amass_stage_args a) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.n_tokens) return;
    int64_t out = -1;
    const int32_t* qsl = a.query_start_loc;
    if (a.n_req > 0 && t >= qsl[0] && t < qsl[a.n_req]) {
        int lo = 0, hi = a.n_req - 1;                      // last request with qsl <= t
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (qsl[mid] <= t) lo = mid;
            else hi = mid - 1;
        }
        const ReqRange q = req_range(a.seq_lens, qsl, lo, a.page);
        if (q.active) {
            const int pos = q.ctx + (t - qsl[lo]);
            const int p = pos / a.page;
            if (p < a.max_pages) {
                const int blk = a.block_table[(int64_t)lo * a.bt_st + p];
                if (blk >= 0 && blk < a.nb) {
                    const int vb = a.vbo[blk];
                    if (vb >= 0) out = (int64_t)vb * a.page + pos % a.page;
                }
            }
        }
    }
    a.v_slot[t] = out;
}

// ------------------------------------------------------------------ scatter
// grid (n_tokens): token t's n_kv x d V row -> its staging slot
__global__ __launch_bounds__(128) void stage_scatter_kernel(const amass_scatter_args a) {
    const int t = blockIdx.x;
    const int64_t vs = a.v_slot[t];
    if (vs < 0) return;
    const int64_t vb = vs / a.page;
    const int off = (int)(vs % a.page);
    if (vb >= a.nv) return;
    const int cpr = a.d / 8;
    const uint16_t* src = (const uint16_t*)a.value + (int64_t)t * a.v_st;
    uint16_t* dst = (uint16_t*)a.v_pool + vb * a.vp_sb + (int64_t)off * a.vp_st;
    for (int x = threadIdx.x; x < a.n_kv * cpr; x += blockDim.x) {
        const int kv = x / cpr, ch = x % cpr;
        *reinterpret_cast<uint4*>(dst + (int64_t)kv * a.vp_sh + 8 * ch) =
            *reinterpret_cast<const uint4*>(src + (int64_t)kv * a.v_sh + 8 * ch);
    }
}

static bool al16(const void* p, int64_t elems) {
    return (((uintptr_t)p) & 15) == 0 && (elems % 8) == 0;
}

}  // namespace amass

using namespace amass;

extern "C" int amass_tier_invalidate(const amass_invalidate_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->block_table || !a->seq_lens || !a->query_start_loc || !a->page2slot ||
        !a->slot2page || !a->pool_valid)
        return AMASS_ERR_NULL;
    if (a->n_req < 0 || a->n_layers < 1 || a->nb < 1 || a->n_kv < 1 || a->slots < 1 ||
        a->page < 1 || a->max_pages < 1)
        return AMASS_ERR_GEOMETRY;
    if (a->n_req == 0) return AMASS_OK;
    hipLaunchKernelGGL(invalidate_kernel, dim3(a->n_req, a->n_layers), dim3(256), 0,
                       (hipStream_t)stream, *a);
    return check_launch();
}

extern "C" int amass_stage_begin_step(const amass_stage_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->block_table || !a->seq_lens || !a->query_start_loc || !a->vbo || !a->v_flushed ||
        !a->free_stack || !a->free_top || !a->v_slot || !a->flush_list || !a->flush_cnt ||
        !a->overflow || !a->mark || !a->first || !a->v_pool || !a->pool || !a->pool_valid)
        return AMASS_ERR_NULL;
    if (a->n_req < 0 || a->n_tokens < 0 || a->max_pages < 1 || a->n_layers < 1 || a->nb < 1 ||
        a->nv < 1 || a->n_kv < 1 || a->page < 1 || a->maxf < 1 || a->d < 8 || a->d % 8)
        return AMASS_ERR_GEOMETRY;
    if (!al16(a->v_pool, a->vp_sl) || a->vp_sb % 8 || a->vp_st % 8 || a->vp_sh % 8 ||
        !al16(a->pool, a->d))
        return AMASS_ERR_GEOMETRY;
    hipStream_t s = (hipStream_t)stream;
    const int n_chunks = (a->max_pages + ST_CHUNK - 1) / ST_CHUNK;
    if (a->n_req > 0) {
        hipLaunchKernelGGL(stage_mark_kernel, dim3(n_chunks, a->n_req), dim3(ST_CHUNK), 0, s,
                           *a, n_chunks);
        int rc = check_launch();
        if (rc) return rc;
    }
    hipLaunchKernelGGL(stage_collect_kernel, dim3(1), dim3(ST_THREADS), 0, s, *a, n_chunks);
    int rc = check_launch();
    if (rc) return rc;
    hipLaunchKernelGGL(stage_flush_copy_kernel, dim3(a->maxf, a->n_layers), dim3(256), 0, s, *a);
    if ((rc = check_launch())) return rc;
    hipLaunchKernelGGL(stage_alloc_kernel, dim3(1), dim3(ST_THREADS), 0, s, *a);
    if ((rc = check_launch())) return rc;
    if (a->n_tokens > 0) {
        hipLaunchKernelGGL(stage_vslot_kernel, dim3((a->n_tokens + 255) / 256), dim3(256), 0,
                           s, *a);
        rc = check_launch();
    }
    return rc;
}

extern "C" int amass_stage_scatter(const amass_scatter_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if (!a->value || !a->v_slot || !a->v_pool) return AMASS_ERR_NULL;
    if (a->n_tokens < 0 || a->n_kv < 1 || a->d < 8 || a->d % 8 || a->page < 1 || a->nv < 1)
        return AMASS_ERR_GEOMETRY;
    if (!al16(a->value, a->v_st) || a->v_sh % 8 || !al16(a->v_pool, a->vp_sb) ||
        a->vp_st % 8 || a->vp_sh % 8)
        return AMASS_ERR_GEOMETRY;
    if (a->n_tokens == 0) return AMASS_OK;
    hipLaunchKernelGGL(stage_scatter_kernel, dim3(a->n_tokens), dim3(128), 0,
                       (hipStream_t)stream, *a);
    return check_launch();
}
