// Int8 matrix-core front end shared by the quad and r8 page-score kernels (gfx950).
//
// Both scores start with the same small integer product per page: the 2G int8 query
// limbs of one kv head against the r' (or r) columns of the page's code matrix plus its
// mean codes, [2G x d] x [d x (r'+1)].  It runs on v_mfma_i32_16x16x64_i8 with M = the
// limb rows and K = 64 d per instruction; lane = 16 kg + n feeds 16 consecutive d
// (d = 64 t + 16 kg + s) of column n and receives result rows 4kg..4kg+3 of column n.
// The code columns come in groups of 16 / r' pages x r' ranks from the tiled records
// (below); the mean codes keep one page per column.
//
// q limbs: qi = rint(q * inv) with inv = 16383 / max|q| and qs = max|q| / 16383 (both
// correctly rounded divides), clamped to +-16383; hi = rint(qi / 128) clamped to +-127,
// lo = qi - 128 hi, so 128 hi + lo == qi and every contraction
// comb = 128 (hi . x) + (lo . x) is an exact int32 sum (the recipe of the reference's
// selection/quad_score_cuda.py:902-935 and selection/score_cuda.py:182-215, with IEEE
// divides where the reference compiles with fast math).
#pragma once
#include <mutex>

#include "common.h"

namespace amass {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int SC_TILE = 16;     // pages per MFMA tile (the N dimension)

__device__ __forceinline__ i32x4_t ld16(const int8_t* p) {
    return *reinterpret_cast<const i32x4_t*>(p);
}

__device__ __forceinline__ i32x4_t mfma_i8(i32x4_t a, i32x4_t b, i32x4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// bytes per code column / 16-byte loads per column and lane (int8: two K-steps; int4:
// one word set, byte j = code[j] | code[j + 64] << 4)
template <int VB> constexpr int col_bytes() { return VB == 8 ? 128 : 64; }
template <int VB> constexpr int loads_per_col() { return VB == 8 ? 2 : 1; }

// MFMA over one column: int8 -> two K-steps; int4 -> both K-steps from one word set
// (shifting the low nibble up and masking gives 16 * code as a signed byte).
template <int VB>
__device__ __forceinline__ i32x4_t col_mfma(const i32x4_t (&qa)[2], const i32x4_t* x) {
    i32x4_t acc = {0, 0, 0, 0};
    if constexpr (VB == 8) {
        acc = mfma_i8(qa[0], x[0], acc);
        acc = mfma_i8(qa[1], x[1], acc);
    } else {
        const i32x4_t m = {(int)0xF0F0F0F0u, (int)0xF0F0F0F0u, (int)0xF0F0F0F0u,
                           (int)0xF0F0F0F0u};
        acc = mfma_i8(qa[0], (x[0] << 4) & m, acc);
        acc = mfma_i8(qa[1], x[0] & m, acc);
    }
    return acc;
}

// Combined int32 contractions of result rows (4kg, 4kg+1) -> x and (4kg+2, 4kg+3) -> y.
template <int VB>
__device__ __forceinline__ void comb2(i32x4_t acc, int& x, int& y) {
    x = acc[0] * 128 + acc[1];
    y = acc[2] * 128 + acc[3];
    if constexpr (VB == 4) { x >>= 4; y >>= 4; }   // exact: both are multiples of 16
}

__device__ __forceinline__ float half_at(const uint32_t (&w)[4], int k) {
    return fp16_to_f32((uint16_t)((w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu));
}

// ---- tiled code records (quad_V / r8_Vk) ------------------------------------------------
// Column groups: an MFMA's 16 columns are PP = 16 / r' pages x r' ranks, so a tile is r'
// groups; lane (kg, n) of group j holds rank k = n % r' of page j PP + n / r'.
template <int RP> constexpr int group_pages() { return SC_TILE / RP; }
// the page whose mu, scales and score lane n carries (where the rank sums of the groups
// land, see rank_sum): lane n holds group n % r' of its r'-lane set n / r'
template <int RP>
__device__ __forceinline__ int lane_page(int n) {
    return (n % RP) * group_pages<RP>() + n / RP;
}

// V codes stream once per step: non-temporal 16-byte loads (each instruction reads PP
// runs of 64 r' contiguous bytes; the hint measured +10 % over plain loads on this
// pattern, and -10 % on one of 16 pages x 64 bytes).  NT = false gives plain loads, for
// records whose per-head size is not a whole number of 128-byte lines (two heads' waves
// then read the two parts of a shared line, and under the hint the L2 does not keep the
// line for the second of them: 272-byte records fetched 1.05x their bytes with the hint)
// and for the short runs of r' = 2.
template <bool NT = true>
__device__ __forceinline__ i32x4_t ld16_stream(const int8_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const i32x4_t*>(p));
    else return *reinterpret_cast<const i32x4_t*>(p);
}

// Record addresses as 32-bit byte offsets from the record buffer's base: block b's
// records start at rec + b rec_sb, one 32-bit product per lane and tile, which the lanes
// then exchange (group_blocks) instead of block ids.  A load is then the kernel's uniform
// base plus one 32-bit offset (the scalar-base form of the global load: no 64-bit
// arithmetic per lane and one VGPR per address; a 64-bit product per group load costs
// three quarter-rate multiplies).  The callers keep a layer's record buffer under 4 GiB,
// so every offset fits.
__device__ __forceinline__ int rec_off(int blk, int64_t rec_sb) {
    return (int)((uint32_t)blk * (uint32_t)rec_sb);
}
// base + the block's offset + a byte offset inside the block, summed as unsigned 32-bit
// (the offsets are carried in int lanes but may exceed 2^31)
__device__ __forceinline__ const int8_t* at_off(const int8_t* base, int off, int add) {
    return base + ((uint32_t)off + (uint32_t)add);
}

// the record offset (rec_off) of every group's page for this lane: lane m of a row
// carries page lane_page(m); group j's page for lane n is lane_page((n / RP) RP + j)
template <int RP>
__device__ __forceinline__ void group_blocks(int blk_own, int n, int (&gb)[RP]) {
    constexpr int PP = group_pages<RP>();
    if constexpr (PP >= 4) {            // r' <= 4: one lane permute per group
#pragma unroll
        for (int j = 0; j < RP; ++j)
            gb[j] = __shfl(blk_own, (threadIdx.x & 48) + (n / RP) * RP + j, WAVE);
        return;
    }
#pragma unroll
    for (int j = 0; j < RP; ++j) {
        int b = __builtin_amdgcn_readlane(blk_own, j);
#pragma unroll
        for (int pp = 1; pp < PP; ++pp) {
            const int c = __builtin_amdgcn_readlane(blk_own, pp * RP + j);
            b = n / RP == pp ? c : b;
        }
        gb[j] = b;
    }
}

// group j's V at rec + gb[j] (its record offset, rec_off) + lv, lv = h * VM + the lane's
// V offset 16 (kg r' + n % r')
template <int RP, int VB, int J0, int NG, bool NT = true>
__device__ __forceinline__ void load_groups(const int8_t* rec, int lv, const int (&gb)[RP],
                                            i32x4_t* v) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const int8_t* p = at_off(rec, gb[J0 + j], lv);
        if constexpr (VB == 8) {
            v[2 * j] = ld16_stream<NT>(p);
            v[2 * j + 1] = ld16_stream<NT>(p + 64 * RP);
        } else {
            v[j] = ld16_stream<NT>(p);
        }
    }
}

// Raw bf16 words of the A-row query of lane row n: row n holds limb (n & 1) of group
// head g = n >> 1 (DUP: g = (n >> 1) % G, so rows 2G..15 repeat rows 0..2G-1; otherwise
// rows of g >= G are zero).  Words cover d = 64 t + 16 kg + 2 i (+1).
__device__ __forceinline__ void load_q_rows(const uint16_t* q, int64_t q_st, int64_t q_hs,
                                            int req, int h, int G, int n, int kg, bool dup,
                                            uint32_t (&qw)[2][8]) {
    const int qg0 = n >> 1;
    const bool live = dup || qg0 < G;
    const int gq = dup ? qg0 % G : (live ? qg0 : G - 1);   // unconditional loads
    const uint16_t* qrow = q + (int64_t)req * q_st + (int64_t)(h * G + gq) * q_hs;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint4 x0 = *reinterpret_cast<const uint4*>(qrow + 64 * t + 16 * kg);
        const uint4 x1 = *reinterpret_cast<const uint4*>(qrow + 64 * t + 16 * kg + 8);
        qw[t][0] = x0.x; qw[t][1] = x0.y; qw[t][2] = x0.z; qw[t][3] = x0.w;
        qw[t][4] = x1.x; qw[t][5] = x1.y; qw[t][6] = x1.z; qw[t][7] = x1.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) qw[t][i] = live ? qw[t][i] : 0u;
    }
}

// Quantise the rows loaded by load_q_rows to int8 limbs: qa[t] is the A operand of
// K-step t; returns this row's qs (the row's amax is reduced over its four kg lanes).
__device__ __forceinline__ float quantize_q_rows(const uint32_t (&qw)[2][8], int n,
                                                 i32x4_t (&qa)[2]) {
    // |bf16| orders like its magnitude bits: take the max as integers
    uint32_t amax = 0;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            amax = max(amax, max(qw[t][i] & 0x7FFFu, (qw[t][i] >> 16) & 0x7FFFu));
    float mx = __uint_as_float(amax << 16);
    mx = xor32_maxf(xor16_maxf(mx));
    mx = fmaxf(mx, 1e-12f);
    const float qs = mx / 16383.0f;            // correctly rounded divides
    const float inv = 16383.0f / mx;
    const bool lo_limb = n & 1;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 4 * wi + j;
                const uint32_t wv = qw[t][e >> 1];
                const float fv = (e & 1) ? bf16hi(wv) : bf16lo(wv);
                // qi = rint(q / qs) clamped to +-16383, hi = rint(qi / 128) clamped to
                // +-127, lo = qi - 128 hi: small integers, exact in fp32, so the limbs are
                // formed without integer round trips and converted once
                const float qf = __builtin_amdgcn_fmed3f(rintf(__fmul_rn(fv, inv)), -16383.0f,
                                                         16383.0f);
                const float hf = __builtin_amdgcn_fmed3f(rintf(qf * 0.0078125f), -127.0f, 127.0f);
                const int v = (int)(lo_limb ? fmaf(-128.0f, hf, qf) : hf);
                word |= ((uint32_t)(v & 0xFF)) << (8 * j);
            }
            qa[t][wi] = (int)word;
        }
    }
    return qs;
}

// Workgroups per CU that kernel `k` keeps resident at `threads` per workgroup (queried
// once per kernel and workgroup size; falls back to one per CU on 256 CUs).
static inline int resident_per_cu(const void* k, int threads, int& cus) {
    struct Entry { const void* k; int threads, per_cu; };
    static Entry cache[64];
    static int n_cache = 0;
    static int cached_cus = 0;
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n_cache; ++i)
        if (cache[i].k == k && cache[i].threads == threads) {
            cus = cached_cus;
            return cache[i].per_cu;
        }
    int dev = 0, per_cu = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, threads, 0) != hipSuccess ||
        per_cu < 1) {
        cus = 256;
        return 1;
    }
    cached_cus = ncu;
    if (n_cache < 64) cache[n_cache++] = Entry{k, threads, per_cu};
    cus = ncu;
    return per_cu;
}

// kv heads (waves) per workgroup: min(n_kv, 8), so the heads of one block are read by one
// CU together, or 4 when that keeps more waves resident per CU (a kernel above 128 VGPRs
// fits one 8-wave workgroup per CU but three 4-wave ones).  Returns the heads per
// workgroup and the resident workgroups per CU for it.
static inline int pick_heads(const void* k, int n_kv, int& per_cu, int& cus) {
    int hw = n_kv < 8 ? n_kv : 8;
    per_cu = resident_per_cu(k, hw * 64, cus);
    if (hw == 8 && n_kv % 4 == 0) {
        int cus4 = 0;
        const int per4 = resident_per_cu(k, 4 * 64, cus4);
        if (per4 * 4 > per_cu * 8) {
            hw = 4;
            per_cu = per4;
            cus = cus4;
        }
    }
    return hw;
}

// Chunks per head group: one per resident workgroup slot (a chunk runs alone on its CU
// slot, so equal chunks finish together).
static inline int score_target(int resident, int head_groups) {
    const int t = resident / (head_groups > 0 ? head_groups : 1);
    return t < 1 ? 1 : t;
}

// ---- balanced split of a (ragged) batch's page tiles over the grid ---------------------
// Request r has tiles_r = ceil(n_sel_hi[r] / 16) tiles.  At tpw tiles per workgroup it takes
// n_r = ceil(tiles_r / tpw) workgroups, numbered consecutively over the batch, and its
// workgroup j walks tiles j, j + n_r, j + 2 n_r, ... (a uniform batch is the plain strided
// split).  tpw is the smallest value >= ceil(T / target) whose total sum n_r fits `target`
// (a binary search, skipped when the first value fits): `target` is what stays resident
// at once, so every workgroup starts in the first round and the launch takes tpw tile
// steps.  (With tpw = ceil(T / target) alone, the per-request rounding can push sum n_r
// past the resident slots on a ragged batch; the surplus workgroups then run as a second
// round and the launch takes up to twice as long.)  Nothing depends on host-side
// knowledge of the lengths (the launch stays graph-capturable); the grid is target + n_req
// workgroups, an upper bound of sum n_r, and workgroups past the last one exit at once.
struct TileWalk {
    int req;       // request
    int first;     // first tile
    int stride;    // tile stride (workgroups of the request)
    int count;     // tiles walked
    int nsh;       // the request's n_sel_hi (from the walk's own loads; <= the row width)
};

__device__ __forceinline__ int tiles_of(int nsh) {
    return nsh > 0 ? (nsh + SC_TILE - 1) / SC_TILE : 0;
}

// scored pages of request r: n_sel_hi, at most the rows' width mp (the score rows are mp
// pages wide whatever lengths a caller passes)
__device__ __forceinline__ int scored_of(const int32_t* nsh, int r, int mp) {
    return min(nsh[r], mp);
}

// tiles of requests base + lane (0 past the batch)
__device__ __forceinline__ int lane_tiles(const int32_t* nsh, int n_req, int mp, int base) {
    const int r = base + (threadIdx.x & 63);
    return r < n_req ? tiles_of(scored_of(nsh, r, mp)) : 0;
}

// workgroups the batch takes at tpw tiles per workgroup (every lane gets the sum);
// t0 = lane_tiles(0)
__device__ __forceinline__ int walk_total(const int32_t* nsh, int n_req, int mp, int t0,
                                          int tpw) {
    int tot = wave_sum_uniform((t0 + tpw - 1) / tpw);
    for (int base = WAVE; base < n_req; base += WAVE)
        tot += wave_sum_uniform((lane_tiles(nsh, n_req, mp, base) + tpw - 1) / tpw);
    return tot;
}

__device__ __forceinline__ int walk_tpw(const int32_t* nsh, int n_req, int mp, int target,
                                        int t0) {
    int total = wave_sum_uniform(t0), tmax = wave_max_uniform(t0);
    for (int base = WAVE; base < n_req; base += WAVE) {
        const int t = lane_tiles(nsh, n_req, mp, base);
        total += wave_sum_uniform(t);
        tmax = max(tmax, wave_max_uniform(t));
    }
    if (total <= 0) return 1;
    int lo = (total + target - 1) / target;
    if (walk_total(nsh, n_req, mp, t0, lo) <= target) return lo;
    int hi = max(lo, tmax);                 // at hi every request takes one workgroup
    ++lo;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (walk_total(nsh, n_req, mp, t0, mid) <= target) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

__device__ __forceinline__ bool tile_walk(const int32_t* nsh, int n_req, int mp, int target,
                                          int x, TileWalk& w) {
    const int lane = threadIdx.x & 63;
    const int v0 = lane < n_req ? scored_of(nsh, lane, mp) : 0;
    const int t0 = tiles_of(v0);
    const int tpw = walk_tpw(nsh, n_req, mp, target, t0);
    int before = 0;                                     // workgroups of earlier batches
    for (int base = 0; base < n_req; base += WAVE) {
        const int v = base == 0 ? v0 : (base + lane < n_req ? scored_of(nsh, base + lane, mp) : 0);
        const int t = tiles_of(v);
        const int nw = (t + tpw - 1) / tpw;
        const int incl = wave_incl_scan(nw);
        const int in_batch = __builtin_amdgcn_readlane(incl, WAVE - 1);
        if (x < before + in_batch) {
            const unsigned long long hit = __ballot(before + incl > x);
            const int src = __ffsll((long long)hit) - 1;
            const int excl = __builtin_amdgcn_readlane(incl - nw, src);
            const int tr = __builtin_amdgcn_readlane(t, src);
            w.req = base + src;
            w.nsh = __builtin_amdgcn_readlane(v, src);
            w.stride = __builtin_amdgcn_readlane(nw, src);
            w.first = x - before - excl;
            w.count = (tr - w.first + w.stride - 1) / w.stride;
            return true;
        }
        before += in_batch;
    }
    return false;
}

}  // namespace amass
