// Page-summary builder for gfx950: the quad and r8 summaries of finalised K pages.
//
// Math per (block, kv-head) of a 16-token page (reference selection/quad_build.py:1-25,
// 124-198 and selection/build.py:297-348,396-412):
//   mu  = mean_t K[t]                       dc = K - mu            (16, d) fp32
//   Gm  = dc dc^T (16 x 16)                 S2, U = eigh(Gm), eigenvalues ascending
//   S2r = clamp(top-r eigenvalues, 1e-10)   U8 = their eigenvectors, S8 = sqrt(S2r)
//   Vk  = dc^T U8 / S8 (d, r)               c = U8 * S8 (16, r)    (r8 only)
//   quant: lvl = 127 | 7, s = max(amax / lvl, 1e-8) fp32, code = clamp(rint(x / s), +-lvl),
//          stored scale fp16(s); mu per (block, head), Vk per column ("col") or per
//          (block, head) ("tensor"), c per token ("page") or per (block, head) ("tensor")
//   quad stores sig2 = fp16(S2r); r8 stores c; both the content tag K[15][:TAGW].
// Output goes straight into the packed records the score kernels read
// (AMASS_QUAD_REC_BYTES / AMASS_R8_REC_BYTES / AMASS_CLSE_REC_BYTES).
//
// One wave per (block, kv-head, layer), one wave per workgroup (the Jacobi rounds'
// barriers then wait for no other wave).  The K page is staged in LDS as
// fp32; the Gram is 32 v_mfma_f32_16x16x4f32 whose A and B operands are the same
// register (lane (kg, t) holds dc[t][32 kg + c] for K-step c -- any split of d over the
// K steps gives the same sum).  The eigenproblem is solved by parallel (round-robin)
// Jacobi in LDS: per round, 8 disjoint (p, q) pairs, their rotations computed by 8
// lanes, then A <- A J, V <- V J and A <- J^T A, each one update per lane and element
// pair.  Sweeps stop once every wave's off-diagonal mass is below 1e-12 of the diagonal
// mass (at most 16 sweeps, the reference's count), a workgroup-uniform decision.
#include "common.h"

namespace amass {

constexpr int BP = 16;           // tokens per page
constexpr int BD = 128;          // head dim
constexpr int BW = 1;            // waves (kv heads) per workgroup
constexpr int BSWEEPS = 16;
constexpr int BKP = BD + 1;      // padded fp32 row of the K tile
constexpr int BAP = BP + 1;      // padded row of A / V

typedef float f32x4v __attribute__((ext_vector_type(4)));

struct BuildLds {
    float k[BW][BP][BKP];        // K, then dc
    float a[BW][BP][BAP];        // Jacobi matrix
    float v[BW][BP][BAP];        // eigenvectors (columns)
    float cs[BW][8], sn[BW][8];  // this round's rotations
    int pp[BW][8], qq[BW][8];
    int idx[BW][8];              // eigen-index of output column k (ascending eigenvalue)
    float s2[BW][8];             // clamped eigenvalue of output column k
    int conv[BW];
};

// circle-method pairing of 16 indices: round r in [0, 15), pair i in [0, 8)
__device__ __forceinline__ void round_pair(int r, int i, int& p, int& q) {
    int a, b;
    if (i == 0) {
        a = 15;
        b = r;
    } else {
        a = r + i;
        a = a >= 15 ? a - 15 : a;
        b = r - i;
        b = b < 0 ? b + 15 : b;
    }
    p = a < b ? a : b;
    q = a < b ? b : a;
}

__device__ __forceinline__ float quant_scale(float amax, float lvl) {
    return fmaxf(__fdiv_rn(amax, lvl), 1e-8f);
}
__device__ __forceinline__ int quant_code(float x, float s, float lvl) {
    return (int)fminf(fmaxf(rintf(__fdiv_rn(x, s)), -lvl), lvl);
}
__device__ __forceinline__ uint16_t f2h_bits(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// KIND 0: quad record; 1: r8 record; 2: CLSE (the r8 record + the residual energy)
template <int KIND>
__global__ __launch_bounds__(BW * WAVE) void summary_build_kernel(const amass_build_args a) {
    constexpr bool R8 = KIND >= 1;
    constexpr bool CLSE = KIND == 2;
    __shared__ BuildLds L;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int h = blockIdx.y * nw + w;
    const int64_t blk = a.blocks[blockIdx.x];
    const int r = a.rank;
    const int layer = blockIdx.z;
    const void* kbase = a.k_layers ? (const void*)a.k_layers[layer] : a.k;

    // ---- K page -> LDS (fp32), content tag ---------------------------------------------
    const uint16_t* kp = (const uint16_t*)kbase + blk * a.k_sb + (int64_t)h * a.k_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int chunk = lane + 64 * i;            // 256 chunks of 8 bf16
        const int t = chunk >> 4, d0 = 8 * (chunk & 15);
        const uint4 x = *reinterpret_cast<const uint4*>(kp + (int64_t)t * a.k_st + d0);
        const uint32_t wv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            L.k[w][t][d0 + 2 * j] = bf16lo(wv[j]);
            L.k[w][t][d0 + 2 * j + 1] = bf16hi(wv[j]);
        }
    }
    if (a.tag != nullptr && lane < a.tagw) {
        uint16_t* tg = (uint16_t*)a.tag + layer * a.tag_lsb + blk * a.tag_sb + (int64_t)h * a.tag_sh;
        tg[lane] = kp[(int64_t)(BP - 1) * a.k_st + lane];
    }
    __syncthreads();

    // ---- mu, dc ---------------------------------------------------------------------------
    float mu[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int d = lane + 64 * e;
        float s = 0.f;
#pragma unroll
        for (int t = 0; t < BP; ++t) s += L.k[w][t][d];
        mu[e] = s * (1.0f / BP);
#pragma unroll
        for (int t = 0; t < BP; ++t) L.k[w][t][d] -= mu[e];
    }
    __syncthreads();

    // ---- Gram on the matrix cores; V = I -------------------------------------------------
    {
        const int t = lane & 15, kg = lane >> 4;
        f32x4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int c = 0; c < 32; ++c) {
            const float x = L.k[w][t][32 * kg + c];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, x, acc, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            L.a[w][4 * kg + j][t] = acc[j];
            L.v[w][4 * kg + j][t] = (4 * kg + j == t) ? 1.f : 0.f;
        }
    }
    __syncthreads();
    // trace of the centred scatter (the sum of all eigenvalues), for CLSE's residual
    float trace = 0.f;
    if constexpr (CLSE) trace = wave_sumf(lane < BP ? L.a[w][lane][lane] : 0.f);

    // ---- parallel Jacobi ----------------------------------------------------------------
    for (int sweep = 0; sweep < BSWEEPS; ++sweep) {
        // convergence: off-diagonal vs diagonal mass of every wave's matrix
        {
            float off = 0.f, dg = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = (lane + 64 * e) >> 4, j = (lane + 64 * e) & 15;
                const float x = L.a[w][i][j];
                if (i == j) dg += x * x; else off += x * x;
            }
            off = wave_sumf(off);
            dg = wave_sumf(dg);
            if (lane == 0) L.conv[w] = off <= 1e-12f * dg;
            __syncthreads();
            int all = 1;
            for (int x = 0; x < nw; ++x) all &= L.conv[x];
            __syncthreads();
            if (all) break;
        }
        for (int rnd = 0; rnd < BP - 1; ++rnd) {
            if (lane < 8) {
                int p, q;
                round_pair(rnd, lane, p, q);
                const float apq = L.a[w][p][q];
                float c = 1.f, s = 0.f;
                if (fabsf(apq) > 1e-30f) {
                    const float theta = (L.a[w][q][q] - L.a[w][p][p]) / (2.f * apq);
                    const float tt = (theta >= 0.f ? 1.f : -1.f) /
                                     (fabsf(theta) + sqrtf(theta * theta + 1.f));
                    c = 1.f / sqrtf(tt * tt + 1.f);
                    s = tt * c;
                }
                L.pp[w][lane] = p;
                L.qq[w][lane] = q;
                L.cs[w][lane] = c;
                L.sn[w][lane] = s;
            }
            __syncthreads();
            // columns: A <- A J, V <- V J   (items: row k, pair i)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int it = lane + 64 * e, k = it & 15, i = it >> 4;
                const int p = L.pp[w][i], q = L.qq[w][i];
                const float c = L.cs[w][i], s = L.sn[w][i];
                const float akp = L.a[w][k][p], akq = L.a[w][k][q];
                L.a[w][k][p] = c * akp - s * akq;
                L.a[w][k][q] = s * akp + c * akq;
                const float vkp = L.v[w][k][p], vkq = L.v[w][k][q];
                L.v[w][k][p] = c * vkp - s * vkq;
                L.v[w][k][q] = s * vkp + c * vkq;
            }
            __syncthreads();
            // rows: A <- J^T A   (items: column k, pair i)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int it = lane + 64 * e, k = it & 15, i = it >> 4;
                const int p = L.pp[w][i], q = L.qq[w][i];
                const float c = L.cs[w][i], s = L.sn[w][i];
                const float apk = L.a[w][p][k], aqk = L.a[w][q][k];
                L.a[w][p][k] = c * apk - s * aqk;
                L.a[w][q][k] = s * apk + c * aqk;
            }
            __syncthreads();
        }
    }

    // ---- top-r eigenpairs, ascending among themselves ------------------------------------
    if (lane < BP) {
        const float li = L.a[w][lane][lane];
        int rank = 0;                                  // rank in descending order
        for (int j = 0; j < BP; ++j) {
            const float lj = L.a[w][j][j];
            rank += (lj > li) || (lj == li && j < lane);
        }
        if (rank < r) {
            const int k = r - 1 - rank;
            L.idx[w][k] = lane;
            L.s2[w][k] = fmaxf(li, 1e-10f);
        }
    }
    __syncthreads();

    // ---- record addressing ---------------------------------------------------------------
    // quad / r8: head h's record [V | mu (| c rows)] at h VM, its scale block (quad 48,
    // r8 64 bytes) at n_kv VM + TB h.  CLSE: [V | mu] at h VM, its tail of TB bytes
    // [c rows | scale part] at n_kv VM + TB h (AMASS_CLSE_REC_BYTES).
    const int CB = a.v_bits == 8 ? BD : BD / 2;
    const int crow = R8 ? r * a.c_bits / 8 : 0;
    const int VM = r * CB + BD + (CLSE ? 0 : 16 * crow);
    const int TB = CLSE ? 16 * crow + 16 * ((36 + 2 * r + 15) / 16) : (R8 ? 64 : 48);
    int8_t* lrec = a.rec + layer * a.rec_lsb + blk * a.rec_sb;
    int8_t* rec = lrec + (int64_t)h * VM;
    int8_t* tail = lrec + (int64_t)a.n_kv * VM + (int64_t)TB * h;
    int8_t* crows = CLSE ? tail : rec + r * CB + BD;
    uint16_t* meta = (uint16_t*)(CLSE ? tail + 16 * crow : tail);
    const float vlvl = a.v_bits == 8 ? 127.f : 7.f;

    // ---- Vk = dc^T U8 / S8, per-column (or per-head) int8 / int4 ----------------------
    float vk[2][8];
    float amx[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        amx[k] = 0.f;
        if (k < r) {
            const int col = L.idx[w][k];
            const float inv8 = 1.f / sqrtf(L.s2[w][k]);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int d = lane + 64 * e;
                float acc = 0.f;
#pragma unroll
                for (int t = 0; t < BP; ++t) acc += L.k[w][t][d] * L.v[w][t][col];
                vk[e][k] = acc * inv8;
            }
            amx[k] = wave_maxf(fmaxf(fabsf(vk[0][k]), fabsf(vk[1][k])));
        }
    }
    float vsc[8];
    if (a.v_grain == 1) {                               // one scale per (block, head)
        float m = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) m = k < r ? fmaxf(m, amx[k]) : m;
#pragma unroll
        for (int k = 0; k < 8; ++k) vsc[k] = quant_scale(m, vlvl);
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) vsc[k] = quant_scale(amx[k], vlvl);
    }
    // the tiled layout of the score kernels' column groups: 16 bytes per (K-step t, d
    // group kg, column k) at ((t * 4 + kg) * r + k) * 16 (int4: t folded into the nibbles)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (k < r) {
            const int c0 = quant_code(vk[0][k], vsc[k], vlvl);
            const int c1 = quant_code(vk[1][k], vsc[k], vlvl);
            const int o0 = ((lane >> 4) * r + k) * 16 + (lane & 15);
            if (a.v_bits == 8) {
                rec[o0] = (int8_t)c0;
                rec[o0 + 64 * r] = (int8_t)c1;
            } else {
                rec[o0] = (int8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
            }
        }
    }

    // ---- mu -------------------------------------------------------------------------------
    const float mamax = wave_maxf(fmaxf(fabsf(mu[0]), fabsf(mu[1])));
    const float msc = quant_scale(mamax, 127.f);
    rec[r * CB + lane] = (int8_t)quant_code(mu[0], msc, 127.f);
    rec[r * CB + lane + 64] = (int8_t)quant_code(mu[1], msc, 127.f);

    // ---- r8: c = U8 * S8 per token -------------------------------------------------------
    float csc_t = 0.f;                                  // this lane's token scale (r8)
    if constexpr (R8) {
        const float clvl = a.c_bits == 8 ? 127.f : 7.f;
        float cv[8];
        float m = 0.f;
        const int t = lane & 15;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            cv[k] = k < r ? L.v[w][t][L.idx[w][k]] * sqrtf(L.s2[w][k]) : 0.f;
            m = fmaxf(m, fabsf(cv[k]));
        }
        if (a.c_grain >= 1) {                           // one scale per (block, head)
            m = fmaxf(m, __shfl_xor(m, 1, WAVE));
            m = fmaxf(m, __shfl_xor(m, 2, WAVE));
            m = fmaxf(m, __shfl_xor(m, 4, WAVE));
            m = fmaxf(m, __shfl_xor(m, 8, WAVE));
        }
        csc_t = quant_scale(m, clvl);
        if (lane < BP) {
            int8_t* cr = crows + t * crow;
            if (a.c_bits == 8) {
                for (int k = 0; k < r; ++k) cr[k] = (int8_t)quant_code(cv[k], csc_t, clvl);
            } else {
                for (int k = 0; k < r; k += 2) {
                    const int lo = quant_code(cv[k], csc_t, clvl);
                    const int hi = quant_code(cv[k + 1], csc_t, clvl);
                    cr[k / 2] = (int8_t)((lo & 0xF) | ((hi & 0xF) << 4));
                }
            }
        }
    }

    // ---- the fp16 scale block (CLSE: the tail's scale part) ------------------------------
    const float cs_in = __shfl(csc_t, (lane - 8) & 63, WAVE);   // c_scale of token lane - 8
    const uint32_t cs_bits = __float_as_uint(__shfl(csc_t, 0, WAVE));  // c_grain 2: fp32
    if constexpr (CLSE) {
        // halves: c_scale of token lane (0..15), V_scale (16..16+r), mu_scale, the residual,
        // zero to the tail's end
        const float cs_t = __shfl(csc_t, lane & 15, WAVE);
        if (lane < (TB - 16 * crow) / 2) {
            float v = 0.f;
            if (lane < 16) v = cs_t;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (k < r && lane == 16 + k) v = vsc[k];
            if (lane == 16 + r) v = msc;
            if (lane == 17 + r) {
                float top = 0.f;
                for (int k = 0; k < r; ++k) top += L.s2[w][k];
                v = fmaxf(trace - top, 0.f);
            }
            meta[lane] = f2h_bits(v);
        }
        return;
    }
    if (lane < 32) {
        float v = 0.f;
        bool set = false;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (lane == k && k < r) { v = vsc[k]; set = true; }
        if constexpr (R8) {
            if (lane >= 8 && lane < 24 && a.c_grain != 2) { v = cs_in; set = true; }
            else if (lane == 24) { v = msc; set = true; }
        } else {
            if (lane >= 8 && lane < 8 + r) { v = L.s2[w][lane - 8]; set = true; }
            else if (lane == 16) { v = msc; set = true; }
        }
        uint16_t h = set ? f2h_bits(v) : (uint16_t)0;
        if constexpr (R8) {
            if (a.c_grain == 2 && (lane == 8 || lane == 9))   // the page's fp32 c scale
                h = (uint16_t)(lane == 8 ? (cs_bits & 0xFFFFu) : (cs_bits >> 16));
        }
        if (lane < TB / 2) meta[lane] = h;
    }
}

}  // namespace amass

using namespace amass;

extern "C" int amass_summary_build(const amass_build_args* a, void* stream) {
    if (!a) return AMASS_ERR_NULL;
    if ((!a->k && !a->k_layers) || !a->blocks || !a->rec) return AMASS_ERR_NULL;
    if (a->d != BD || a->page != BP || a->n < 0 || a->n_kv < 1) return AMASS_ERR_GEOMETRY;
    if (a->kind < 0 || a->kind > 2) return AMASS_ERR_GEOMETRY;
    if (a->rank < 1 || a->rank > 8) return AMASS_ERR_UNSUPPORTED;
    if (a->v_bits != 8 && a->v_bits != 4) return AMASS_ERR_GEOMETRY;
    if (a->kind >= 1 && a->c_bits != 8 && a->c_bits != 4) return AMASS_ERR_GEOMETRY;
    if (a->c_grain < 0 || a->c_grain > (a->kind == 1 ? 2 : 1)) return AMASS_ERR_GEOMETRY;
    if ((a->v_bits == 4 || (a->kind >= 1 && a->c_bits == 4)) && (a->rank & 1))
        return AMASS_ERR_GEOMETRY;
    if (a->tag && (a->tagw < 0 || a->tagw > 64)) return AMASS_ERR_GEOMETRY;
    const int nw = a->n_kv < BW ? a->n_kv : BW;
    if (a->n_kv % nw != 0) return AMASS_ERR_GEOMETRY;
    const int crow = a->kind >= 1 ? a->rank * a->c_bits / 8 : 0;
    const int vm = a->rank * (a->v_bits == 8 ? BD : BD / 2) + BD + 16 * crow;
    const int64_t rec_bytes = a->kind == 2 ? AMASS_CLSE_REC_BYTES(a->rank, a->v_bits, a->c_bits)
                              : (a->kind == 1 ? vm + 64 : AMASS_QUAD_REC_BYTES(a->rank, a->v_bits));
    if (a->rec_sb < (int64_t)a->n_kv * rec_bytes) return AMASS_ERR_GEOMETRY;
    if (a->n_layers < 1 || (a->n_layers > 1 && !a->k_layers)) return AMASS_ERR_GEOMETRY;
    if (a->n == 0) return AMASS_OK;
    const dim3 grid(a->n, a->n_kv / nw, a->n_layers), blk(nw * WAVE);
    hipStream_t s = (hipStream_t)stream;
    if (a->kind == 2)
        hipLaunchKernelGGL(summary_build_kernel<2>, grid, blk, 0, s, *a);
    else if (a->kind == 1)
        hipLaunchKernelGGL(summary_build_kernel<1>, grid, blk, 0, s, *a);
    else
        hipLaunchKernelGGL(summary_build_kernel<0>, grid, blk, 0, s, *a);
    return check_launch();
}
