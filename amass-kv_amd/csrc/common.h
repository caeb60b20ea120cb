// Device helpers shared by the gfx950 kernels of the AMASS hot path.
//
// Wave64 throughout: a "unit" of 8 lanes (one DPP half-row) cooperates on one
// (page, kv-head) record in the score kernels; full-wave reductions use DPP inside
// rows of 16 lanes and ds_swizzle/bpermute across rows.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/amass_hip.h"

namespace amass {

typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// ---------------------------------------------------------------- 16-bit floats
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}
// lower / upper bf16 of a packed dword
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> bf16 round-to-nearest-even (finite inputs; NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFF) ? 0x40 : 0));
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

__device__ __forceinline__ float fp16_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// ---------------------------------------------------------------- DPP lane moves
// quad_perm [1,0,3,2] (xor 1), [2,3,0,1] (xor 2); row_half_mirror pairs lane i with
// 7-i inside each group of 8 -- a valid first butterfly stage of an 8-lane reduction.
constexpr int DPP_XOR1 = 0xB1;
constexpr int DPP_XOR2 = 0x4E;
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// sum / max over the 8 lanes of a unit (lanes 8u..8u+7); every lane gets the result
__device__ __forceinline__ int unit8_sum(int v) {
    v += dpp_i<DPP_HALF_MIRROR>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_XOR1>(v);
    return v;
}
__device__ __forceinline__ float unit8_maxf(float v) {
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    return v;
}

// Wave-uniform int sum / max and inclusive scan with DPP inside rows of 16 lanes and
// readlane across the 4 rows: no LDS round trips (the shuffle forms below each take one
// per step).  All 64 lanes must be active.
constexpr int DPP_ROW_SHR1 = 0x111;
constexpr int DPP_ROW_SHR2 = 0x112;
constexpr int DPP_ROW_SHR4 = 0x114;
constexpr int DPP_ROW_SHR8 = 0x118;

__device__ __forceinline__ int row16_sum(int v) {   // every lane: sum of its row
    v += dpp_i<DPP_HALF_MIRROR>(v);
    v += dpp_i<DPP_XOR2>(v);
    v += dpp_i<DPP_XOR1>(v);
    v += dpp_i<DPP_ROW_MIRROR>(v);
    return v;
}
__device__ __forceinline__ int wave_sum_uniform(int v) {
    v = row16_sum(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
           __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ int wave_max_uniform(int v) {
    v = max(v, dpp_i<DPP_HALF_MIRROR>(v));
    v = max(v, dpp_i<DPP_XOR2>(v));
    v = max(v, dpp_i<DPP_XOR1>(v));
    v = max(v, dpp_i<DPP_ROW_MIRROR>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
// inclusive prefix sum over the lanes (row_shr steps leave 0 where the source is outside
// the row)
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += dpp_i<DPP_ROW_SHR1>(v);
    v += dpp_i<DPP_ROW_SHR2>(v);
    v += dpp_i<DPP_ROW_SHR4>(v);
    v += dpp_i<DPP_ROW_SHR8>(v);
    const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
              r2 = __builtin_amdgcn_readlane(v, 47);
    const int row = (threadIdx.x & 63) >> 4;
    return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// Wave-uniform reductions and an inclusive scan of other types, the same DPP row steps
// and readlane across rows (every lane gets the result).  All 64 lanes must be active.
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_maxf_uniform(float v) {
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
                 fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)dpp_i<CTRL>((int)v);
}
__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint32_t wave_minu_uniform(uint32_t v) {
    v = min(v, dpp_u<DPP_HALF_MIRROR>(v));
    v = min(v, dpp_u<DPP_XOR2>(v));
    v = min(v, dpp_u<DPP_XOR1>(v));
    v = min(v, dpp_u<DPP_ROW_MIRROR>(v));
    return min(min(readlane_u(v, 0), readlane_u(v, 16)), min(readlane_u(v, 32), readlane_u(v, 48)));
}
__device__ __forceinline__ uint32_t wave_maxu_uniform(uint32_t v) {
    v = max(v, dpp_u<DPP_HALF_MIRROR>(v));
    v = max(v, dpp_u<DPP_XOR2>(v));
    v = max(v, dpp_u<DPP_XOR1>(v));
    v = max(v, dpp_u<DPP_ROW_MIRROR>(v));
    return max(max(readlane_u(v, 0), readlane_u(v, 16)), max(readlane_u(v, 32), readlane_u(v, 48)));
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    const uint32_t lo = dpp_u<CTRL>((uint32_t)v), hi = dpp_u<CTRL>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long v, int l) {
    return ((unsigned long long)readlane_u((uint32_t)(v >> 32), l) << 32) |
           readlane_u((uint32_t)v, l);
}
__device__ __forceinline__ unsigned long long wave_sum_u64_uniform(unsigned long long v) {
    v += dpp_u64<DPP_HALF_MIRROR>(v);
    v += dpp_u64<DPP_XOR2>(v);
    v += dpp_u64<DPP_XOR1>(v);
    v += dpp_u64<DPP_ROW_MIRROR>(v);
    return (readlane_u64(v, 0) + readlane_u64(v, 16)) + (readlane_u64(v, 32) + readlane_u64(v, 48));
}
__device__ __forceinline__ unsigned long long wave_incl_scan_u64(unsigned long long v) {
    v += dpp_u64<DPP_ROW_SHR1>(v);
    v += dpp_u64<DPP_ROW_SHR2>(v);
    v += dpp_u64<DPP_ROW_SHR4>(v);
    v += dpp_u64<DPP_ROW_SHR8>(v);
    const unsigned long long r0 = readlane_u64(v, 15), r1 = readlane_u64(v, 31),
                             r2 = readlane_u64(v, 47);
    const int row = (threadIdx.x & 63) >> 4;
    return v + (row >= 1 ? r0 : 0ull) + (row >= 2 ? r1 : 0ull) + (row >= 3 ? r2 : 0ull);
}

// Lane pairs l, l^16 and l, l^32 through the gfx950 permlane swaps (no LDS round trip):
// with both operands v, permlane16_swap returns (v[l], v[l^16]) up to order and
// permlane32_swap (v[l], v[l^32]); max and sum are symmetric in the pair.
__device__ __forceinline__ float xor16_maxf(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor32_maxf(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor16_sumf(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor32_sumf(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// max over the 16 lanes of a row (every lane of the row gets it); all lanes active
__device__ __forceinline__ float row16_maxf(float v) {
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return v;
}
// v[l ^ 32] (the upper half reads the lower one's value and vice versa)
__device__ __forceinline__ float xor32_f(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? p[0] : p[1]);
}

// full-wave reductions (result in every lane)
__device__ __forceinline__ float wave_maxf(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}
__device__ __forceinline__ float wave_sumf(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ int wave_sumi(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ int wave_maxi(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, WAVE));
    return v;
}
__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// ---------------------------------------------------------------- byte transposes
// perm(a, b, sel): result byte i = byte sel_i of the 8-byte value {a:b} (b = bytes 0-3).
__device__ __forceinline__ uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
    return __builtin_amdgcn_perm(a, b, sel);
}
// 4x4 byte transpose: y_k = (x0.b_k, x1.b_k, x2.b_k, x3.b_k)
__device__ __forceinline__ void transpose4x4(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                             uint32_t& y0, uint32_t& y1, uint32_t& y2,
                                             uint32_t& y3) {
    const uint32_t t0 = perm(x1, x0, 0x05010400u);  // x0.b0 x1.b0 x0.b1 x1.b1
    const uint32_t t1 = perm(x1, x0, 0x07030602u);  // x0.b2 x1.b2 x0.b3 x1.b3
    const uint32_t t2 = perm(x3, x2, 0x05010400u);
    const uint32_t t3 = perm(x3, x2, 0x07030602u);
    y0 = perm(t2, t0, 0x05040100u);
    y1 = perm(t2, t0, 0x07060302u);
    y2 = perm(t3, t1, 0x05040100u);
    y3 = perm(t3, t1, 0x07060302u);
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---------------------------------------------------------------- order keys
// fp32 -> order-preserving uint32 (ascending float order == ascending uint order).
// -0.0 maps to the key of +0.0: the two compare equal, so they tie (lower index wins).
__device__ __forceinline__ uint32_t f2u(float f) {
    uint32_t u = __float_as_uint(f);
    u = (u == 0x80000000u) ? 0u : u;
    uint32_t mask = (uint32_t)(-(int32_t)(u >> 31)) | 0x80000000u;
    return u ^ mask;
}
__device__ __forceinline__ float u2f(uint32_t x) {
    uint32_t mask = ((x >> 31) - 1u) | 0x80000000u;
    return __uint_as_float(x ^ mask);
}

// ---------------------------------------------------------------- deterministic exp
// exp(x) for x <= 0 built only from correctly rounded fp32 +,-,*, rint and ldexp, so the
// host oracle reproduces it bit for bit.  Cody-Waite reduction by ln2 (hi part has 16
// trailing zero bits so n*hi is exact), degree-7 Taylor on |r| <= ln2/2, ldexp back.
// x <= -80 returns 0 (far below the 2^-32 mass quantum).  HIP compiles with FMA
// contraction on (and its __fmul_rn / __fadd_rn are plain * and +, fused like any
// other): the pragma keeps every product and sum below separately rounded.
__device__ __forceinline__ float exp_det(float x) {
#pragma clang fp contract(off)
    if (!(x > -80.0f)) return 0.0f;
    const float n = rintf(x * 0x1.715476p+0f);
    const float r = (x - n * 0x1.62e400p-1f) - n * 0x1.7f7d1cp-20f;
    float p = 0x1.a01a02p-13f;           // 1/5040
    p = p * r + 0x1.6c16c2p-10f;         // 1/720
    p = p * r + 0x1.111112p-7f;          // 1/120
    p = p * r + 0x1.555556p-5f;          // 1/24
    p = p * r + 0x1.555556p-3f;          // 1/6
    p = p * r + 0x1.000000p-1f;          // 1/2
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)n);
}

// page mass in 2^-32 fixed point (see amass_select_args)
__device__ __forceinline__ unsigned long long mass_q(float score, float smax, int kind) {
    float w;
    if (kind == 0) {
        w = exp_det(__fsub_rn(score, smax));
    } else {
        w = fminf(fmaxf(score, 0.0f), 1024.0f);
        if (!(w == w)) w = 0.0f;
    }
    return (unsigned long long)(__fmul_rn(w, 4294967296.0f));
}

// ---------------------------------------------------------------- cross-workgroup tickets
// Whether this workgroup is the last of `n` to arrive at the int32 ticket *t (every thread
// gets the answer; call it from every thread of the workgroup).  Every wave first waits
// until its global stores have reached the L2 (a vector store leaves the counter once the
// write-through L1 has passed it on), the barrier gathers the waves, and thread 0 releases
// the workgroup's stores device-wide (an agent-scope fence: a write-back of the XCD's L2)
// before it takes the ticket.  The last arrival resets the ticket to zero, so every launch
// leaves it as it found it, and acquires the other workgroups' stores (an agent-scope
// fence: an invalidate of this CU's L1 and the XCD's L2) before the barrier lets its waves
// read them.  One fence per workgroup, not per wave: the L2 write-back and invalidate are
// whole-cache actions.  No workgroup ever waits for another.
__device__ __forceinline__ bool last_arrival(int32_t* t, int n) {
    __shared__ int last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        last = atomicAdd(t, 1) == n - 1;
        if (last) {
            atomicExch(t, 0);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
    return last;
}

}  // namespace amass

// status bookkeeping shared by the host wrappers
namespace amass {
int record_hip(hipError_t e);
int check_launch();
}  // namespace amass
