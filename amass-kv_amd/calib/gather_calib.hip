// HBM-counter calibration kernel (measurement only; not part of the hot path's C ABI).
//
// Reads every (block, kv head) K and V slice of a paged bf16 KV cache once, in the order
// of a block list, with exactly the decode kernel's access pattern: per (page, head) one
// wave issues 4 K and 4 V 16-byte non-temporal loads per lane (K: token lane%16, bytes
// 16*(lane/16) + 64*i of its 256-byte row; V: tokens 4*(lane/16) + u, bytes
// 16*(lane%16)), four waves of a workgroup taking four heads of the same blocks.  The
// loaded words are XOR-folded into one 32-bit word per wave, so the kernel's algorithmic
// traffic is exact: n_blocks * n_kv * 2 * page * d * 2 bytes read + 4 bytes per block-list
// entry, and 4 bytes written per wave.  Profiling it beside the hot path gives the factor
// between rocprofv3's FETCH_SIZE and the bytes this access pattern really moves.
//
// Built into libamass_calib.so (separate from libamass_hip.so).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace amass_calib {

constexpr int WAVE = 64;
constexpr int PAGE = 16;      // tokens per page
constexpr int D = 128;        // head dim (bf16)
constexpr int PPW = 16;       // pages per wave

__device__ __forceinline__ uint4 ld_nt(const uint16_t* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u x = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(x[0], x[1], x[2], x[3]);
}

__device__ __forceinline__ uint32_t fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

__global__ void __launch_bounds__(256)
gather_calib_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                    int64_t k_sb, int64_t k_st, int64_t k_sh, int64_t v_sb, int64_t v_st,
                    int64_t v_sh, const int32_t* __restrict__ blocks, int n_blocks, int n_kv,
                    uint32_t* __restrict__ out) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int kh = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (kh >= n_kv) return;
    const int j0 = blockIdx.x * PPW;
    const int n = min(PPW, n_blocks - j0);
    const int blk_l = lane < n ? blocks[j0 + lane] : 0;
    const uint16_t* kl = k + (int64_t)kh * k_sh + (int64_t)(lane & 15) * k_st + 8 * (lane >> 4);
    const uint16_t* vl = v + (int64_t)kh * v_sh + (int64_t)(4 * (lane >> 4)) * v_st +
                         8 * (lane & 15);
    uint32_t acc = 0;
    int i = 0;
    for (; i + 1 < n; i += 2) {       // two pages' loads in flight per wave
        const int64_t b0 = (int64_t)__builtin_amdgcn_readlane(blk_l, i);
        const int64_t b1 = (int64_t)__builtin_amdgcn_readlane(blk_l, i + 1);
        uint4 x[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            x[u] = ld_nt(kl + b0 * k_sb + 32 * u);
            x[4 + u] = ld_nt(vl + b0 * v_sb + (int64_t)u * v_st);
            x[8 + u] = ld_nt(kl + b1 * k_sb + 32 * u);
            x[12 + u] = ld_nt(vl + b1 * v_sb + (int64_t)u * v_st);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) acc ^= fold(x[u]);
    }
    if (i < n) {
        const int64_t b0 = (int64_t)__builtin_amdgcn_readlane(blk_l, i);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            acc ^= fold(ld_nt(kl + b0 * k_sb + 32 * u));
            acc ^= fold(ld_nt(vl + b0 * v_sb + (int64_t)u * v_st));
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, WAVE);
    if (lane == 0) out[(int64_t)kh * gridDim.x + blockIdx.x] = acc;
}

}  // namespace amass_calib

// Returns 0, or -1 for arguments the kernel does not take (the launch is not issued), or
// -2 when the launch fails.  `out` holds ceil(n_blocks / 16) * n_kv words; every block id
// in `blocks` must index the cache (the host checks this before calling).
extern "C" int amass_calib_gather(const void* k, const void* v, int64_t k_sb, int64_t k_st,
                                  int64_t k_sh, int64_t v_sb, int64_t v_st, int64_t v_sh,
                                  const int32_t* blocks, int32_t n_blocks, int32_t n_kv,
                                  uint32_t* out, hipStream_t stream) {
    using namespace amass_calib;
    if (!k || !v || !blocks || !out || n_blocks <= 0 || n_kv <= 0) return -1;
    if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) return -1;
    if ((k_sb | k_st | k_sh | v_sb | v_st | v_sh) & 7) return -1;
    const dim3 grid((n_blocks + PPW - 1) / PPW, (n_kv + 3) / 4);
    hipLaunchKernelGGL(gather_calib_kernel, grid, dim3(256), 0, stream,
                       (const uint16_t*)k, (const uint16_t*)v, k_sb, k_st, k_sh, v_sb, v_st,
                       v_sh, blocks, n_blocks, n_kv, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
