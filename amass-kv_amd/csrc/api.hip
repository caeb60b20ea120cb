// Host-side entry points of libamass_hip.so that launch no kernel: status bookkeeping,
// the pinned device-mapped host pool, copy-engine runs and ABI introspection.
#include <atomic>

#include "common.h"

namespace amass {

static std::atomic<int> g_last_hip{0};

int record_hip(hipError_t e) {
    if (e != hipSuccess) {
        g_last_hip.store((int)e);
        return AMASS_ERR_HIP;
    }
    return AMASS_OK;
}

int check_launch() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_last_hip.store((int)e);
        return AMASS_ERR_LAUNCH;
    }
    return AMASS_OK;
}

}  // namespace amass

using namespace amass;

extern "C" int amass_abi_version(void) { return AMASS_ABI_VERSION; }

extern "C" size_t amass_abi_struct_size(int which) {
    switch (which) {
        case 0: return sizeof(amass_quad_score_args);
        case 1: return sizeof(amass_r8_score_args);
        case 2: return sizeof(amass_derive_args);
        case 3: return sizeof(amass_nrm_args);
        case 4: return sizeof(amass_select_args);
        case 5: return sizeof(amass_decode_args);
        case 6: return sizeof(amass_tier_plan_args);
        case 7: return sizeof(amass_tier_fetch_args);
        case 8: return sizeof(amass_copy_run);
        case 9: return sizeof(amass_build_args);
        case 10: return sizeof(amass_clse_score_args);
        case 11: return sizeof(amass_invalidate_args);
        case 12: return sizeof(amass_stage_args);
        case 13: return sizeof(amass_scatter_args);
        default: return 0;
    }
}

extern "C" const char* amass_status_string(int status) {
    switch (status) {
        case AMASS_OK: return "ok";
        case AMASS_ERR_NULL: return "required pointer is NULL";
        case AMASS_ERR_GEOMETRY: return "unsupported or inconsistent geometry";
        case AMASS_ERR_UNSUPPORTED: return "configuration not implemented";
        case AMASS_ERR_LAUNCH: return "kernel launch failed";
        case AMASS_ERR_HIP: return "HIP runtime error";
        case AMASS_ERR_CAPACITY: return "fixed capacity exceeded";
        default: return "unknown status";
    }
}

extern "C" int amass_last_hip_error(void) { return g_last_hip.load(); }

extern "C" int amass_host_pool_alloc(size_t bytes, void** host_ptr, void** dev_ptr) {
    if (!host_ptr || !dev_ptr) return AMASS_ERR_NULL;
    *host_ptr = nullptr;
    *dev_ptr = nullptr;
    if (bytes == 0) return AMASS_ERR_GEOMETRY;
    void* h = nullptr;
    int rc = record_hip(hipHostMalloc(&h, bytes, hipHostMallocMapped));
    if (rc) return rc;
    void* d = nullptr;
    rc = record_hip(hipHostGetDevicePointer(&d, h, 0));
    if (rc) {
        (void)hipHostFree(h);
        return rc;
    }
    *host_ptr = h;
    *dev_ptr = d;
    return AMASS_OK;
}

extern "C" int amass_host_pool_free(void* host_ptr) {
    if (!host_ptr) return AMASS_ERR_NULL;
    return record_hip(hipHostFree(host_ptr));
}

extern "C" int amass_tier_dma(const amass_copy_run* runs, int32_t n, void* stream) {
    if (n < 0) return AMASS_ERR_GEOMETRY;
    if (n > 0 && !runs) return AMASS_ERR_NULL;
    // every run is checked before the first copy is issued
    for (int32_t i = 0; i < n; ++i) {
        const amass_copy_run& c = runs[i];
        if (!c.dst || !c.src || c.width <= 0 || c.height <= 0) return AMASS_ERR_GEOMETRY;
        if (c.height > 1 && (c.dpitch < c.width || c.spitch < c.width)) return AMASS_ERR_GEOMETRY;
    }
    hipStream_t s = (hipStream_t)stream;
    for (int32_t i = 0; i < n; ++i) {
        const amass_copy_run& c = runs[i];
        int rc;
        if (c.height == 1)
            rc = record_hip(hipMemcpyAsync(c.dst, c.src, (size_t)c.width, hipMemcpyHostToDevice, s));
        else
            rc = record_hip(hipMemcpy2DAsync(c.dst, (size_t)c.dpitch, c.src, (size_t)c.spitch,
                                             (size_t)c.width, (size_t)c.height,
                                             hipMemcpyHostToDevice, s));
        if (rc) return rc;
    }
    return AMASS_OK;
}
