// runtime.hpp -- the objects behind the C ABI's opaque handles.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "kernels.hpp"
#include "tsr_hip.h"

namespace tsr {
int hip_err(hipError_t e, const char * what);
}
void tsr_expk_table(tsr::ExpkTab * t);

// Device scratch owned by a context (FA partials, the isums y sink). It only grows; growing waits
// for the context's stream first, so no queued kernel still uses the old block.
struct tsr_scratch {
    void * ptr = nullptr;
    size_t bytes = 0;
    template <class Ctx>
    int reserve(Ctx * ctx, size_t need) {
        if (need <= bytes) return TSR_HIP_OK;
        (void)ctx;
        (void)hipDeviceSynchronize();             // no stream may still use the old block
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
        const size_t n = (need + (1u << 20) - 1u) & ~(size_t)((1u << 20) - 1u);
        const int rc = tsr::hip_err(hipMalloc(&ptr, n), "hipMalloc scratch");
        if (rc == 0) bytes = n;
        return rc;
    }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

struct tsr_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mtx;
    int n_cu = 0;
    char name[128] = {0};
    tsr_hip_counters ctr{};
    tsr_scratch scratch;
    tsr::ExpkTab expk{};
    hipStream_t pick(void * s) const { return s ? (hipStream_t)s : stream; }
};

struct tsr_hip_weight {
    uint32_t fmt = 0, N = 0, K = 0;
    uint8_t * dev = nullptr;     // meta region at 0, quant region at quant_off
    size_t quant_off = 0;
    size_t bytes = 0;
};

// A q8_0 KV cache plane in the device layout: cell-major rows; per row the E/32 fp16 scales
// ("meta", padded to 16 bytes) and the E int8 quants, in separate regions.
struct tsr_hip_kv {
    uint32_t E = 0, kv_size = 0;
    uint8_t * dev = nullptr;
    size_t meta_row = 0;         // bytes per cell of the meta region
    size_t quant_off = 0;        // byte offset of the quant region
    size_t bytes = 0;
};
