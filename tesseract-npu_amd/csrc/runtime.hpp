// runtime.hpp -- the objects behind the C ABI's opaque handles.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>

#include "kernels.hpp"
#include "tsr_hip.h"

namespace tsr {
int hip_err(hipError_t e, const char * what);
}
void tsr_expk_table(tsr::ExpkTab * t);
struct tsr_hip_ctx;
// The fixed device array of tsr_hip_flash_attn_noalloc (bytes) and the lookup of its device address,
// made once per context with the context's device current.
constexpr size_t kFaNoAllocBytes = (size_t)16 << 20;
int tsr_fa_fixed_init(tsr_hip_ctx * ctx);

// Device scratch owned by a context (FA partials and work lists, prefill QA images, the isums y
// sink). It only grows. reserve() orders its users: a call on another stream than the previous
// user first waits (hipStreamWaitEvent) for the work queued on that stream, so two calls never use
// the block at once; growing waits for the whole device first, so no queued kernel still uses the
// old block. Under graph capture neither a growth nor a wait on another stream can be recorded:
// reserve() then fails with TSR_HIP_E_ARG (warm the context up outside the capture). A graph whose
// capture used the scratch holds its address: `gen` counts the reallocations, and a replay after one
// is refused (tsr_hip_graph_launch) instead of writing freed memory.
inline bool tsr_capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}
struct tsr_scratch {
    void * ptr = nullptr;
    size_t bytes = 0;
    hipStream_t last = nullptr;
    hipEvent_t ev = nullptr;
    uint64_t gen = 0;                            // reallocations so far
    bool captured = false;                       // a capture in progress used the block
    int reserve(size_t need, hipStream_t s) {
        if (tsr_capturing(s)) captured = true;
        if (last != nullptr && last != s) {
            if (tsr_capturing(s)) return TSR_HIP_E_ARG;
            if (ev == nullptr) {
                const int rc = tsr::hip_err(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate");
                if (rc) return rc;
            }
            int rc = tsr::hip_err(hipEventRecord(ev, last), "hipEventRecord");
            if (rc == 0) rc = tsr::hip_err(hipStreamWaitEvent(s, ev, 0), "hipStreamWaitEvent");
            if (rc) return rc;
        }
        last = s;
        if (need <= bytes) return TSR_HIP_OK;
        if (tsr_capturing(s)) return TSR_HIP_E_ARG;
        (void)hipDeviceSynchronize();             // no stream may still use the old block
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
        const size_t n = (need + (1u << 20) - 1u) & ~(size_t)((1u << 20) - 1u);
        ++gen;
        const int rc = tsr::hip_err(hipMalloc(&ptr, n), "hipMalloc scratch");
        if (rc == 0) bytes = n;
        return rc;
    }
    void release() {
        if (ptr) (void)hipFree(ptr);
        if (ev) (void)hipEventDestroy(ev);
        ptr = nullptr;
        ev = nullptr;
        bytes = 0;
        last = nullptr;
    }
};

// Pinned host staging for stream-ordered host-to-device copies whose source the caller may reuse at
// once: the bytes are copied into a slot at the call, and the device copy reads the slot. A slot is
// reused only after the copy that last read it has run (its event), so the host can run up to kSlots
// copies ahead of the device. Not usable under graph capture (a slot's contents change per call).
struct tsr_staging {
    static constexpr uint32_t kSlots = 64, kSlotBytes = 16384;
    uint8_t * host = nullptr;
    hipEvent_t ev[kSlots] = {};
    bool used[kSlots] = {};
    uint32_t next = 0;
    int copy(void * dst_dev, const void * src, size_t bytes, hipStream_t s) {
        if (bytes > kSlotBytes) return TSR_HIP_E_RANGE;
        if (host == nullptr) {
            int rc = tsr::hip_err(hipHostMalloc((void **)&host, (size_t)kSlots * kSlotBytes, hipHostMallocDefault),
                                  "hipHostMalloc staging");
            for (uint32_t i = 0; rc == 0 && i < kSlots; ++i)
                rc = tsr::hip_err(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming), "hipEventCreate");
            if (rc) { release(); return rc; }
        }
        const uint32_t k = next;
        next = (next + 1u) % kSlots;
        if (used[k]) {
            const int rc = tsr::hip_err(hipEventSynchronize(ev[k]), "hipEventSynchronize staging");
            if (rc) return rc;
        }
        uint8_t * slot = host + (size_t)k * kSlotBytes;
        memcpy(slot, src, bytes);
        int rc = tsr::hip_err(hipMemcpyAsync(dst_dev, slot, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync staging");
        if (rc == 0) rc = tsr::hip_err(hipEventRecord(ev[k], s), "hipEventRecord staging");
        used[k] = rc == 0;
        return rc;
    }
    void release() {
        for (uint32_t i = 0; i < kSlots; ++i) {
            if (ev[i]) (void)hipEventSynchronize(ev[i]);
        }
        for (uint32_t i = 0; i < kSlots; ++i) {
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            ev[i] = nullptr;
            used[i] = false;
        }
        if (host) (void)hipHostFree(host);
        host = nullptr;
        next = 0;
    }
};

struct tsr_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mtx;
    int n_cu = 0;
    uint32_t n_xcd = 0;                 // XCDs whose round-robin of workgroups was verified at open (0: none)
    char name[128] = {0};
    tsr_hip_counters ctr{};
    tsr_scratch scratch;
    tsr_staging staging;
    tsr::ExpkTab expk{};
    uint32_t fa_spin_max = 1u << 20;    // polls of the fused decode FA's tile-key wait (s_sleep 1 each)
    uint8_t * fa_fixed = nullptr;       // device address of this device's fixed FA array (tsr_fa_fixed_init)
    hipStream_t pick(void * s) const { return s ? (hipStream_t)s : stream; }
    // The device flag word raised by a kernel given no flag word of its own (tsr_hip_get_flags), in a
    // small allocation that also holds the two-pass ARGMAX's slice results after its first 256 bytes
    // (written before they are read in every call; calls on different streams of one context that
    // overlap share them).
    static constexpr size_t kFlagsBytes = 256 + (size_t)tsr::kAmRows * tsr::kAmParts * 8u;
    int32_t * flags_dev = nullptr;
    int32_t * flag(int32_t * p) const { return p ? p : flags_dev; }
    uint64_t * am_part() const { return (uint64_t *)((uint8_t *)flags_dev + 256); }
};

struct tsr_hip_weight {
    uint32_t fmt = 0, N = 0, K = 0;
    uint32_t rb = 0;             // rows per row block of the layout (wlayout.hpp)
    uint8_t * dev = nullptr;
    size_t bytes = 0;
};

// A q8_0 KV cache plane in the device layout of k_kv.hip: cells in groups of 16; the fp16 block
// scales ("meta") and the int8 quants in separate regions.
struct tsr_hip_kv {
    uint32_t E = 0, kv_size = 0;
    uint8_t * dev = nullptr;
    size_t meta_row = 0;         // bytes per cell of the meta region
    size_t quant_off = 0;        // byte offset of the quant region
    size_t bytes = 0;
};
