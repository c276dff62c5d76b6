// Decode attention over the compressed cache with no workspace argument and no allocation:
// the split partials live in a fixed per-GPU scratch array. For callers that cannot call
// hipMalloc (HIP-graph capture, tight serving loops, harnesses that forbid allocation).
//
// The array is a file-scope __device__ object, so every GPU the library runs on holds its
// own copy for the life of the process. Host code never uses its name as an address: the
// first call on a device asks the runtime for that device's address (hipGetSymbolAddress,
// with the device current) and keeps it. The device is the one the call's stream belongs
// to (hipStreamGetDevice), not whichever device happens to be current, so a call on another
// GPU's stream gets that GPU's array. A failed lookup is not kept: the next call on the
// device asks again. Every call on a GPU shares that GPU's array; calls that overlap on one
// GPU (other streams, other threads) race on it.
#include <atomic>
#include <mutex>

#include "common.hpp"
#include "../../include/exactkv.h"

namespace exkv {

constexpr int64_t kScratchBytes = int64_t(32) << 20;   // split partials: o, m, l in fp32
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

static std::atomic<void*> g_scratch[kMaxDevices];      // nullptr until a lookup succeeds
static std::mutex g_scratch_mu;

// The device of `stream` (the null stream: the current device).
static int stream_device(hipStream_t stream, int* dev) {
    hipDevice_t d = -1;
    const hipError_t e = hipStreamGetDevice(stream, &d);
    if (e != hipSuccess) return hip_status(e, "attn_compressed_noalloc: hipStreamGetDevice");
    EXKV_REQUIRE(d >= 0 && d < kMaxDevices, "attn_compressed_noalloc: device %d out of range", (int)d);
    *dev = (int)d;
    return EXKV_OK;
}

// Device dev's copy of the scratch array. The lookup runs with dev current (the caller's
// current device is restored afterwards) and is kept only once it has succeeded.
static int scratch_of_device(int dev, float** out) {
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            int cur = -1;
            hipError_t e = hipGetDevice(&cur);
            if (e != hipSuccess) return hip_status(e, "attn_compressed_noalloc: hipGetDevice");
            if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
                return hip_status(e, "attn_compressed_noalloc: hipSetDevice");
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (cur != dev) {
                const hipError_t r = hipSetDevice(cur);
                if (e == hipSuccess && r != hipSuccess) e = r;
            }
            if (e != hipSuccess) return hip_status(e, "attn_compressed_noalloc: hipGetSymbolAddress");
            EXKV_REQUIRE(p != nullptr, "attn_compressed_noalloc: no scratch address for device %d", dev);
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = static_cast<float*>(p);
    return EXKV_OK;
}

}  // namespace exkv

extern "C" int64_t exkv_noalloc_scratch_bytes(void) { return exkv::kScratchBytes; }

extern "C" int exkv_attn_compressed_noalloc(const void* q, const void* k_sm, const void* k_code, const void* k_base,
                                            const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw,
                                            int64_t k_raw_rows, const void* v_sm, const void* v_code,
                                            const void* v_base, const int32_t* v_rowmask, const int32_t* v_rowoff,
                                            const void* v_raw, int64_t v_raw_rows, void* out, int32_t B, int32_t Hq,
                                            int32_t Hkv, int32_t D, int32_t T, int32_t TS, const int32_t* lens,
                                            int64_t lens_stride, int32_t nsplit, int32_t split_len, int32_t window,
                                            float qk_scale, hipStream_t stream) {
    EXKV_REQUIRE(B > 0 && Hq > 0 && nsplit > 0 && exkv::head_dim_ok(D),
                 "attn_compressed_noalloc: bad shape B=%d Hq=%d nsplit=%d D=%d", B, Hq, nsplit, D);
    const int64_t partials = (int64_t)B * Hq * nsplit;             // (sequence, query head, split)
    const int64_t need = partials * (D + 2) * (int64_t)sizeof(float);
    EXKV_REQUIRE(need <= exkv::kScratchBytes,
                 "attn_compressed_noalloc: %lld split partials need %lld bytes, more than the %lld-byte scratch",
                 (long long)partials, (long long)need, (long long)exkv::kScratchBytes);
    int dev = -1;
    int rc = exkv::stream_device(stream, &dev);
    if (rc != EXKV_OK) return rc;
    float* s = nullptr;
    rc = exkv::scratch_of_device(dev, &s);
    if (rc != EXKV_OK) return rc;
    float* ws_o = s;                                                // [B*Hq, nsplit, D]
    float* ws_m = ws_o + partials * D;                              // [B*Hq, nsplit]
    float* ws_l = ws_m + partials;
    // every partial is written by the split kernel before the merge reads it, so the
    // array's previous contents never matter; no arrival counters (merge as a second kernel)
    return exkv_attn_compressed(q, k_sm, k_code, k_base, k_rowmask, k_rowoff, k_raw, k_raw_rows, v_sm, v_code, v_base,
                                v_rowmask, v_rowoff, v_raw, v_raw_rows, ws_o, ws_m, ws_l, nullptr, out, B, Hq, Hkv, D,
                                T, TS, lens, lens_stride, nsplit, split_len, window, qk_scale, stream);
}
