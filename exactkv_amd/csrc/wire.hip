// Wire form of one sequence's compressed cache: pack into / unpack from one contiguous
// byte blob (KV offload, transfer between pools or processes).
//
// No counterpart in the reference (its buffers() hands out the six tensors,
// cache.py:121-123). Layout (little-endian; every section starts at a multiple of 256 B):
//   header  256 B   u32 magic "EXKV", version 1, heads, head_dim, tokens, full_pages,
//                   tail_rows, raw_rows; u64 offsets of the six sections and the total
//   tail    bf16 [T % 16, H, 128]     the open page's tokens
//   rowmask i32  [T / 16, H]
//   base    u8   [T / 16, H, 128]
//   sm      u8   [16 * (T / 16), H, 128]
//   code    u8   [16 * (T / 16), H, 64]
//   raw     bf16 [N, 128]             raw rows of the full pages, (page, head, token) order
// rowoff is implicit: the running count of raw rows in (page, head) order.
//
// The sequence's pages are given as pool page indices (a contiguous cache's sequence b
// is pages b * TS/16 + p), so one path serves contiguous and paged caches. All three
// kernels are HBM copies: the page sections move as 16-byte vectors, one workgroup per
// page; raw rows are gathered or scattered one 256-byte row per wavefront pass.
#include "common.hpp"
#include "../../include/exactkv.h"

namespace exkv {

constexpr uint32_t kWireMagic = 0x564B5845u;   // "EXKV"
constexpr uint32_t kWireVersion = 1;

__host__ __device__ inline int64_t al256(int64_t n) { return (n + 255) / 256 * 256; }

struct WireLayout {
    int64_t off_tail, off_rowmask, off_base, off_sm, off_code, off_raw;
    __host__ __device__ WireLayout(int H, int T) {
        const int64_t npf = T / kPage, tail = T % kPage;
        off_tail = 256;
        off_rowmask = off_tail + al256(tail * H * kD * 2);
        off_base = off_rowmask + al256(npf * H * 4);
        off_sm = off_base + al256(npf * H * kD);
        off_code = off_sm + al256(npf * kPage * H * kD);
        off_raw = off_code + al256(npf * kPage * H * kD / 2);
    }
};

struct WireArgs {
    uint8_t* sm;
    uint8_t* code;
    uint8_t* base;
    int32_t* rowmask;
    int32_t* rowoff;
    uint16_t* raw;
    int64_t raw_rows;         // rows in the cache's raw array
    int64_t cap;              // unpack: slots at or past cap are dropped (as in the encoder)
    const int32_t* pages;     // [npf (+1 open page)] pool page of each sequence page
    int64_t pool_pages;
    int64_t tail_row;         // first raw row of the sequence's tail area
    int32_t* ws;              // [npf * H + 2]: raw offsets, then total, then the counter before
    uint8_t* blob;
    int64_t blob_bytes;       // raw rows past the blob's end are neither read nor written
    int32_t* cnt;             // unpack: the cache's raw-pool counter (pack: nullptr)
    int32_t* before;
    int H, T, npf, open_page;
};

__device__ inline int64_t wire_pidx(const WireArgs& a, int p) {
    return (int64_t)min((uint32_t)a.pages[p], (uint32_t)(a.pool_pages - 1));
}

// Raw offsets of the full pages in (page, head) order: ws[u] = start + running count,
// ws[n] = total, ws[n + 1] = start (the pool counter for unpack, 0 for pack). Unpack
// also advances the counter (*before = old value), as the encoder does.
template <bool UNPACK>
__global__ void __launch_bounds__(1024) wire_scan_kernel(WireArgs a) {
    const int n = a.npf * a.H;
    const int per = (n + 1023) / 1024;
    const int u0 = threadIdx.x * per, u1 = min(u0 + per, n);
    const int32_t* rm = reinterpret_cast<const int32_t*>(a.blob + WireLayout(a.H, a.T).off_rowmask);
    auto mask = [&](int u) -> uint32_t {
        if (UNPACK) return (uint32_t)rm[u];
        return (uint32_t)a.rowmask[wire_pidx(a, u / a.H) * a.H + u % a.H];
    };
    int local = 0;
    for (int u = u0; u < u1; ++u) local += popc32(mask(u) & 0xFFFFu);
    const int start = UNPACK ? *a.cnt : 0;
    int total;
    int run = start + block_excl_scan(local, total);
    for (int u = u0; u < u1; ++u) {
        a.ws[u] = run;
        run += popc32(mask(u) & 0xFFFFu);
    }
    if (threadIdx.x == 0) {
        a.ws[n] = total;
        a.ws[n + 1] = start;
        if (UNPACK) {
            *a.before = start;
            *a.cnt = start + total;
        }
    }
}

__device__ inline void copy16(const uint8_t* src, uint8_t* dst, int64_t bytes) {
    const uint4* s = reinterpret_cast<const uint4*>(src);
    uint4* d = reinterpret_cast<uint4*>(dst);
    for (int64_t i = threadIdx.x; i < bytes / 16; i += blockDim.x) d[i] = s[i];
}

// One 256-byte bf16 row by one wavefront (64 lanes x 4 bytes).
__device__ inline void copy_row(const uint16_t* src, uint16_t* dst, int lane) {
    reinterpret_cast<uint32_t*>(dst)[lane] = reinterpret_cast<const uint32_t*>(src)[lane];
}

// Blocks 0 .. npf-1: page p's sections and raw rows; block npf: the tail and the header.
template <bool UNPACK>
__global__ void __launch_bounds__(256) wire_copy_kernel(WireArgs a) {
    const WireLayout L(a.H, a.T);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int H = a.H;
    const int p = blockIdx.x;
    uint16_t* braw = reinterpret_cast<uint16_t*>(a.blob + L.off_raw);
    uint16_t* btail = reinterpret_cast<uint16_t*>(a.blob + L.off_tail);
    int32_t* brm = reinterpret_cast<int32_t*>(a.blob + L.off_rowmask);
    if (p < a.npf) {
        const int64_t pidx = wire_pidx(a, p);
        const int64_t sm_bytes = (int64_t)kPage * H * kD, code_bytes = sm_bytes / 2, base_bytes = (int64_t)H * kD;
        uint8_t* bsm = a.blob + L.off_sm + p * sm_bytes;
        uint8_t* bcode = a.blob + L.off_code + p * code_bytes;
        uint8_t* bbase = a.blob + L.off_base + p * base_bytes;
        uint8_t* csm = a.sm + pidx * sm_bytes;
        uint8_t* ccode = a.code + pidx * code_bytes;
        uint8_t* cbase = a.base + pidx * base_bytes;
        if (UNPACK) {
            copy16(bsm, csm, sm_bytes);
            copy16(bcode, ccode, code_bytes);
            copy16(bbase, cbase, base_bytes);
        } else {
            copy16(csm, bsm, sm_bytes);
            copy16(ccode, bcode, code_bytes);
            copy16(cbase, bbase, base_bytes);
        }
        const int start = a.ws[a.npf * H + 1];
        for (int h = w; h < H; h += 4) {
            const int u = p * H + h;
            const uint32_t m = UNPACK ? (uint32_t)brm[u] & 0xFFFFu : (uint32_t)a.rowmask[pidx * H + h] & 0xFFFFu;
            const int32_t dst_first = a.ws[u];            // pool slot (unpack) / blob row (pack)
            if (lane == 0) {
                if (UNPACK) {
                    a.rowmask[pidx * H + h] = (int32_t)m;
                    a.rowoff[pidx * H + h] = dst_first;
                } else {
                    brm[u] = (int32_t)m;
                }
            }
            if (m == 0) continue;
            const int64_t src_first = UNPACK ? (int64_t)(dst_first - start) : (int64_t)a.rowoff[pidx * H + h];
            const int64_t blob_rows = (a.blob_bytes - L.off_raw) / (kD * 2);
            int k = 0;
            for (int r = 0; r < kPage; ++r) {
                if (!((m >> r) & 1u)) continue;
                if (UNPACK) {
                    const int64_t slot = (int64_t)dst_first + k, brow = src_first + k;
                    if (slot < a.cap && brow < blob_rows) copy_row(braw + brow * kD, a.raw + slot * kD, lane);
                } else {
                    const int64_t slot = min(src_first + k, a.raw_rows - 1), brow = (int64_t)dst_first + k;
                    if (brow < blob_rows) copy_row(a.raw + slot * kD, braw + brow * kD, lane);
                }
                ++k;
            }
        }
        return;
    }
    // the tail: rows (r, h) of the open page <-> the tail area's row h * 16 + r
    const int tail = a.T % kPage;
    for (int i = w; i < tail * H; i += 4) {
        const int r = i / H, h = i % H;
        uint16_t* crow = a.raw + (a.tail_row + (int64_t)h * kPage + r) * kD;
        if (UNPACK)
            copy_row(btail + (int64_t)i * kD, crow, lane);
        else
            copy_row(crow, btail + (int64_t)i * kD, lane);
    }
    if (UNPACK) {
        if (a.open_page) {                             // open the sequence's last page
            for (int h = threadIdx.x; h < H; h += blockDim.x) {
                const int64_t pg = wire_pidx(a, a.npf) * H + h;
                a.rowmask[pg] = 0xFFFF;
                a.rowoff[pg] = (int32_t)(a.tail_row + (int64_t)h * kPage);
            }
        }
        return;
    }
    // zero the two alignment gaps (after rowmask and after base) and the header's tail
    const int64_t g0 = L.off_rowmask + (int64_t)a.npf * H * 4, g1 = L.off_base + (int64_t)a.npf * H * kD;
    for (int64_t i = g0 + threadIdx.x; i < L.off_base; i += blockDim.x) a.blob[i] = 0;
    for (int64_t i = g1 + threadIdx.x; i < L.off_sm; i += blockDim.x) a.blob[i] = 0;
    if (threadIdx.x >= 22 && threadIdx.x < 64) reinterpret_cast<uint32_t*>(a.blob)[threadIdx.x] = 0u;
    if (threadIdx.x == 0) {
        uint32_t* h32 = reinterpret_cast<uint32_t*>(a.blob);
        const int n = a.ws[a.npf * H];
        h32[0] = kWireMagic;
        h32[1] = kWireVersion;
        h32[2] = (uint32_t)H;
        h32[3] = (uint32_t)kD;
        h32[4] = (uint32_t)a.T;
        h32[5] = (uint32_t)a.npf;
        h32[6] = (uint32_t)tail;
        h32[7] = (uint32_t)n;
        uint64_t* h64 = reinterpret_cast<uint64_t*>(a.blob + 32);
        h64[0] = (uint64_t)L.off_tail;
        h64[1] = (uint64_t)L.off_rowmask;
        h64[2] = (uint64_t)L.off_base;
        h64[3] = (uint64_t)L.off_sm;
        h64[4] = (uint64_t)L.off_code;
        h64[5] = (uint64_t)L.off_raw;
        h64[6] = (uint64_t)(L.off_raw + (int64_t)n * kD * 2);
    }
}

}  // namespace exkv

using namespace exkv;

extern "C" int64_t exkv_wire_bytes(int32_t H, int32_t T, int64_t raw_rows) {
    if (H <= 0 || T < 0 || raw_rows < 0) return -1;
    return WireLayout(H, T).off_raw + raw_rows * kD * 2;
}

static int wire_check(const char* what, int32_t H, int32_t T, int32_t D, const int32_t* pages, int64_t pool_pages,
                      const void* blob, int64_t blob_bytes) {
    EXKV_REQUIRE(D == kD, "%s: head dim must be 128 (got %d)", what, D);
    EXKV_REQUIRE(H > 0 && T >= 0, "%s: bad H=%d or T=%d", what, H, T);
    EXKV_REQUIRE(pool_pages > 0 && (pages || T < kPage), "%s: no page list", what);
    EXKV_REQUIRE(blob && ((uintptr_t)blob % 256) == 0, "%s: the blob must be 256-byte aligned", what);
    EXKV_REQUIRE(blob_bytes >= WireLayout(H, T).off_raw, "%s: blob of %lld bytes is smaller than the %lld of its sections",
                 what, (long long)blob_bytes, (long long)WireLayout(H, T).off_raw);
    return EXKV_OK;
}

extern "C" int exkv_wire_pack(const void* sm, const void* code, const void* base, const int32_t* rowmask,
                              const int32_t* rowoff, const void* raw, int64_t raw_rows, const int32_t* pages,
                              int64_t pool_pages, int64_t tail_row, int32_t H, int32_t T, int32_t D,
                              int32_t* ws, void* blob, int64_t blob_bytes, hipStream_t stream) {
    const int rc = wire_check("wire_pack", H, T, D, pages, pool_pages, blob, blob_bytes);
    if (rc != EXKV_OK) return rc;
    EXKV_REQUIRE(sm && code && base && rowmask && rowoff && raw && ws && raw_rows > 0, "wire_pack: null pointer");
    EXKV_REQUIRE(T % kPage == 0 || (tail_row >= 0 && tail_row + (int64_t)H * kPage <= raw_rows),
                 "wire_pack: tail area outside the raw pool");
    WireArgs a{(uint8_t*)sm, (uint8_t*)code, (uint8_t*)base, (int32_t*)rowmask, (int32_t*)rowoff, (uint16_t*)raw,
               raw_rows, 0, pages, pool_pages, tail_row, ws, (uint8_t*)blob, blob_bytes, nullptr, nullptr, H, T,
               T / kPage, 0};
    hipLaunchKernelGGL(wire_scan_kernel<false>, dim3(1), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(wire_copy_kernel<false>, dim3(T / kPage + 1), dim3(256), 0, stream, a);
    return hip_status(hipGetLastError(), "wire_pack");
}

extern "C" int exkv_wire_unpack(const void* blob, int64_t blob_bytes, void* sm, void* code, void* base, int32_t* rowmask,
                                int32_t* rowoff, void* raw, int64_t raw_rows, int64_t cap, int32_t* cnt,
                                int32_t* before, const int32_t* pages, int32_t open_page, int64_t pool_pages,
                                int64_t tail_row, int32_t H, int32_t T, int32_t D, int32_t* ws,
                                hipStream_t stream) {
    const int rc = wire_check("wire_unpack", H, T, D, pages, pool_pages, blob, blob_bytes);
    if (rc != EXKV_OK) return rc;
    EXKV_REQUIRE(sm && code && base && rowmask && rowoff && raw && ws && cnt && before, "wire_unpack: null pointer");
    EXKV_REQUIRE(cap >= 0 && cap <= raw_rows, "wire_unpack: cap %lld exceeds the raw pool", (long long)cap);
    EXKV_REQUIRE(!open_page || pages, "wire_unpack: an open page needs its page index");
    EXKV_REQUIRE((T % kPage == 0 && !open_page) || (tail_row >= cap && tail_row + (int64_t)H * kPage <= raw_rows),
                 "wire_unpack: tail area outside the raw pool");
    WireArgs a{(uint8_t*)sm, (uint8_t*)code, (uint8_t*)base, rowmask, rowoff, (uint16_t*)raw, raw_rows, cap, pages,
               pool_pages, tail_row, ws, (uint8_t*)const_cast<void*>(blob), blob_bytes, cnt, before, H, T, T / kPage,
               open_page ? 1 : 0};
    hipLaunchKernelGGL(wire_scan_kernel<true>, dim3(1), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(wire_copy_kernel<true>, dim3(T / kPage + 1), dim3(256), 0, stream, a);
    return hip_status(hipGetLastError(), "wire_unpack");
}
