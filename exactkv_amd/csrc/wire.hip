// Wire form of sequences of a compressed cache: pack each into one contiguous byte blob,
// or unpack blobs into the cache (KV offload, transfer between pools or processes).
//
// No counterpart in the reference (its buffers() hands out the six tensors,
// cache.py:121-123). Blob layout (little-endian; sections at multiples of 256 B):
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
// A sequence's pages are given as pool page indices (a contiguous cache's sequence b is
// pages b * TS/16 + p), so one path serves contiguous and paged caches. One call handles a
// batch of sequences in two launches: a scan (one workgroup per sequence) places the raw
// rows, then one workgroup per (page, sequence) moves the page's 3200 bytes per head as
// 16-byte vectors -- every load of a thread issued before its stores -- and its raw rows;
// the workgroup after a sequence's last full page moves the tail and writes the header.
// Sequences whose arguments do not fit (tokens, blob size, or for unpack the blob header)
// are skipped, so no access leaves the buffers; the Python wrappers check them first.
#include "common.hpp"
#include "errors.hpp"
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
    int64_t raw_rows;           // rows of the cache's raw array
    int64_t cap;                // unpack: slots at or past cap are dropped (as in the encoder)
    int64_t pool_pages;         // pages of the cache's arrays (page entries are clamped to it)
    const int32_t* pages;       // [nseq, page_stride] pool page of each sequence page
    int64_t page_stride;
    const int32_t* tokens;      // [nseq]
    const int64_t* tail_rows;   // [nseq] first raw row of each sequence's tail area
    const uint64_t* blobs;      // [nseq] blob addresses (256-byte aligned)
    const int64_t* blob_bytes;  // [nseq]
    const int32_t* open;        // unpack: [nseq] open the page after the last full page
    int32_t* ws;                // [nseq, ws_stride]: T or -1, start, raw rows, raw offsets
    int64_t ws_stride;
    int32_t* cnt;               // unpack: the raw-pool counter (advanced by the batch total)
    int32_t* before;
    int nseq, H, max_tokens;
};

struct Seq {
    int T = -1, npf = 0;        // T < 0: skipped
    uint8_t* blob = nullptr;
    int64_t bytes = 0;
};

// Sequence s's tokens and blob, or T = -1 if they do not fit.
template <bool UNPACK>
__device__ inline Seq wire_seq(const WireArgs& a, int s) {
    Seq q;
    const int T = a.tokens[s];
    if (T < 0 || T > a.max_tokens) return q;
    const WireLayout L(a.H, T);
    const int64_t bytes = a.blob_bytes[s];
    if (bytes < L.off_raw || (a.blobs[s] & 255u) != 0) return q;
    uint8_t* blob = reinterpret_cast<uint8_t*>(a.blobs[s]);
    if (UNPACK) {
        const uint32_t* h = reinterpret_cast<const uint32_t*>(blob);
        if (h[0] != kWireMagic || h[1] != kWireVersion || h[2] != (uint32_t)a.H || h[3] != (uint32_t)kD ||
            h[4] != (uint32_t)T)
            return q;
    }
    q.T = T;
    q.npf = T / kPage;
    q.blob = blob;
    q.bytes = bytes;
    return q;
}

__device__ inline int64_t wire_pidx(const WireArgs& a, int s, int p) {
    const int64_t col = min((int64_t)p, a.page_stride - 1);
    return (int64_t)min((uint32_t)a.pages[(int64_t)s * a.page_stride + col], (uint32_t)(a.pool_pages - 1));
}

// Per sequence s (one workgroup each) the scan writes its row of ws:
//   ws[s][0] = T, or -1 if the sequence is skipped (the copy kernel follows this verdict),
//   ws[s][1] = start_s, ws[s][2] = its raw rows, ws[s][3 + u] = start_s + running count of
//   raw rows over units u = (page, head).
// Pack: start 0 (blob row). Unpack: start_s = *cnt + the raw rows the headers of blobs
// 0..s-1 declare (pool slot).
constexpr int kWsHead = 3;
constexpr int kScanPer = 8;                   // units a thread keeps in registers

template <bool UNPACK>
__global__ void __launch_bounds__(1024) wire_scan_kernel(WireArgs a) {
    const int s = blockIdx.x;
    const Seq q = wire_seq<UNPACK>(a, s);
    const int H = a.H;
    const int n = q.T < 0 ? 0 : q.npf * H;
    int32_t* ws = a.ws + (int64_t)s * a.ws_stride;
    const int per = (n + 1023) / 1024;
    const int u0 = min((int)threadIdx.x * per, n), u1 = min(u0 + per, n);
    const int32_t* brm =
        q.T < 0 ? nullptr : reinterpret_cast<const int32_t*>(q.blob + WireLayout(H, q.T).off_rowmask);
    auto mask = [&](int u) -> uint32_t {
        if (UNPACK) return (uint32_t)brm[u] & 0xFFFFu;
        return (uint32_t)a.rowmask[wire_pidx(a, s, u / H) * H + u % H] & 0xFFFFu;
    };
    // up to kScanPer units per thread: every load issued before the first use
    uint32_t mk[kScanPer];
    int local = 0;
    if (per <= kScanPer) {
        if (n > 0) {                                // unconditional (clamped) loads
#pragma unroll
            for (int k = 0; k < kScanPer; ++k) mk[k] = mask(min(u0 + k, n - 1));
#pragma unroll
            for (int k = 0; k < kScanPer; ++k) mk[k] = u0 + k < u1 ? mk[k] : 0u;
        } else {
#pragma unroll
            for (int k = 0; k < kScanPer; ++k) mk[k] = 0u;
        }
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) local += popc32(mk[k]);
    } else {
        for (int u = u0; u < u1; ++u) local += popc32(mask(u));
    }
    int start = 0;
    if (UNPACK) {                                  // raw rows declared by the earlier blobs
        int decl = 0;
        for (int j = (int)threadIdx.x; j < s; j += blockDim.x) {
            const Seq o = wire_seq<UNPACK>(a, j);
            if (o.T >= 0) decl += (int)reinterpret_cast<const uint32_t*>(o.blob)[7];
        }
        int all;
        block_excl_scan(decl, all);
        start = *a.cnt + all;
    }
    int total;
    int run = start + block_excl_scan(local, total);
    // unpack: the blob's rows must be exactly those its header declares -- the later blobs'
    // pool slots and the counter are placed by the declared counts -- else skip it
    int declared = total;
    if (UNPACK && q.T >= 0) declared = (int)reinterpret_cast<const uint32_t*>(q.blob)[7];
    if (per <= kScanPer) {
#pragma unroll
        for (int k = 0; k < kScanPer; ++k) {
            if (u0 + k < u1) ws[kWsHead + u0 + k] = run;
            run += popc32(mk[k]);
        }
    } else {
        for (int u = u0; u < u1; ++u) {
            ws[kWsHead + u] = run;
            run += popc32(mask(u));
        }
    }
    if (threadIdx.x == 0) {
        ws[0] = declared == total ? q.T : -1;
        ws[1] = start;
        ws[2] = declared;
    }
}

// One 256-byte bf16 row by one wavefront (64 lanes x 4 bytes).
__device__ inline void copy_row(const uint16_t* src, uint16_t* dst, int lane) {
    reinterpret_cast<uint32_t*>(dst)[lane] = reinterpret_cast<const uint32_t*>(src)[lane];
}

// A page's raw rows of one head: all loads, then all stores. src_row(k) / dst_row(k) give
// the k-th raw row's source and destination (nullptr: skip).
template <typename Src, typename Dst>
__device__ inline void copy_rows(uint32_t m, int lane, Src src_row, Dst dst_row) {
    uint32_t v[kPage];
    int k = 0;
#pragma unroll
    for (int r = 0; r < kPage; ++r) {
        if ((m >> r) & 1u) {
            const uint16_t* sp = src_row(k);
            v[r] = sp ? reinterpret_cast<const uint32_t*>(sp)[lane] : 0u;
            ++k;
        }
    }
    k = 0;
#pragma unroll
    for (int r = 0; r < kPage; ++r) {
        if ((m >> r) & 1u) {
            uint16_t* dp = dst_row(k);
            if (dp && src_row(k)) reinterpret_cast<uint32_t*>(dp)[lane] = v[r];
            ++k;
        }
    }
}

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Three sections of 16-byte vectors (ns, nc, nb > 0) by one 256-thread workgroup, in rounds
// of KS + KC + 1 vectors per thread: all loads of a round (clamped to the section, so they
// need no branch) are issued, then tied through an empty asm so that the compiler cannot
// sink them into the guarded stores, which would serialise load, wait and store again.
template <int KS, int KC>
__device__ inline void copy_page_sections(const v4u* s0, const v4u* s1, const v4u* s2, v4u* d0, v4u* d1, v4u* d2,
                                          int ns, int nc, int nb) {
    const int t = (int)threadIdx.x;
    for (int i0 = 0, j0 = 0, k0 = 0; i0 < ns || j0 < nc || k0 < nb; i0 += 256 * KS, j0 += 256 * KC, k0 += 256) {
        v4u va[KS], vb[KC], vc;
#pragma unroll
        for (int k = 0; k < KS; ++k) va[k] = s0[min(i0 + t + 256 * k, ns - 1)];
#pragma unroll
        for (int k = 0; k < KC; ++k) vb[k] = s1[min(j0 + t + 256 * k, nc - 1)];
        vc = s2[min(k0 + t, nb - 1)];
#pragma unroll
        for (int k = 0; k < KS; ++k) asm volatile("" : "+v"(va[k]));
#pragma unroll
        for (int k = 0; k < KC; ++k) asm volatile("" : "+v"(vb[k]));
        asm volatile("" : "+v"(vc));
#pragma unroll
        for (int k = 0; k < KS; ++k)
            if (i0 + t + 256 * k < ns) d0[i0 + t + 256 * k] = va[k];
#pragma unroll
        for (int k = 0; k < KC; ++k)
            if (j0 + t + 256 * k < nc) d1[j0 + t + 256 * k] = vb[k];
        if (k0 + t < nb) d2[k0 + t] = vc;
    }
}

// Workgroup (p, s): page p < npf of sequence s, or its tail (p == npf). The scan's row of
// ws decides whether the sequence is skipped and where its raw rows go.
template <bool UNPACK>
__global__ void __launch_bounds__(256) wire_copy_kernel(WireArgs a) {
    const int s = blockIdx.y, p = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int H = a.H;
    const int32_t* ws = a.ws + (int64_t)s * a.ws_stride;
    // independent loads first: the scan's verdict, the blob, the page entry
    const int T = ws[0], start = ws[1];
    uint8_t* blob = reinterpret_cast<uint8_t*>(a.blobs[s]);
    const int64_t bytes = a.blob_bytes[s];
    const int64_t pidx = wire_pidx(a, s, p);
    if (UNPACK && s == 0 && p == 0 && threadIdx.x == 0) {
        // the counter after the batch: the last sequence's start + its raw rows (the scan's
        // reads of *cnt are done; no workgroup of this kernel reads it)
        const int32_t* wl = a.ws + (int64_t)(a.nseq - 1) * a.ws_stride;
        *a.before = start;
        *a.cnt = wl[1] + wl[2];
    }
    if (T < 0 || p > T / kPage) return;
    const int npf = T / kPage;
    const WireLayout L(H, T);
    uint16_t* braw = reinterpret_cast<uint16_t*>(blob + L.off_raw);
    uint16_t* btail = reinterpret_cast<uint16_t*>(blob + L.off_tail);
    int32_t* brm = reinterpret_cast<int32_t*>(blob + L.off_rowmask);
    if (p < npf) {
        // this wavefront's heads h = w + 4 j: lane j holds head h's mask, first raw slot /
        // blob row and (pack) cache rowoff
        const int hl = w + 4 * lane;
        uint32_t mv = 0u;
        int32_t fv = 0, rv = 0;
        if (hl < H) {
            mv = (UNPACK ? (uint32_t)brm[p * H + hl] : (uint32_t)a.rowmask[pidx * H + hl]) & 0xFFFFu;
            fv = ws[kWsHead + p * H + hl];
            if (!UNPACK) rv = a.rowoff[pidx * H + hl];
        }
        const int64_t sm_bytes = (int64_t)kPage * H * kD, code_bytes = sm_bytes / 2, base_bytes = (int64_t)H * kD;
        // the page's sm, code and base bytes: every load of a round issued before its stores
        const int vs = (int)(sm_bytes / 16), vc = (int)(code_bytes / 16), vb = (int)(base_bytes / 16);
        v4u* cs = reinterpret_cast<v4u*>(a.sm + pidx * sm_bytes);
        v4u* cc = reinterpret_cast<v4u*>(a.code + pidx * code_bytes);
        v4u* cb = reinterpret_cast<v4u*>(a.base + pidx * base_bytes);
        v4u* bs = reinterpret_cast<v4u*>(blob + L.off_sm + p * sm_bytes);
        v4u* bc = reinterpret_cast<v4u*>(blob + L.off_code + p * code_bytes);
        v4u* bb = reinterpret_cast<v4u*>(blob + L.off_base + p * base_bytes);
        if (UNPACK)
            copy_page_sections<4, 2>(bs, bc, bb, cs, cc, cb, vs, vc, vb);
        else
            copy_page_sections<4, 2>(cs, cc, cb, bs, bc, bb, vs, vc, vb);
        const int64_t blob_rows = (bytes - L.off_raw) / (kD * 2);
        for (int j = 0; w + 4 * j < H; ++j) {
            const int h = w + 4 * j;
            const uint32_t m = (uint32_t)__shfl(mv, j);
            const int32_t first = __shfl(fv, j);       // pool slot (unpack) / blob row (pack)
            const int32_t roff = __shfl(rv, j);
            if (lane == 0) {
                if (UNPACK) {
                    a.rowmask[pidx * H + h] = (int32_t)m;
                    a.rowoff[pidx * H + h] = first;
                } else {
                    brm[p * H + h] = (int32_t)m;
                }
            }
            if (m == 0) continue;
            if (UNPACK) {
                const int64_t b0r = (int64_t)first - start;
                copy_rows(m, lane,
                          [&](int k) -> const uint16_t* {
                              const int64_t br = b0r + k, slot = (int64_t)first + k;
                              return (br >= 0 && br < blob_rows && slot >= 0 && slot < a.cap) ? braw + br * kD
                                                                                            : nullptr;
                          },
                          [&](int k) -> uint16_t* { return a.raw + ((int64_t)first + k) * kD; });
            } else {
                copy_rows(m, lane,
                          [&](int k) -> const uint16_t* {
                              const int64_t br = (int64_t)first + k;
                              bool bad;
                              const int64_t slot = clamp_slot((int64_t)roff + k, a.raw_rows, bad);
                              if (bad && br < blob_rows) report_error(kErrWire);
                              return br < blob_rows ? a.raw + slot * kD : nullptr;
                          },
                          [&](int k) -> uint16_t* { return braw + ((int64_t)first + k) * kD; });
            }
        }
        return;
    }
    // the tail: rows (r, h) of the open page <-> the tail area's row h * 16 + r
    const int tail = T % kPage;
    const int64_t trow = a.tail_rows[s];
    const bool tail_ok = trow >= (UNPACK ? a.cap : 0) && trow + (int64_t)H * kPage <= a.raw_rows;
    if (tail > 0 && tail_ok) {
        for (int i = w; i < tail * H; i += 4) {
            const int r = i / H, h = i % H;
            uint16_t* crow = a.raw + (trow + (int64_t)h * kPage + r) * kD;
            if (UNPACK)
                copy_row(btail + (int64_t)i * kD, crow, lane);
            else
                copy_row(crow, btail + (int64_t)i * kD, lane);
        }
    }
    if (UNPACK) {
        if (a.open && a.open[s] && tail_ok && npf < a.page_stride) {      // open the next page
            for (int h = threadIdx.x; h < H; h += blockDim.x) {
                const int64_t pg = pidx * H + h;
                a.rowmask[pg] = 0xFFFF;
                a.rowoff[pg] = (int32_t)(trow + (int64_t)h * kPage);
            }
        }
        return;
    }
    // pack: zero the two alignment gaps (after rowmask, after base) and the header's tail
    const int64_t g0 = L.off_rowmask + (int64_t)npf * H * 4, g1 = L.off_base + (int64_t)npf * H * kD;
    for (int64_t i = g0 + threadIdx.x; i < L.off_base; i += blockDim.x) blob[i] = 0;
    for (int64_t i = g1 + threadIdx.x; i < L.off_sm; i += blockDim.x) blob[i] = 0;
    if (threadIdx.x >= 22 && threadIdx.x < 64) reinterpret_cast<uint32_t*>(blob)[threadIdx.x] = 0u;
    if (threadIdx.x == 0) {
        uint32_t* h32 = reinterpret_cast<uint32_t*>(blob);
        const int n = ws[2];
        h32[0] = kWireMagic;
        h32[1] = kWireVersion;
        h32[2] = (uint32_t)H;
        h32[3] = (uint32_t)kD;
        h32[4] = (uint32_t)T;
        h32[5] = (uint32_t)npf;
        h32[6] = (uint32_t)tail;
        h32[7] = (uint32_t)n;
        uint64_t* h64 = reinterpret_cast<uint64_t*>(blob + 32);
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

static int wire_check(const char* what, int32_t nseq, int32_t H, int32_t max_tokens, int32_t D, const int32_t* pages,
                      int64_t page_stride, int64_t pool_pages, const int32_t* tokens, const int64_t* tail_rows,
                      const uint64_t* blobs, const int64_t* blob_bytes, int32_t* ws, int64_t ws_stride) {
    EXKV_REQUIRE(D == kD, "%s: head dim must be 128 (got %d)", what, D);
    EXKV_REQUIRE(nseq >= 0 && H > 0 && max_tokens >= 0, "%s: bad nseq=%d H=%d max_tokens=%d", what, nseq, H,
                 max_tokens);
    EXKV_REQUIRE(page_stride >= 1 && page_stride * kPage >= max_tokens && pool_pages > 0,
                 "%s: page table of %lld columns for %d tokens", what, (long long)page_stride, max_tokens);
    EXKV_REQUIRE(ws_stride >= (int64_t)(max_tokens / kPage) * H + kWsHead, "%s: ws stride %lld below %lld", what,
                 (long long)ws_stride, (long long)(max_tokens / kPage) * H + kWsHead);
    EXKV_REQUIRE(pages && tokens && tail_rows && blobs && blob_bytes && ws, "%s: null pointer", what);
    return EXKV_OK;
}

extern "C" int exkv_wire_pack(const void* sm, const void* code, const void* base, const int32_t* rowmask,
                              const int32_t* rowoff, const void* raw, int64_t raw_rows, int64_t pool_pages,
                              int32_t nseq, const int32_t* pages, int64_t page_stride, const int32_t* tokens,
                              const int64_t* tail_rows, const uint64_t* blobs, const int64_t* blob_bytes,
                              int32_t max_tokens, int32_t H, int32_t D, int32_t* ws, int64_t ws_stride,
                              hipStream_t stream) {
    const int rc = wire_check("wire_pack", nseq, H, max_tokens, D, pages, page_stride, pool_pages, tokens, tail_rows,
                              blobs, blob_bytes, ws, ws_stride);
    if (rc != EXKV_OK) return rc;
    EXKV_REQUIRE(sm && code && base && rowmask && rowoff && raw && raw_rows > 0, "wire_pack: null pointer");
    if (nseq == 0) return EXKV_OK;
    WireArgs a{(uint8_t*)sm, (uint8_t*)code, (uint8_t*)base, (int32_t*)rowmask, (int32_t*)rowoff, (uint16_t*)raw,
               raw_rows, 0, pool_pages, pages, page_stride, tokens, tail_rows, blobs, blob_bytes, nullptr, ws,
               ws_stride, nullptr, nullptr, nseq, H, max_tokens};
    hipLaunchKernelGGL(wire_scan_kernel<false>, dim3(nseq), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(wire_copy_kernel<false>, dim3(max_tokens / kPage + 1, nseq), dim3(256), 0, stream, a);
    return hip_status(hipGetLastError(), "wire_pack");
}

extern "C" int exkv_wire_unpack(void* sm, void* code, void* base, int32_t* rowmask, int32_t* rowoff, void* raw,
                                int64_t raw_rows, int64_t cap, int32_t* cnt, int32_t* before, int64_t pool_pages,
                                int32_t nseq, const int32_t* pages, int64_t page_stride, const int32_t* tokens,
                                const int32_t* open, const int64_t* tail_rows, const uint64_t* blobs,
                                const int64_t* blob_bytes, int32_t max_tokens, int32_t H, int32_t D, int32_t* ws,
                                int64_t ws_stride, hipStream_t stream) {
    const int rc = wire_check("wire_unpack", nseq, H, max_tokens, D, pages, page_stride, pool_pages, tokens,
                              tail_rows, blobs, blob_bytes, ws, ws_stride);
    if (rc != EXKV_OK) return rc;
    EXKV_REQUIRE(sm && code && base && rowmask && rowoff && raw && cnt && before, "wire_unpack: null pointer");
    EXKV_REQUIRE(cap >= 0 && cap <= raw_rows, "wire_unpack: cap %lld exceeds the raw pool", (long long)cap);
    if (nseq == 0) return EXKV_OK;
    WireArgs a{(uint8_t*)sm, (uint8_t*)code, (uint8_t*)base, rowmask, rowoff, (uint16_t*)raw, raw_rows, cap,
               pool_pages, pages, page_stride, tokens, tail_rows, blobs, blob_bytes, open, ws, ws_stride, cnt, before,
               nseq, H, max_tokens};
    hipLaunchKernelGGL(wire_scan_kernel<true>, dim3(nseq), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(wire_copy_kernel<true>, dim3(max_tokens / kPage + 1, nseq), dim3(256), 0, stream, a);
    return hip_status(hipGetLastError(), "wire_unpack");
}

namespace exkv {
hipError_t fetch_errors_wire(uint32_t* out, int first, int clear, hipStream_t stream) {
    return fetch_file_errors(out, first, clear, stream);
}
}  // namespace exkv
