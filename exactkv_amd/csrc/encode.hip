// Page encoder, deterministic raw-slot assignment, device-side append and the
// compressed -> bf16 decoder, for gfx950.
//
// Encoding one call's pages takes four launches on the caller's stream (two when the caller
// gives a scan workspace: 2-4 then run as one chained scan kernel, scan_chain_kernel):
//   1. enc_pages_kernel    one wavefront per (sequence, page, head): exponent window,
//                          zero flag, codes, sign|mantissa bytes, base bytes, rowmask
//                          (reference kernels.py:216-264, codec.py:31-49);
//   2. scan_count_kernel   per block of 1024 units, its raw rows;
//   3. scan_blocks_kernel  the block totals scanned from the counter, which advances
//                          by the total;
//   4. scan_write_kernel   rowoff = counter + exclusive running count of raw rows over
//                          the call's pages in (sequence, page, head) order (codec.py:50-53
//                          order; the reference GPU encoder used an atomic counter,
//                          kernels.py:262), then the raw rows into their slots, skipping
//                          slots >= cap (kernels.py:265-268), so an overflow is seen from
//                          the counter.
// The append path (cache.py:100-112) runs a write (+ page encode), a one-workgroup slot
// scan and a raw-row copy with the token count read from device memory, so a decode step
// can be captured in a HIP graph. Every kernel that touches rows is a template on the
// head dim (64, 128 or 256); the entry points pick the instance.
#include "tile.hpp"
#include "../../include/exactkv.h"

namespace exkv {

__device__ inline uint8_t sm_byte(uint32_t u) { return (uint8_t)(((u >> 8) & 0x80u) | (u & 0x7Fu)); }

// Two 16-bit lanes in one register: the page encoder keeps two channels' exponents per
// register and works on both with packed integer ops (max, min, saturating subtract).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ inline u16x2 as_u16x2(uint32_t x) { return __builtin_bit_cast(u16x2, x); }
__device__ inline uint32_t as_u32(u16x2 x) { return __builtin_bit_cast(uint32_t, x); }
__device__ inline u16x2 vmax(u16x2 a, u16x2 b) { return __builtin_elementwise_max(a, b); }
__device__ inline u16x2 vmin(u16x2 a, u16x2 b) { return __builtin_elementwise_min(a, b); }
__device__ inline u16x2 vsubs(u16x2 a, u16x2 b) { return __builtin_elementwise_sub_sat(a, b); }   // max(a - b, 0)
// bytes 0 and 2 of x as a 16-bit value
__device__ inline uint16_t bytes02(uint32_t x) { return (uint16_t)__builtin_amdgcn_perm(0u, x, 0x0c0c0200u); }

// Encode one 16-token page of one head of D channels (D = 64, 128, 256). The lanes form
// NG token groups (2; 4 for D = 64) of CL = 64 / NG lanes: lane (grp, m) takes tokens
// TPL*grp .. TPL*grp + TPL - 1 (TPL = 16 / NG) and, in pass p, channels c, c + 1 (word lo)
// and c + D/2, c + D/2 + 1 (word hi) with c = 2 CL p + 2m -- so each code byte (channel j
// low nibble, j + D/2 high nibble) and each pair of sm / code bytes is produced by one
// lane, and every load and store moves two channels (one pass for D <= 128, two for 256).
// Per channel, with e the 8-bit exponent:
//   top = max e over the 16 tokens, floor = max(top - 15, 0), zf = (some e == 0) && floor > 0,
//   nibble = max(e - floor, 0) (e <= top keeps it <= 15; e == 0 gives 0 either way),
//   a row is raw if some channel has e != 0 && e < floor + zf, or if any floor >= 128;
// the same rule as the reference's per-element test (code >= 1 for a non-zero in a
// flagged group, code >= 0 otherwise, floor < 128), in packed 16-bit integer arithmetic.
// The token groups combine their per-channel maxima and minima with one cross-group
// shuffle each (two for four groups). Token p's source row is src + p * s_p, except row
// 15 which comes from `last` when given; rows must be 4-byte aligned (even element
// offsets: callers check). Destination rows of consecutive tokens are `rs` rows apart
// (rs = H).
template <int D>
__device__ __attribute__((always_inline)) inline uint32_t encode_page(const uint16_t* src, int64_t s_p,
                                                                  const uint16_t* last, int lane,
                                                                  uint8_t* sm0, uint8_t* code0, int64_t rs,
                                                                  uint8_t* basep, int32_t* rmaskp) {
    static_assert(D == 64 || D == 128 || D == 256, "head dim 64, 128 or 256");
    constexpr int NG = D == 64 ? 4 : 2;            // token groups
    constexpr int TPL = kPage / NG;                // tokens per lane
    constexpr int CL = 64 / NG;                    // lanes per group = channel pairs per pass
    constexpr int HALF = D / 2;
    constexpr int NPASS = HALF / (2 * CL);
    const int grp = lane / CL, m = lane % CL;
    const int64_t sm_stride = rs * D, code_stride = rs * HALF;
    uint32_t esc = 0;                              // bit i: token TPL*grp + i escapes
    bool big = false;
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
        const int c = 2 * CL * pass + 2 * m;
        // per-lane row-0 addresses of the lane's group; token i of the group is i strides on
        const uint16_t* srow = src + (int64_t)(TPL * grp) * s_p + c;
        uint8_t* smrow = sm0 + (int64_t)(TPL * grp) * sm_stride + c;
        uint8_t* coderow = code0 + (int64_t)(TPL * grp) * code_stride + c;
        uint32_t lo[TPL], hi[TPL];                 // bf16 pairs: channels (c, c+1), (c+D/2, c+D/2+1)
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
            const uint16_t* rp = (i == TPL - 1 && grp == NG - 1 && last != nullptr) ? last + c : srow + i * s_p;
            lo[i] = *reinterpret_cast<const uint32_t*>(rp);
            hi[i] = *reinterpret_cast<const uint32_t*>(rp + HALF);
        }
        u16x2 elo[TPL], ehi[TPL];                  // exponents, one channel per 16-bit lane
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
            elo[i] = as_u16x2((lo[i] >> 7) & 0x00FF00FFu);
            ehi[i] = as_u16x2((hi[i] >> 7) & 0x00FF00FFu);
        }
        u16x2 tlo = elo[0], thi = ehi[0], nlo = elo[0], nhi = ehi[0];
#pragma unroll
        for (int i = 1; i < TPL; ++i) {
            tlo = vmax(tlo, elo[i]);
            thi = vmax(thi, ehi[i]);
            nlo = vmin(nlo, elo[i]);
            nhi = vmin(nhi, ehi[i]);
        }
#pragma unroll
        for (int d = CL; d < 64; d <<= 1) {
            tlo = vmax(tlo, as_u16x2((uint32_t)__shfl_xor((int)as_u32(tlo), d)));
            thi = vmax(thi, as_u16x2((uint32_t)__shfl_xor((int)as_u32(thi), d)));
            nlo = vmin(nlo, as_u16x2((uint32_t)__shfl_xor((int)as_u32(nlo), d)));
            nhi = vmin(nhi, as_u16x2((uint32_t)__shfl_xor((int)as_u32(nhi), d)));
        }
        const u16x2 c15 = {15, 15}, one = {1, 1};
        const u16x2 flo = vsubs(tlo, c15), fhi = vsubs(thi, c15);                 // floors
        const u16x2 zlo = vmin(vsubs(one, nlo), vmin(flo, one));                  // zero flags (0 / 1)
        const u16x2 zhi = vmin(vsubs(one, nhi), vmin(fhi, one));
        const u16x2 glo = flo + zlo, ghi = fhi + zhi;                             // non-zero e below: raw
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
            const uint32_t dlo = as_u32(vmin(vsubs(glo, elo[i]), elo[i]));
            const uint32_t dhi = as_u32(vmin(vsubs(ghi, ehi[i]), ehi[i]));
            esc |= (uint32_t)((dlo | dhi) != 0u) << i;
            // code bytes c (nibble of c | nibble of c+D/2 << 4) and c+1 (c+1 | c+1+D/2 << 4)
            const uint32_t cw = as_u32(vsubs(elo[i], flo)) | (as_u32(vsubs(ehi[i], fhi)) << 4);
            // sm bytes: sign over bit 7 of each bf16's mantissa byte
            const uint32_t slo = (lo[i] & 0x007F007Fu) | ((lo[i] >> 8) & 0x00800080u);
            const uint32_t shi = (hi[i] & 0x007F007Fu) | ((hi[i] >> 8) & 0x00800080u);
            uint8_t* sp = smrow + i * sm_stride;
            *reinterpret_cast<uint16_t*>(sp) = bytes02(slo);
            *reinterpret_cast<uint16_t*>(sp + HALF) = bytes02(shi);
            *reinterpret_cast<uint16_t*>(coderow + i * code_stride) = bytes02(cw);
        }
        if (grp == 0) {
            const u16x2 c128 = {128, 128}, c255 = {255, 255};
            const uint32_t blo = as_u32(vmin(flo + zlo * c128, c255)), bhi = as_u32(vmin(fhi + zhi * c128, c255));
            *reinterpret_cast<uint16_t*>(basep + c) = bytes02(blo);
            *reinterpret_cast<uint16_t*>(basep + HALF + c) = bytes02(bhi);
        }
        big = big || ((as_u32(flo) | as_u32(fhi)) & 0xFF80FF80u) != 0u;
    }
    // rowmask: ballot bits [CL*grp, CL*grp + CL) are token TPL*grp + i; a floor of 128 or
    // more in any channel makes every row raw
    uint32_t rm = __ballot(big) != 0 ? 0xFFFFu : 0u;
    constexpr uint64_t kGroup = CL == 64 ? ~0ull : (1ull << CL) - 1ull;
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
        const uint64_t bal = __ballot((esc >> i) & 1u);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi)
            if (((bal >> (CL * gi)) & kGroup) != 0u) rm |= 1u << (TPL * gi + i);
    }
    if (lane == 0 && rmaskp != nullptr) *rmaskp = (int32_t)rm;
    return rm;
}

struct EncArgs {
    const uint16_t* src;
    int64_t s_b, s_pg, s_p, s_h;      // source strides in elements
    uint8_t* sm;
    uint8_t* code;
    uint8_t* base;
    int32_t* rowmask;
    int32_t* rowoff;
    uint16_t* raw;
    int32_t* cnt;
    int32_t* before;
    int64_t cap;
    int b0, pg0, nb, npg, H, TS;
    // Paged destination: page pg of source sequence bi goes to page dst_pages[bi *
    // dst_stride + pg] of the arrays read as B * TS / 16 pages (entries clamped to them);
    // nullptr: page pg0 + pg of sequence b0 + bi.
    const int32_t* dst_pages = nullptr;
    int64_t dst_stride = 0;
    int64_t all_pages = 0;
    int D = kD;                       // head dim: 64, 128 or 256
};

__device__ inline void unit_coords(const EncArgs& a, int64_t u, int& bi, int& pg, int& hk) {
    hk = (int)(u % a.H);
    const int64_t q = u / a.H;
    pg = (int)(q % a.npg);
    bi = (int)(q / a.npg);
}

// Page index of unit (bi, pg) in the arrays read as a list of pages.
__device__ inline int64_t unit_pidx(const EncArgs& a, int bi, int pg) {
    if (a.dst_pages == nullptr) return (int64_t)(a.b0 + bi) * (a.TS / kPage) + (a.pg0 + pg);
    const int32_t e = a.dst_pages[bi * a.dst_stride + pg];
    return (int64_t)min((uint64_t)(uint32_t)e, (uint64_t)(a.all_pages - 1));
}
__device__ inline int64_t unit_page(const EncArgs& a, int bi, int pg, int hk) {
    return unit_pidx(a, bi, pg) * a.H + hk;
}

// One wavefront per unit (sequence, page, head); the unit's coordinates and addresses are
// wavefront-uniform (scalar arithmetic, 32-bit: unit counts are below 2^31).
template <int D>
__global__ void __launch_bounds__(256) enc_pages_kernel(EncArgs a, int nunits) {
    const int lane = threadIdx.x & 63;
    const int u = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (u >= nunits) return;
    const uint32_t q = (uint32_t)u / (uint32_t)a.H, bi = q / (uint32_t)a.npg;
    const int hk = u - (int)(q * (uint32_t)a.H), pg = (int)(q - bi * (uint32_t)a.npg);
    const uint16_t* src = a.src + (int64_t)bi * a.s_b + (int64_t)pg * a.s_pg + (int64_t)hk * a.s_h;
    const int64_t pidx = unit_pidx(a, (int)bi, pg);
    const int64_t row0 = pidx * kPage * a.H + hk, page = pidx * a.H + hk;
    encode_page<D>(src, a.s_p, nullptr, lane, a.sm + row0 * D, a.code + row0 * (D / 2), a.H, a.base + page * D,
                   a.rowmask + page);
}

// The slot scan after a page encode, one unit per thread and 1024 units per block, every
// access coalesced:
//   scan_count_kernel   block g: its units' raw rows -> the rowoff slot of its first unit;
//   scan_blocks_kernel  one workgroup: exclusive scan of the block totals from the
//                       counter -> the same slots; the counter advances by the total;
//   scan_write_kernel   block g: rowoff = its slot's offset + the block's exclusive scan,
//                       then each wavefront copies the raw rows of its escaped units.
// The block totals need no workspace: the slot of a block's first unit is read by that
// block alone, and its final value (the block's offset + 0) is the one read.
constexpr int kScanUnits = 1024;

// Coordinates and page (in the arrays read as pages x heads) of unit u, with the layout
// fixed at compile time (unit counts are below 2^31: the entry points check).
template <bool PAGED>
__device__ inline int64_t unit_page32(const EncArgs& a, int u, int& bi, int& pg, int& hk) {
    const int q = u / a.H;
    hk = u - q * a.H;
    bi = q / a.npg;
    pg = q - bi * a.npg;
    if (PAGED) {
        const int32_t e = a.dst_pages[(int64_t)bi * a.dst_stride + pg];
        return (int64_t)min((uint64_t)(uint32_t)e, (uint64_t)(a.all_pages - 1)) * a.H + hk;
    }
    return ((int64_t)(a.b0 + bi) * (a.TS / kPage) + (a.pg0 + pg)) * a.H + hk;
}

__device__ inline int64_t first_page_of(const EncArgs& a, int64_t g) {
    int bi, pg, hk;
    unit_coords(a, g * kScanUnits, bi, pg, hk);
    return unit_page(a, bi, pg, hk);
}

template <bool PAGED>
__global__ void __launch_bounds__(1024) scan_count_kernel(EncArgs a, int nunits) {
    const int u = blockIdx.x * kScanUnits + threadIdx.x;
    int bi, pg, hk;
    uint32_t m = 0;
    if (u < nunits) m = (uint32_t)a.rowmask[unit_page32<PAGED>(a, u, bi, pg, hk)];
    int total;
    block_excl_scan(popc32(m), total);
    if (threadIdx.x == 0) a.rowoff[first_page_of(a, blockIdx.x)] = total;
}

__global__ void __launch_bounds__(1024) scan_blocks_kernel(EncArgs a, int64_t nblocks) {
    const int64_t per = (nblocks + 1023) / 1024;
    const int64_t g0 = min((int64_t)threadIdx.x * per, nblocks), g1 = min(g0 + per, nblocks);
    const int cnt0 = *a.cnt;
    int local = 0;
    for (int64_t g = g0; g < g1; ++g) local += a.rowoff[first_page_of(a, g)];
    int total;
    int run = cnt0 + block_excl_scan(local, total);
    for (int64_t g = g0; g < g1; ++g) {
        const int64_t p = first_page_of(a, g);
        const int t = a.rowoff[p];
        a.rowoff[p] = run;
        run += t;
    }
    if (threadIdx.x == 0) {
        if (a.before) *a.before = cnt0;
        *a.cnt = cnt0 + total;
    }
}

// The raw rows (D channels) of the escaped units among a wavefront's 64 (lane = unit: mask
// m, first slot off, source row 0 at src). VEC16 (source rows 16-byte aligned): four units
// at a time, a 16-lane group per unit, each lane moving D/16 channels (8 or 16 bytes) of
// every row of its unit per pass (two passes for D = 256) with all the unit's loads of a
// pass in flight; else one unit at a time, 4 bytes of each row per lane per pass. Slots at
// or past cap are skipped (the host grows the pool and encodes again).
template <bool VEC16, int D>
__device__ inline void copy_escaped_rows(const EncArgs& a, uint32_t m, int32_t off, const uint16_t* src,
                                         int lane) {
    uint64_t todo = __ballot(m != 0);
    if (VEC16) {
        constexpr int EPL = D == 64 ? 4 : 8;           // channels per lane per pass
        constexpr int NPASS = D / (16 * EPL);
        const int g = lane >> 4, j = lane & 15;
        while (todo != 0) {
            int pick = -1;                             // group g takes the g-th unit left
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (todo != 0) {
                    if (i == g) pick = __builtin_ctzll(todo);
                    todo &= todo - 1;
                }
            const int from = pick < 0 ? 0 : pick;
            // every lane joins the shuffles (a shuffle from a lane outside the executing
            // ones reads 0): the unit's mask, first slot and source row
            const uint32_t mv = (uint32_t)__shfl((int)m, from);
            const uint32_t mp = pick < 0 ? 0u : mv;
            const int32_t op = __shfl(off, from);
            const uint64_t sp = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(uintptr_t)src, from)) |
                                ((uint64_t)(uint32_t)__shfl((int)(uint32_t)((uintptr_t)src >> 32), from) << 32);
            const int nr = popc32(mp);
#pragma unroll
            for (int pass = 0; pass < NPASS; ++pass) {
                const int c0 = 16 * EPL * pass + EPL * j;
                const uint16_t* s = reinterpret_cast<const uint16_t*>(sp) + c0;
                uint32_t t = mp;
                uint32_t r[kPage][EPL / 2];
#pragma unroll
                for (int k = 0; k < kPage; ++k) {      // the k-th escaped row of the unit
                    const int p = t != 0u ? __builtin_ctz(t) : 0;
                    t &= t - 1u;
                    if (k < nr) {
                        ld_words<EPL / 2>(s + p * a.s_p, r[k]);
                    } else {
#pragma unroll
                        for (int w = 0; w < EPL / 2; ++w) r[k][w] = 0u;
                    }
                }
#pragma unroll
                for (int k = 0; k < kPage; ++k)
                    if (k < nr && (int64_t)op + k < a.cap) st_words<EPL / 2>(a.raw + ((int64_t)op + k) * D + c0, r[k]);
            }
        }
    } else {
        constexpr int NPASS = D > 128 ? D / 128 : 1;
        while (todo != 0) {
            const int l = __builtin_ctzll(todo);
            todo &= todo - 1;
            const uint32_t mp = (uint32_t)__builtin_amdgcn_readlane((int)m, l);
            const int32_t op = __builtin_amdgcn_readlane(off, l);
            const uint64_t sp = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uintptr_t)src, l) |
                                ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uintptr_t)src >> 32), l) << 32);
            const int nr = popc32(mp);
#pragma unroll
            for (int pass = 0; pass < NPASS; ++pass) {
                const int c0 = 128 * pass + 2 * lane;
                if (c0 >= D) continue;                 // D = 64: half the lanes
                const uint16_t* s = reinterpret_cast<const uint16_t*>(sp) + c0;
                uint32_t t = mp;
                uint32_t r[kPage];
#pragma unroll
                for (int k = 0; k < kPage; ++k) {
                    const int p = t != 0u ? __builtin_ctz(t) : 0;
                    t &= t - 1u;
                    r[k] = k < nr ? *reinterpret_cast<const uint32_t*>(s + p * a.s_p) : 0u;
                }
#pragma unroll
                for (int k = 0; k < kPage; ++k)
                    if (k < nr && (int64_t)op + k < a.cap)
                        *reinterpret_cast<uint32_t*>(a.raw + ((int64_t)op + k) * D + c0) = r[k];
            }
        }
    }
}

template <bool PAGED, bool VEC16, int D>
__global__ void __launch_bounds__(1024) scan_write_kernel(EncArgs a, int nunits) {
    __shared__ int s_base;
    if (threadIdx.x == 0) s_base = a.rowoff[first_page_of(a, blockIdx.x)];
    const int u = blockIdx.x * kScanUnits + threadIdx.x;
    int bi = 0, pg = 0, hk = 0;
    int64_t page = 0;
    uint32_t m = 0;
    if (u < nunits) {
        page = unit_page32<PAGED>(a, u, bi, pg, hk);
        m = (uint32_t)a.rowmask[page];
    }
    int total;
    const int off = block_excl_scan(popc32(m), total) + s_base;   // synchronises: s_base is read
    if (u < nunits) a.rowoff[page] = off;
    copy_escaped_rows<VEC16, D>(a, m, off, a.src + bi * a.s_b + pg * a.s_pg + hk * a.s_h, threadIdx.x & 63);
}

template <int D>
static void launch_scan(const EncArgs& a, int64_t n, hipStream_t stream) {
    const unsigned nb = (unsigned)((n + kScanUnits - 1) / kScanUnits);
    const bool paged = a.dst_pages != nullptr;
    const bool vec16 = (uintptr_t)a.src % 16 == 0 && a.s_b % 8 == 0 && a.s_pg % 8 == 0 && a.s_p % 8 == 0 &&
                       a.s_h % 8 == 0;
    if (paged)
        hipLaunchKernelGGL(scan_count_kernel<true>, dim3(nb), dim3(1024), 0, stream, a, (int)n);
    else
        hipLaunchKernelGGL(scan_count_kernel<false>, dim3(nb), dim3(1024), 0, stream, a, (int)n);
    hipLaunchKernelGGL(scan_blocks_kernel, dim3(1), dim3(1024), 0, stream, a, (int64_t)nb);
    auto k = paged ? (vec16 ? scan_write_kernel<true, true, D> : scan_write_kernel<true, false, D>)
                   : (vec16 ? scan_write_kernel<false, true, D> : scan_write_kernel<false, false, D>);
    hipLaunchKernelGGL(k, dim3(nb), dim3(1024), 0, stream, a, (int)n);
}

// ---- two-launch encode: the page kernel, then one scan kernel whose blocks chain
//
// scan_chain_kernel: block = kScanUnits units, as scan_write_kernel, but the blocks take
// their places in ticket order (an atomic counter, so that every block's predecessors have
// started) and chain their raw-row totals with a decoupled look-back (Merrill & Garland,
// "Single-pass Parallel Prefix Scan with Decoupled Look-back", NVIDIA technical report
// NVR-2016-002): a block publishes its total, walks back over its predecessors' published
// words until one that already includes everything before it, and publishes its inclusive
// total. Block 0 starts from the pool counter; the last block writes the counter back.
// rowoff, raw slots and counter come out exactly as from the three-launch scan.
//
// Workspace (the caller's; all zero when first used, then only this kernel writes it):
// ws[0] the ticket counter, ws[1] a call generation, ws[2 + t] block t's word: the call's
// tag (bits 63-32: the generation's low 31 bits with bit 63 set, so that neither words
// left by earlier calls nor never-written zero words are taken for this call's), inclusive
// flag (bit 31), count (bits 30-0). The last ticket holder resets the counter and advances
// the generation, so consecutive calls on one stream share a workspace; calls that
// overlap on one workspace race.
constexpr uint64_t kInclusive = 1ull << 31;
constexpr int kLookbackSpin = 1 << 22;              // bound of the look-back's waits (never reached; reported)

__device__ inline uint64_t ws_ld(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void ws_st(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline uint32_t chain_tag(uint32_t gen) { return (gen & 0x7FFFFFFFu) | 0x80000000u; }

// Exclusive prefix of block `t0 + 1` (t0 >= 0): one wavefront reads 64 predecessors' words
// at a time (lane i: block t - i), nearest first; every word up to the nearest inclusive one
// must carry this call's tag (else the window is read again), and their counts are summed.
__device__ inline int64_t chain_lookback(const uint64_t* ws, uint32_t tag, int t0, int lane) {
    int64_t excl = 0;
    int t = t0;
    for (int s = 0; s < kLookbackSpin; ++s) {
        const int tt = t - lane;
        const uint64_t st = tt >= 0 ? ws_ld(ws + 2 + tt) : (((uint64_t)tag << 32) | kInclusive);
        const bool valid = (uint32_t)(st >> 32) == tag;
        const uint64_t incl = __ballot(valid && (st & kInclusive) != 0);
        const int stop = incl != 0 ? __builtin_ctzll(incl) : 63;
        const uint64_t need = stop == 63 ? ~0ull : (2ull << stop) - 1ull;
        if ((~__ballot(valid) & need) != 0) {          // a predecessor has not published yet
            __builtin_amdgcn_s_sleep(1);
            continue;
        }
        // block totals (<= 16 * kScanUnits each) summed in 32 bits, the inclusive word apart
        int v = lane < stop || (incl == 0 && lane == stop) ? (int)(st & 0x7FFFFFFFull) : 0;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d);
        excl += v;
        if (incl != 0)
            return excl + (int64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(st & 0x7FFFFFFFull), stop);
        t -= 64;
    }
    if (lane == 0) report_error(kErrLookback);          // gave up: the prefix is partial
    return excl;
}

template <bool PAGED, bool VEC16, int D>
__global__ void __launch_bounds__(1024) scan_chain_kernel(EncArgs a, int nunits, int nblocks, uint64_t* ws) {
    __shared__ int s_tile, s_excl;
    __shared__ uint32_t s_gen;
    const int lane = threadIdx.x & 63;
    if (threadIdx.x == 0) {
        const uint32_t gen = (uint32_t)ws_ld(ws + 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the generation is read before the ticket is taken
        const uint32_t t = __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(ws), 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        if (t == (uint32_t)nblocks - 1u) {             // every ticket of this call is out
            ws_st(ws, 0ull);
            ws_st(ws + 1, (uint64_t)(gen + 1u));
        }
        s_tile = (int)t;
        s_gen = gen;
    }
    __syncthreads();
    const int tile = s_tile;
    const uint32_t tag = chain_tag(s_gen);
    if ((uint32_t)tile >= (uint32_t)nblocks) {         // a workspace left inconsistent (misuse): write nothing
        if (threadIdx.x == 0) report_error(kErrScanWs);
        return;
    }
    const int u = tile * kScanUnits + threadIdx.x;
    int bi = 0, pg = 0, hk = 0;
    int64_t page = 0;
    uint32_t m = 0;
    if (u < nunits) {
        page = unit_page32<PAGED>(a, u, bi, pg, hk);
        m = (uint32_t)a.rowmask[page];
    }
    int total;
    const int pre = block_excl_scan(popc32(m), total);   // synchronises
    if (threadIdx.x < 64) {
        int64_t excl;
        if (tile == 0) {
            excl = *a.cnt;
            if (lane == 0 && a.before != nullptr) *a.before = (int32_t)excl;
        } else {
            if (lane == 0) ws_st(ws + 2 + tile, ((uint64_t)tag << 32) | (uint32_t)total);
            excl = chain_lookback(ws, tag, tile - 1, lane);
        }
        if (lane == 0) {
            ws_st(ws + 2 + tile, ((uint64_t)tag << 32) | kInclusive | (uint64_t)(uint32_t)(excl + total));
            if (tile == nblocks - 1) *a.cnt = (int32_t)(excl + total);
            s_excl = (int)excl;
        }
    }
    __syncthreads();
    const int off = s_excl + pre;
    if (u < nunits) a.rowoff[page] = off;
    copy_escaped_rows<VEC16, D>(a, m, off, a.src + bi * a.s_b + pg * a.s_pg + hk * a.s_h, lane);
}

// Encode n units: the page kernel, then the chained scan when the workspace has at least
// 2 + ceil(n / kScanUnits) words, else the three-launch scan.
template <int D>
static void launch_encode_d(const EncArgs& a, int64_t n, uint64_t* ws, int64_t ws_words, hipStream_t stream) {
    hipLaunchKernelGGL(enc_pages_kernel<D>, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream, a, (int)n);
    const int64_t nb = (n + kScanUnits - 1) / kScanUnits;
    if (ws == nullptr || ws_words < 2 + nb) {
        launch_scan<D>(a, n, stream);
        return;
    }
    const bool paged = a.dst_pages != nullptr;
    const bool vec16 = (uintptr_t)a.src % 16 == 0 && a.s_b % 8 == 0 && a.s_pg % 8 == 0 && a.s_p % 8 == 0 &&
                       a.s_h % 8 == 0;
    auto k = paged ? (vec16 ? scan_chain_kernel<true, true, D> : scan_chain_kernel<true, false, D>)
                   : (vec16 ? scan_chain_kernel<false, true, D> : scan_chain_kernel<false, false, D>);
    hipLaunchKernelGGL(k, dim3((unsigned)nb), dim3(kScanUnits), 0, stream, a, (int)n, (int)nb, ws);
}

static void launch_encode(const EncArgs& a, int64_t n, uint64_t* ws, int64_t ws_words, hipStream_t stream) {
    if (a.D == 64)
        launch_encode_d<64>(a, n, ws, ws_words, stream);
    else if (a.D == 256)
        launch_encode_d<256>(a, n, ws, ws_words, stream);
    else
        launch_encode_d<128>(a, n, ws, ws_words, stream);
}

// Copy one page's raw rows (token p's row at src + p*s_p, D channels) into slots rowoff + k (< cap).
template <int D>
__device__ inline void copy_raw_rows(const uint16_t* src, int64_t s_p, uint32_t m, int32_t off, int64_t cap,
                                     uint16_t* raw, int lane) {
    int k = 0;
    for (int p = 0; p < kPage; ++p) {
        if (!((m >> p) & 1u)) continue;
        const int64_t slot = (int64_t)off + k++;
        if (slot >= cap) continue;
        const uint16_t* s = src + p * s_p;
        uint16_t* d = raw + slot * D;
#pragma unroll
        for (int c = 0; c < D; c += 64) d[c + lane] = s[c + lane];
    }
}

// Row of D channels: d[c] = s[c], lanes striding by 64.
template <int D>
__device__ inline void copy_row(uint16_t* d, const uint16_t* s, int lane) {
#pragma unroll
    for (int c = 0; c < D; c += 64) d[c + lane] = s[c + lane];
}

// ---------------------------------------------------------------- device-side append

struct AppendArgs {
    const uint16_t* x;        // [B, H, D] (row strides sx_b, sx_h in elements)
    int64_t sx_b, sx_h;
    uint8_t* sm;
    uint8_t* code;
    uint8_t* base;
    int32_t* rowmask;
    int32_t* rowoff;
    uint16_t* raw;
    int32_t* cnt;
    int32_t* before;
    int32_t* state;           // state[0] = tokens held (T)
    int64_t cap;
    int B, H, TS;
};

// One append in one launch. Each wavefront takes (sequence, head) units u = its index,
// + the grid's wavefronts, ...: it writes the token into the unit's open page (the tail
// area) and, when the token completes page T/16, encodes the page (its rowmask stored
// device-coherently, for the last block) and opens the next one (rowmask all ones, rowoff
// into the tail area). Every block then counts itself in on state[1] (zero between calls)
// once its stores are complete; the last block to arrive -- which therefore follows every
// block's rowmask stores -- assigns the page's raw-row slots by an exclusive scan over the
// units in (sequence, head) order from *cnt (the codec's slot order), copies the raw rows
// (tokens 0-14 from the tail area, written by earlier appends; token 15 from x), sets
// *before and *cnt, and advances state[0]. Replaces three launches (write and encode, slot
// scan, raw-row copy), measured 0.87 ms of a c4 decode step for 64 caches.
constexpr int kAppendThreads = 1024;
// At most this many blocks: every block's arrival is an atomic on one word, and those
// serialise (measured at c4, 64 caches per step: 256 blocks 10.2 us per launch); the
// waves loop over the units instead.
constexpr int kAppendBlocks = 64;
constexpr int kAppendBatch = 8;                     // token rows a wave has in flight

__device__ inline void st_dev_i32(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int32_t ld_dev_i32(const int32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One raw row into the pool by one thread: src 4-byte aligned (x rows) or 16 (tail rows).
template <int D>
__device__ inline void copy_row_thread(uint16_t* dst, const uint16_t* src) {
    if (((uintptr_t)src & 15u) == 0) {
        for (int c0 = 0; c0 < 2 * D / 16; c0 += 8) {   // 16-byte pieces, eight in flight
            uint4 v[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) v[c] = reinterpret_cast<const uint4*>(src)[c0 + c];
#pragma unroll
            for (int c = 0; c < 8; ++c)                // registers, not a copy through the stack
                asm volatile("" : "+v"(v[c].x), "+v"(v[c].y), "+v"(v[c].z), "+v"(v[c].w));
#pragma unroll
            for (int c = 0; c < 8; ++c) reinterpret_cast<uint4*>(dst)[c0 + c] = v[c];
        }
    } else {
        for (int c0 = 0; c0 < D / 2; c0 += 16) {       // dwords, sixteen in flight
            uint32_t v[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) v[c] = reinterpret_cast<const uint32_t*>(src)[c0 + c];
#pragma unroll
            for (int c = 0; c < 16; ++c) asm volatile("" : "+v"(v[c]));
#pragma unroll
            for (int c = 0; c < 16; ++c) reinterpret_cast<uint32_t*>(dst)[c0 + c] = v[c];
        }
    }
}

// The last block's share of a page end (all kAppendThreads threads call it). Thread t takes
// units [t * per, (t + 1) * per): their rowmasks (device-coherent loads, eight in flight),
// the block's exclusive scan of their raw-row counts from *cnt (the codec's slot order),
// rowoff. Then the raw rows (rows 0-14 from the unit's tail area, written by earlier
// appends; row 15 from x): with up to kAppendLdsUnits units, spread over the threads one row
// each -- the units' first raw-row ranks go to LDS and the thread holding raw row g finds its
// unit by binary search -- so that a page end costs about one round trip; with more units,
// each thread moves its own units' rows. Rows at or past cap are not written (the counter
// shows the overflow).
constexpr int kAppendLdsUnits = 8192;

template <int D>
__device__ inline void append_slots(const AppendArgs& a, int T) {
    __shared__ int s_rank[kAppendLdsUnits + 1];
    __shared__ uint16_t s_mask[kAppendLdsUnits];
    const int n = a.B * a.H, NP = a.TS / kPage, pg = T / kPage;
    const int per = (n + kAppendThreads - 1) / kAppendThreads;
    const int u0 = min((int)threadIdx.x * per, n), u1 = min(u0 + per, n);
    auto page_of = [&](int u) { return ((int64_t)(u / a.H) * NP + pg) * a.H + u % a.H; };
    auto src_row = [&](int u, int r) -> const uint16_t* {
        return r == kPage - 1 ? a.x + (u / a.H) * a.sx_b + (u % a.H) * a.sx_h
                              : a.raw + (a.cap + (int64_t)u * kPage + r) * D;
    };
    const bool table = n <= kAppendLdsUnits;          // uniform
    const int cnt0 = *a.cnt;
    int local = 0;
    for (int c0 = u0; c0 < u1; c0 += 8) {
        uint32_t m[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) m[k] = c0 + k < u1 ? (uint32_t)ld_dev_i32(a.rowmask + page_of(c0 + k)) : 0u;
#pragma unroll
        for (int k = 0; k < 8; ++k) local += popc32(m[k]);
    }
    int total;
    int run = block_excl_scan(local, total);
    for (int c0 = u0; c0 < u1; c0 += 8) {
        uint32_t m[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) m[k] = c0 + k < u1 ? (uint32_t)ld_dev_i32(a.rowmask + page_of(c0 + k)) : 0u;
        for (int k = 0; k < 8 && c0 + k < u1; ++k) {
            const int u = c0 + k;
            a.rowoff[page_of(u)] = cnt0 + run;
            if (table) {
                s_rank[u] = run;
                s_mask[u] = (uint16_t)m[k];
            } else {
                int j = 0;
                for (int r = 0; r < kPage; ++r)
                    if ((m[k] >> r) & 1u) {
                        const int64_t slot = (int64_t)cnt0 + run + j++;
                        if (slot < a.cap) copy_row_thread<D>(a.raw + slot * D, src_row(u, r));
                    }
            }
            run += popc32(m[k]);
        }
    }
    if (table) {
        if (threadIdx.x == 0) s_rank[n] = total;
        __syncthreads();
        for (int g = threadIdx.x; g < total && (int64_t)cnt0 + g < a.cap; g += kAppendThreads) {
            int lo = 0, hi = n - 1;                    // the unit u with s_rank[u] <= g < s_rank[u + 1]
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_rank[mid] <= g) lo = mid; else hi = mid - 1;
            }
            const uint32_t m = s_mask[lo];
            int k = g - s_rank[lo], r = 0;             // g is the k-th raw row of unit lo's page
            for (; r < kPage - 1; ++r)
                if (((m >> r) & 1u) && k-- == 0) break;
            copy_row_thread<D>(a.raw + ((int64_t)cnt0 + g) * D, src_row(lo, r));
        }
    }
    if (threadIdx.x == 0) {
        *a.before = cnt0;
        *a.cnt = cnt0 + total;
    }
}

template <int D>
__global__ void __launch_bounds__(kAppendThreads) append_kernel(AppendArgs a) {
    const int T = a.state[0];
    if (T < 0 || T >= a.TS) return;                   // full cache: nothing is written (no block counts in)
    const int n = a.B * a.H, p = T % kPage, NP = a.TS / kPage, pg = T / kPage;
    const int lane = threadIdx.x & 63, wpb = kAppendThreads / 64;
    const int u0 = blockIdx.x * wpb + (int)(threadIdx.x >> 6), nw = (int)gridDim.x * wpb;
    // the token rows, kAppendBatch units at a time with all their loads in flight
    for (int ub = u0; ub < n; ub += kAppendBatch * nw) {
        uint16_t v[kAppendBatch][D / 64];
#pragma unroll
        for (int i = 0; i < kAppendBatch; ++i) {
            const int u = min(ub + i * nw, n - 1);
            const uint16_t* x = a.x + (u / a.H) * a.sx_b + (u % a.H) * a.sx_h;
#pragma unroll
            for (int c = 0; c < D / 64; ++c) v[i][c] = x[64 * c + lane];
        }
#pragma unroll
        for (int i = 0; i < kAppendBatch; ++i) {
            const int u = ub + i * nw;
            if (u >= n) break;
            uint16_t* tail = a.raw + (a.cap + (int64_t)u * kPage + p) * D;
#pragma unroll
            for (int c = 0; c < D / 64; ++c) tail[64 * c + lane] = v[i][c];
        }
    }
    // a page end: the page of every unit
    for (int u = u0; p == kPage - 1 && u < n; u += nw) {
        const int b = u / a.H, h = u % a.H;
        uint16_t* tail = a.raw + (a.cap + (int64_t)u * kPage) * D;
        const uint16_t* x = a.x + b * a.sx_b + h * a.sx_h;
        const int64_t row0 = ((int64_t)b * a.TS + (int64_t)pg * kPage) * a.H + h;
        const int64_t page = ((int64_t)b * NP + pg) * a.H + h;
        const uint32_t rm = encode_page<D>(tail, D, x, lane, a.sm + row0 * D, a.code + row0 * (D / 2), a.H,
                                           a.base + page * D, nullptr);
        if (lane == 0) {
            st_dev_i32(a.rowmask + page, (int32_t)rm);
            if (pg + 1 < NP) {
                a.rowmask[page + a.H] = 0xFFFF;
                a.rowoff[page + a.H] = (int32_t)(a.cap + (int64_t)u * kPage);
            }
        }
    }
    __shared__ int s_last;
    // at a page end the last block reads every unit's rowmask: this wave's stores are
    // complete before the block counts itself in; otherwise the count only orders every
    // block's read of state[0] before the last block's write of it
    if (p == kPage - 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(a.state + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    if (p == kPage - 1) append_slots<D>(a, T);
    __syncthreads();
    if (threadIdx.x == 0) {
        st_dev_i32(a.state + 1, 0);
        a.state[0] = T + 1;
    }
}

// Plain bf16 cache (reference cache.py:129-146): buf[b, T, h] = x[b, h], T from device.
template <int D>
__global__ void __launch_bounds__(256) bf16_append_kernel(const uint16_t* x, int64_t sx_b, int64_t sx_h,
                                                          uint16_t* buf, const int32_t* state, int B, int H,
                                                          int TS) {
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= B * H) return;
    const int T = state[0];
    if (T < 0 || T >= TS) return;
    const int b = u / H, h = u % H;
    copy_row<D>(buf + (((int64_t)b * TS + T) * H + h) * D, x + b * sx_b + h * sx_h, lane);
}

__global__ void bump_kernel(int32_t* state, int TS) {
    if (state[0] < TS) state[0] += 1;
}

// Opens the page that holds token state[0] of every (sequence, head): rowmask 0xFFFF and
// rowoff = cap + (b * H + h) * 16, the (sequence, head)'s rows after the escaped-row slots.
// The page index comes from the device token count, so the caches call it when they are
// filled and after their raw pool moves, without indexing the page table on the host.
// Nothing is written for a full cache (state[0] >= TS).
__global__ void __launch_bounds__(256) open_page_kernel(int32_t* rowmask, int32_t* rowoff, const int32_t* state,
                                                        int64_t cap, int B, int H, int TS) {
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
    const int T = state[0];
    if (u >= B * H || T < 0 || T >= TS) return;
    const int64_t page = ((int64_t)(u / H) * (TS / kPage) + T / kPage) * H + u % H;
    rowmask[page] = 0xFFFF;
    rowoff[page] = (int32_t)(cap + (int64_t)u * kPage);
}

// Paged caches: the same for sequence slots slots[0 .. n): slot s's open page is table entry
// lens[s] / 16 (when it exists), its rows at cap + (s * H + h) * 16.
__global__ void __launch_bounds__(256) open_pages_paged_kernel(int32_t* rowmask, int32_t* rowoff,
                                                               const int32_t* slots, int n, const int32_t* lens,
                                                               const int32_t* bt, int64_t bt_stride, int max_seqs,
                                                               int max_pages, int pool_pages, int64_t cap, int H) {
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n * H) return;
    const int s = (int)min((uint32_t)slots[u / H], (uint32_t)(max_seqs - 1)), h = u % H;
    const int T = lens[s];
    if (T < 0 || T / kPage >= max_pages) return;
    const int64_t pidx = min((uint32_t)bt[s * bt_stride + T / kPage], (uint32_t)(pool_pages - 1));
    rowmask[pidx * H + h] = 0xFFFF;
    rowoff[pidx * H + h] = (int32_t)(cap + ((int64_t)s * H + h) * kPage);
}

// ---------------------------------------------------------------- paged append

// One token for each of n sequences held in a pool of pages. Sequence slot s (batch row i
// -> s = slots[i], or i) owns pool pages bt[s * bt_stride + pg] (clamped to the pool) and
// has lens[s] tokens, the new one included: the caller raises lens before the append, so
// the new token is token lens[s] - 1 and the kernels never write lens. Its open page is
// held in the tail area at raw rows cap + (s * H + h) * 16; when the new token fills it,
// the page is encoded into its pool page and the next table entry is opened.
struct PagedAppendArgs {
    const uint16_t* x;        // [n, H, D] (row strides sx_b, sx_h in elements)
    int64_t sx_b, sx_h;
    uint8_t* sm;
    uint8_t* code;
    uint8_t* base;
    int32_t* rowmask;
    int32_t* rowoff;
    uint16_t* raw;
    int32_t* cnt;
    int32_t* before;
    const int32_t* slots;     // [n] or nullptr
    const int32_t* lens;      // [max_seqs]
    const int32_t* bt;        // [max_seqs, bt_stride]
    int64_t bt_stride;
    int64_t cap;
    int n, H, max_seqs, max_pages, pool_pages;
};

__device__ inline int paged_slot(const PagedAppendArgs& a, int i) {
    return a.slots ? min((uint32_t)a.slots[i], (uint32_t)(a.max_seqs - 1)) : i;
}
__device__ inline int64_t paged_pidx(const PagedAppendArgs& a, int s, int pg) {
    return (int64_t)min((uint32_t)a.bt[s * a.bt_stride + pg], (uint32_t)(a.pool_pages - 1));
}
// Token index of the new token of slot s, or -1 if it does not fit.
__device__ inline int paged_new_token(const PagedAppendArgs& a, int s) {
    const int T = a.lens[s] - 1;
    return (T >= 0 && T < a.max_pages * kPage) ? T : -1;
}

template <int D>
__global__ void __launch_bounds__(256) paged_append_write_kernel(PagedAppendArgs a) {
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= a.n * a.H) return;
    const int i = u / a.H, h = u % a.H;
    const int s = paged_slot(a, i);
    const int T = paged_new_token(a, s);
    if (T < 0) return;
    const int p = T % kPage;
    const int64_t tslot = a.cap + ((int64_t)s * a.H + h) * kPage;
    uint16_t* tail = a.raw + tslot * D;
    const uint16_t* x = a.x + i * a.sx_b + h * a.sx_h;
    copy_row<D>(tail + p * D, x, lane);
    if (p != kPage - 1) return;
    const int pg = T / kPage;
    const int64_t pidx = paged_pidx(a, s, pg);
    const int64_t row0 = pidx * kPage * a.H + h;
    const int64_t page = pidx * a.H + h;
    encode_page<D>(tail, D, x, lane, a.sm + row0 * D, a.code + row0 * (D / 2), a.H, a.base + page * D,
                   a.rowmask + page);
    if (pg + 1 < a.max_pages && lane == 0) {
        const int64_t next = paged_pidx(a, s, pg + 1) * a.H + h;
        a.rowmask[next] = 0xFFFF;
        a.rowoff[next] = (int32_t)tslot;
    }
}

// Raw slots for the pages filled by this append, in (batch row, head, token) order.
__global__ void __launch_bounds__(1024) paged_append_scan_kernel(PagedAppendArgs a) {
    const int n = a.n * a.H;
    const int per = (n + 1023) / 1024;
    const int u0 = threadIdx.x * per, u1 = min(u0 + per, n);
    const int cnt0 = *a.cnt;
    int local = 0, filled = 0;
    for (int u = u0; u < u1; ++u) {
        const int s = paged_slot(a, u / a.H);
        const int T = paged_new_token(a, s);
        if (T < 0 || T % kPage != kPage - 1) continue;
        filled = 1;
        local += popc32((uint32_t)a.rowmask[paged_pidx(a, s, T / kPage) * a.H + u % a.H]);
    }
    const int any = __syncthreads_or(filled);
    if (!any) return;                                  // uniform: no page filled, counter untouched
    int total;
    int run = cnt0 + block_excl_scan(local, total);
    for (int u = u0; u < u1; ++u) {
        const int s = paged_slot(a, u / a.H);
        const int T = paged_new_token(a, s);
        if (T < 0 || T % kPage != kPage - 1) continue;
        const int64_t page = paged_pidx(a, s, T / kPage) * a.H + u % a.H;
        a.rowoff[page] = run;
        run += popc32((uint32_t)a.rowmask[page]);
    }
    if (threadIdx.x == 0) {
        *a.before = cnt0;
        *a.cnt = cnt0 + total;
    }
}

template <int D>
__global__ void __launch_bounds__(256) paged_append_rawcopy_kernel(PagedAppendArgs a) {
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= a.n * a.H) return;
    const int h = u % a.H;
    const int s = paged_slot(a, u / a.H);
    const int T = paged_new_token(a, s);
    if (T < 0 || T % kPage != kPage - 1) return;
    const int64_t page = paged_pidx(a, s, T / kPage) * a.H + h;
    const uint32_t m = (uint32_t)a.rowmask[page];
    if (m == 0) return;
    copy_raw_rows<D>(a.raw + (a.cap + ((int64_t)s * a.H + h) * kPage) * D, D, m, a.rowoff[page], a.cap, a.raw,
                     lane);
}

// bf16 twin: pool[(page * 16 + T % 16) * H + h] = x[i, h], page = bt[s, T / 16].
template <int D>
__global__ void __launch_bounds__(256) paged_bf16_append_kernel(PagedAppendArgs a, uint16_t* buf) {
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= a.n * a.H) return;
    const int i = u / a.H, h = u % a.H;
    const int s = paged_slot(a, i);
    const int T = paged_new_token(a, s);
    if (T < 0) return;
    const int64_t row = paged_pidx(a, s, T / kPage) * kPage + T % kPage;
    copy_row<D>(buf + (row * a.H + h) * D, a.x + i * a.sx_b + h * a.sx_h, lane);
}

// ---------------------------------------------------------------- decode to bf16

struct DecArgs {
    CSrc c;
    uint16_t* out;            // [B, T, H, D]
    int B, T, TS, H;
    // paged: page pg of sequence b is pool page bt[b * bt_stride + pg] (clamped to pool_pages)
    const int32_t* bt = nullptr;
    int64_t bt_stride = 0;
    int64_t pool_pages = 0;
};

// One wavefront per (sequence, page, head), lane = (token r, channel group g): the page
// rebuild of the attention kernels (tile.hpp), any head dim.
template <int D>
__global__ void __launch_bounds__(256) decode_kernel(DecArgs a) {
    constexpr int R = Run<D>::R;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int NP = a.TS / kPage;
    const int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= (int64_t)a.B * NP * a.H) return;
    const int h = (int)(u % a.H);
    const int pg = (int)((u / a.H) % NP);
    const int b = (int)(u / ((int64_t)a.H * NP));
    if (pg * kPage >= a.T) return;
    const int t = pg * kPage + r;
    const int64_t pidx = a.bt ? (int64_t)min((uint32_t)a.bt[b * a.bt_stride + pg], (uint32_t)(a.pool_pages - 1))
                              : (int64_t)b * NP + pg;
    const int64_t page = pidx * a.H + h;
    PageBytesD<D> pb;
    load_page_d<D>(a.c, (pidx * kPage + r) * a.H + h, page, g, pb);
    const uint32_t rmask = (uint32_t)a.c.rowmask[page];
    const int32_t roff = a.c.rowoff[page];
    uint32_t v[Run<D>::V];
    rebuild_page_d<D>(a.c, pb, rmask, roff, r, g, v);
    if (t >= a.T) return;
    uint16_t* o = a.out + (((int64_t)b * a.T + t) * a.H + h) * D + g * R;
    st_words<R / 2>(o, v);
    st_words<R / 2>(o + D / 2, v + R / 2);
}

template <int D>
static void launch_decode(const DecArgs& a, int64_t n, hipStream_t stream) {
    hipLaunchKernelGGL(decode_kernel<D>, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream, a);
}
static void launch_decode_any(int D, const DecArgs& a, int64_t n, hipStream_t stream) {
    if (D == 64)
        launch_decode<64>(a, n, stream);
    else if (D == 256)
        launch_decode<256>(a, n, stream);
    else
        launch_decode<128>(a, n, stream);
}

}  // namespace exkv

using namespace exkv;

static int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

// The instance of kernel template K for head dim D (64, 128 or 256; checked by the caller).
#define EXKV_FOR_D(K, D) ((D) == 64 ? K<64> : (D) == 256 ? K<256> : K<128>)

extern "C" int exkv_encode_pages(const void* src, int64_t s_b, int64_t s_pg, int64_t s_p, int64_t s_h,
                                 void* sm, void* code, void* base, int32_t* rowmask, int32_t* rowoff, void* raw,
                                 int32_t* cnt, int32_t* before, int64_t cap, int64_t raw_rows, int32_t B,
                                 int32_t b0, int32_t pg0, int32_t nb, int32_t npg, int32_t H, int32_t TS,
                                 int32_t D, void* scan_ws, int64_t scan_ws_words, hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "encode_pages: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0, "encode_pages: TS must be a positive multiple of 16 (got %d)", TS);
    EXKV_REQUIRE(H > 0 && B > 0, "encode_pages: bad H=%d or B=%d", H, B);
    EXKV_REQUIRE(nb >= 0 && npg >= 0 && b0 >= 0 && pg0 >= 0, "encode_pages: negative range");
    EXKV_REQUIRE(b0 + nb <= B, "encode_pages: sequences [%d, %d) outside the cache (B=%d)", b0, b0 + nb, B);
    EXKV_REQUIRE(pg0 + npg <= TS / kPage, "encode_pages: pages [%d, %d) outside the cache (%d pages)", pg0,
                 pg0 + npg, TS / kPage);
    EXKV_REQUIRE(cap >= 0 && cap <= raw_rows, "encode_pages: cap %lld exceeds the raw pool (%lld rows)",
                 (long long)cap, (long long)raw_rows);
    EXKV_REQUIRE(src && sm && code && base && rowmask && rowoff && raw && cnt, "encode_pages: null pointer");
    EXKV_REQUIRE((uintptr_t)src % 4 == 0 && s_b % 2 == 0 && s_pg % 2 == 0 && s_p % 2 == 0 && s_h % 2 == 0,
                 "encode_pages: source rows must start at even elements (4-byte aligned)");
    const int64_t n = (int64_t)nb * npg * H;
    if (n == 0) return EXKV_OK;
    EXKV_REQUIRE(n <= INT32_MAX - 1024, "encode_pages: %lld pages x heads in one call (limit 2^31 - 1025)",
                 (long long)n);
    EXKV_REQUIRE(scan_ws == nullptr || (uintptr_t)scan_ws % 8 == 0, "encode_pages: scan workspace must be 8-byte aligned");
    EncArgs a{(const uint16_t*)src, s_b, s_pg, s_p, s_h, (uint8_t*)sm, (uint8_t*)code, (uint8_t*)base,
              rowmask, rowoff, (uint16_t*)raw, cnt, before, cap, b0, pg0, nb, npg, H, TS};
    a.D = D;
    launch_encode(a, n, (uint64_t*)scan_ws, scan_ws_words, stream);
    return launch_status("encode_pages");
}

// Pages of nb source sequences x npg pages into arbitrary pages of B x TS caches read as a
// list of B * TS / 16 pages: page pg of source sequence bi goes to page dst_pages[bi *
// dst_stride + pg]. Same kernels, raw-slot order (unit order) and bytes as
// exkv_encode_pages.
extern "C" int exkv_encode_pages_paged(const void* src, int64_t s_b, int64_t s_pg, int64_t s_p, int64_t s_h,
                                       void* sm, void* code, void* base, int32_t* rowmask, int32_t* rowoff,
                                       void* raw, int32_t* cnt, int32_t* before, int64_t cap, int64_t raw_rows,
                                       int32_t B, const int32_t* dst_pages, int64_t dst_stride, int32_t nb,
                                       int32_t npg, int32_t H, int32_t TS, int32_t D, void* scan_ws,
                                       int64_t scan_ws_words, hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "encode_pages_paged: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0, "encode_pages_paged: TS must be a positive multiple of 16 (got %d)", TS);
    EXKV_REQUIRE(H > 0 && B > 0, "encode_pages_paged: bad H=%d or B=%d", H, B);
    EXKV_REQUIRE(nb >= 0 && npg >= 0, "encode_pages_paged: negative range");
    EXKV_REQUIRE(dst_pages && dst_stride >= npg, "encode_pages_paged: need a page table of >= %d columns", npg);
    EXKV_REQUIRE(cap >= 0 && cap <= raw_rows, "encode_pages_paged: cap %lld exceeds the raw pool (%lld rows)",
                 (long long)cap, (long long)raw_rows);
    EXKV_REQUIRE(src && sm && code && base && rowmask && rowoff && raw && cnt, "encode_pages_paged: null pointer");
    EXKV_REQUIRE((uintptr_t)src % 4 == 0 && s_b % 2 == 0 && s_pg % 2 == 0 && s_p % 2 == 0 && s_h % 2 == 0,
                 "encode_pages_paged: source rows must start at even elements (4-byte aligned)");
    const int64_t n = (int64_t)nb * npg * H;
    if (n == 0) return EXKV_OK;
    EXKV_REQUIRE(n <= INT32_MAX - 1024, "encode_pages_paged: %lld pages x heads in one call (limit 2^31 - 1025)",
                 (long long)n);
    EncArgs a{(const uint16_t*)src, s_b, s_pg, s_p, s_h, (uint8_t*)sm, (uint8_t*)code, (uint8_t*)base,
              rowmask, rowoff, (uint16_t*)raw, cnt, before, cap, 0, 0, nb, npg, H, TS};
    a.dst_pages = dst_pages;
    a.dst_stride = dst_stride;
    a.all_pages = (int64_t)B * (TS / kPage);
    a.D = D;
    EXKV_REQUIRE(scan_ws == nullptr || (uintptr_t)scan_ws % 8 == 0,
                 "encode_pages_paged: scan workspace must be 8-byte aligned");
    launch_encode(a, n, (uint64_t*)scan_ws, scan_ws_words, stream);
    return launch_status("encode_pages_paged");
}

extern "C" int exkv_cache_append(const void* x, int64_t sx_b, int64_t sx_h, void* sm, void* code, void* base,
                                 int32_t* rowmask, int32_t* rowoff, void* raw, int32_t* cnt, int32_t* before,
                                 int32_t* state, int64_t cap, int64_t raw_rows, int32_t B, int32_t H,
                                 int32_t TS, int32_t D, hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "append: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0 && B > 0 && H > 0, "append: bad shape B=%d H=%d TS=%d", B, H, TS);
    EXKV_REQUIRE(cap >= 0 && cap + (int64_t)B * H * kPage <= raw_rows,
                 "append: raw pool (%lld rows) smaller than cap + tail area", (long long)raw_rows);
    EXKV_REQUIRE(x && sm && code && base && rowmask && rowoff && raw && cnt && before && state,
                 "append: null pointer");
    EXKV_REQUIRE((uintptr_t)x % 4 == 0 && sx_b % 2 == 0 && sx_h % 2 == 0,
                 "append: token rows must start at even elements (4-byte aligned)");
    AppendArgs a{(const uint16_t*)x, sx_b, sx_h, (uint8_t*)sm, (uint8_t*)code, (uint8_t*)base, rowmask, rowoff,
                 (uint16_t*)raw, cnt, before, state, cap, B, H, TS};
    const int64_t blocks = ((int64_t)B * H + kAppendThreads / 64 - 1) / (kAppendThreads / 64);   // a unit per wave
    const unsigned grid = (unsigned)(blocks < kAppendBlocks ? blocks : kAppendBlocks);
    hipLaunchKernelGGL(EXKV_FOR_D(append_kernel, D), dim3(grid), dim3(kAppendThreads), 0, stream, a);
    return launch_status("cache_append");
}

extern "C" int exkv_bf16_append(const void* x, int64_t sx_b, int64_t sx_h, void* buf, int32_t* state,
                                int32_t B, int32_t H, int32_t TS, int32_t D, hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "bf16_append: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(B > 0 && H > 0 && TS > 0, "bf16_append: bad shape");
    EXKV_REQUIRE(x && buf && state, "bf16_append: null pointer");
    hipLaunchKernelGGL(EXKV_FOR_D(bf16_append_kernel, D), dim3((unsigned)((B * H + 3) / 4)), dim3(256), 0, stream,
                       (const uint16_t*)x, sx_b, sx_h, (uint16_t*)buf, (const int32_t*)state, B, H, TS);
    hipLaunchKernelGGL(bump_kernel, dim3(1), dim3(1), 0, stream, state, TS);
    return launch_status("bf16_append");
}

extern "C" int exkv_cache_open_page(int32_t* rowmask, int32_t* rowoff, const int32_t* state, int64_t cap,
                                    int64_t raw_rows, int32_t B, int32_t H, int32_t TS, hipStream_t stream) {
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0 && B > 0 && H > 0, "open_page: bad shape B=%d H=%d TS=%d", B, H, TS);
    EXKV_REQUIRE(cap >= 0 && cap + (int64_t)B * H * kPage <= raw_rows && cap + (int64_t)B * H * kPage <= INT32_MAX,
                 "open_page: raw pool (%lld rows) smaller than cap + tail area", (long long)raw_rows);
    EXKV_REQUIRE(rowmask && rowoff && state, "open_page: null pointer");
    hipLaunchKernelGGL(open_page_kernel, dim3((unsigned)((B * H + 255) / 256)), dim3(256), 0, stream, rowmask,
                       rowoff, state, cap, B, H, TS);
    return launch_status("cache_open_page");
}

extern "C" int exkv_cache_open_pages_paged(int32_t* rowmask, int32_t* rowoff, const int32_t* slots, int32_t n,
                                           const int32_t* lens, const int32_t* block_table, int64_t bt_stride,
                                           int32_t max_seqs, int32_t max_pages, int32_t pool_pages, int64_t cap,
                                           int64_t raw_rows, int32_t H, hipStream_t stream) {
    EXKV_REQUIRE(n >= 0 && n <= max_seqs && H > 0 && max_pages > 0 && bt_stride >= max_pages && pool_pages > 0,
                 "open_pages_paged: bad shape n=%d H=%d max_seqs=%d max_pages=%d", n, H, max_seqs, max_pages);
    EXKV_REQUIRE(cap >= 0 && cap + (int64_t)max_seqs * H * kPage <= raw_rows &&
                     cap + (int64_t)max_seqs * H * kPage <= INT32_MAX,
                 "open_pages_paged: raw pool (%lld rows) smaller than cap + tail area", (long long)raw_rows);
    EXKV_REQUIRE(rowmask && rowoff && lens && block_table && (slots || n == 0), "open_pages_paged: null pointer");
    if (n == 0) return EXKV_OK;
    hipLaunchKernelGGL(open_pages_paged_kernel, dim3((unsigned)((n * H + 255) / 256)), dim3(256), 0, stream,
                       rowmask, rowoff, slots, n, lens, block_table, bt_stride, max_seqs, max_pages, pool_pages, cap,
                       H);
    return launch_status("cache_open_pages_paged");
}

static int check_paged_append(const char* what, int32_t n, int32_t H, int32_t D, int32_t max_seqs,
                              int32_t max_pages, int64_t bt_stride, int32_t pool_pages) {
    EXKV_REQUIRE(head_dim_ok(D), "%s: head dim must be 64, 128 or 256 (got %d)", what, D);
    EXKV_REQUIRE(n >= 0 && H > 0 && max_seqs > 0 && n <= max_seqs, "%s: bad shape n=%d H=%d max_seqs=%d", what, n,
                 H, max_seqs);
    EXKV_REQUIRE(max_pages > 0 && bt_stride >= max_pages && pool_pages > 0,
                 "%s: bad page table (max_pages=%d stride=%lld pool=%d)", what, max_pages, (long long)bt_stride,
                 pool_pages);
    return EXKV_OK;
}

extern "C" int exkv_cache_append_paged(const void* x, int64_t sx_b, int64_t sx_h, void* sm, void* code, void* base,
                                       int32_t* rowmask, int32_t* rowoff, void* raw, int32_t* cnt, int32_t* before,
                                       int64_t cap, int64_t raw_rows, const int32_t* slots, const int32_t* lens,
                                       const int32_t* block_table, int64_t bt_stride, int32_t n, int32_t H,
                                       int32_t max_seqs, int32_t max_pages, int32_t pool_pages, int32_t D,
                                       hipStream_t stream) {
    const int rc = check_paged_append("append_paged", n, H, D, max_seqs, max_pages, bt_stride, pool_pages);
    if (rc != EXKV_OK) return rc;
    EXKV_REQUIRE(cap >= 0 && cap + (int64_t)max_seqs * H * kPage <= raw_rows,
                 "append_paged: raw pool (%lld rows) smaller than cap + tail area", (long long)raw_rows);
    EXKV_REQUIRE(x && sm && code && base && rowmask && rowoff && raw && cnt && before && lens && block_table,
                 "append_paged: null pointer");
    EXKV_REQUIRE((uintptr_t)x % 4 == 0 && sx_b % 2 == 0 && sx_h % 2 == 0,
                 "append_paged: token rows must start at even elements (4-byte aligned)");
    if (n == 0) return EXKV_OK;
    PagedAppendArgs a{(const uint16_t*)x, sx_b, sx_h, (uint8_t*)sm, (uint8_t*)code, (uint8_t*)base, rowmask,
                      rowoff, (uint16_t*)raw, cnt, before, slots, lens, block_table, bt_stride, cap, n, H,
                      max_seqs, max_pages, pool_pages};
    const unsigned grid = (unsigned)((n * H + 3) / 4);
    hipLaunchKernelGGL(EXKV_FOR_D(paged_append_write_kernel, D), dim3(grid), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(paged_append_scan_kernel, dim3(1), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(EXKV_FOR_D(paged_append_rawcopy_kernel, D), dim3(grid), dim3(256), 0, stream, a);
    return launch_status("cache_append_paged");
}

extern "C" int exkv_bf16_append_paged(const void* x, int64_t sx_b, int64_t sx_h, void* buf, const int32_t* slots,
                                      const int32_t* lens, const int32_t* block_table, int64_t bt_stride, int32_t n,
                                      int32_t H, int32_t max_seqs, int32_t max_pages, int32_t pool_pages, int32_t D,
                                      hipStream_t stream) {
    const int rc = check_paged_append("bf16_append_paged", n, H, D, max_seqs, max_pages, bt_stride, pool_pages);
    if (rc != EXKV_OK) return rc;
    EXKV_REQUIRE(x && buf && lens && block_table, "bf16_append_paged: null pointer");
    if (n == 0) return EXKV_OK;
    PagedAppendArgs a{(const uint16_t*)x, sx_b, sx_h, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                      nullptr, nullptr, slots, lens, block_table, bt_stride, 0, n, H, max_seqs, max_pages,
                      pool_pages};
    hipLaunchKernelGGL(EXKV_FOR_D(paged_bf16_append_kernel, D), dim3((unsigned)((n * H + 3) / 4)), dim3(256), 0,
                       stream, a, (uint16_t*)buf);
    return launch_status("bf16_append_paged");
}

extern "C" int exkv_decode_to_bf16_paged(const void* sm, const void* code, const void* base,
                                         const int32_t* rowmask, const int32_t* rowoff, const void* raw,
                                         int64_t raw_rows, int64_t pool_pages, const int32_t* block_table,
                                         int64_t bt_stride, void* out, int32_t B, int32_t T, int32_t H, int32_t D,
                                         hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "decode_to_bf16_paged: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(B > 0 && H > 0 && bt_stride > 0 && pool_pages > 0, "decode_to_bf16_paged: bad shape");
    EXKV_REQUIRE(T >= 0 && T <= bt_stride * kPage, "decode_to_bf16_paged: T=%d exceeds the table's %lld pages", T,
                 (long long)bt_stride);
    EXKV_REQUIRE(raw_rows > 0, "decode_to_bf16_paged: empty raw pool");
    EXKV_REQUIRE(sm && code && base && rowmask && rowoff && raw && out && block_table,
                 "decode_to_bf16_paged: null pointer");
    if (T == 0) return EXKV_OK;
    const int TS = (T + kPage - 1) / kPage * kPage;     // pages the tokens touch
    DecArgs a{CSrc{(const uint8_t*)sm, (const uint8_t*)code, (const uint8_t*)base, rowmask, rowoff,
                   (const uint16_t*)raw, raw_rows},
              (uint16_t*)out, B, T, TS, H};
    a.bt = block_table;
    a.bt_stride = bt_stride;
    a.pool_pages = pool_pages;
    launch_decode_any(D, a, (int64_t)B * (TS / kPage) * H, stream);
    return launch_status("decode_to_bf16_paged");
}

extern "C" int exkv_decode_to_bf16(const void* sm, const void* code, const void* base, const int32_t* rowmask,
                                   const int32_t* rowoff, const void* raw, int64_t raw_rows, void* out,
                                   int32_t B, int32_t T, int32_t TS, int32_t H, int32_t D, hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "decode_to_bf16: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0 && B > 0 && H > 0, "decode_to_bf16: bad shape");
    EXKV_REQUIRE(T >= 0 && T <= TS, "decode_to_bf16: T=%d outside [0, TS=%d]", T, TS);
    EXKV_REQUIRE(raw_rows > 0, "decode_to_bf16: empty raw pool");
    EXKV_REQUIRE(sm && code && base && rowmask && rowoff && raw && out, "decode_to_bf16: null pointer");
    if (T == 0) return EXKV_OK;
    DecArgs a{CSrc{(const uint8_t*)sm, (const uint8_t*)code, (const uint8_t*)base, rowmask, rowoff,
                   (const uint16_t*)raw, raw_rows},
              (uint16_t*)out, B, T, TS, H};
    launch_decode_any(D, a, (int64_t)B * (TS / kPage) * H, stream);
    return launch_status("decode_to_bf16");
}

namespace exkv {
hipError_t fetch_errors_encode(uint32_t* out, int first, int clear, hipStream_t stream) {
    return fetch_file_errors(out, first, clear, stream);
}
}  // namespace exkv
