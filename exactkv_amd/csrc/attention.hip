// Split-K GQA decode attention for gfx950, over the compressed cache or over plain bf16.
//
// Reference: exactkv/kernels.py _split_c_kernel :142-165, _split_ref_kernel :168-194,
// _attn_block :46-59, _reduce_kernel :33-43.
//
// Grid: x = token split, y = (sequence, KV head, group of 16 query heads). A workgroup is
// 8 wavefronts (one workgroup per CU: it owns ~150 KB of LDS). The wavefronts take the
// split's 16-token pages round robin, each with its own online-softmax state, and are
// merged through LDS at the end (one partial per split).
//
// Memory pipeline (per wavefront): each page is brought into a private LDS ring with a
// fixed number (kDmaPerPage) of direct-to-LDS loads (global_load_lds_dwordx4/_dword), two
// pages ahead for the compressed cache (3-stage ring) and one ahead for bf16 (2 stages).
// The compiler does not order LDS reads after these loads, so every stage is read only
// after an explicit s_waitcnt vmcnt(N) whose N counts the younger loads in flight. Rows
// are placed with XOR swizzles chosen so that the later LDS reads are conflict-free.
//
// Per page:
//   * K and V are rebuilt bit-exactly in VGPRs from the staged bytes (tile.hpp), lane =
//     token; raw rows are spliced in from loads issued before the next page's DMA (so the
//     compiler's own wait for them counts only that younger batch).
//   * S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (tokens = rows, the G query heads of the
//     KV head = columns, padded to 16); online softmax in base 2, scores scaled by
//     D^-1/2 log2(e), p rounded to bf16 for P.V, l summed from fp32 p.
//   * V goes back to LDS as a bf16 row tile (the compressed stage is consumed by then;
//     the bf16 twin's stage already holds that tile), and ds_read_b64_tr_b16 reads it as
//     the V^T operand of v_mfma_f32_16x16x16_bf16; the C layout of S^T is exactly the
//     P^T operand layout, and O^T accumulates with lane = head, so the softmax rescale
//     needs no cross-lane traffic.
// Everything after the K/V rebuild is shared by the two kernels, so the compressed and
// uncompressed results are identical bit for bit.
#include "tile.hpp"
#include "../../include/exactkv.h"

#define EXKV_LDS __attribute__((address_space(3)))

namespace exkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kDmaPerPage = 8;        // direct-to-LDS loads per page, both kernels

// compressed page stage (bytes): K sm 16x128 | K code 16x64 | V sm | V code | K base,
// V base (128 each) | meta (K rowmask, K rowoff, V rowmask, V rowoff)
constexpr int CS_KSM = 0, CS_KCODE = 2048, CS_VSM = 3072, CS_VCODE = 5120, CS_BASE = 6144,
              CS_META = 6400, CS_BYTES = 6416;
// bf16 page stage: K rows 16x256 | V rows 16x256
constexpr int BS_K = 0, BS_V = 4096, BS_BYTES = 8192;

template <bool COMP>
struct Ring {
    static constexpr int stage = COMP ? CS_BYTES : BS_BYTES;
    static constexpr int nst = COMP ? 3 : 2;
    static constexpr int vtile = COMP ? 0 : BS_V;    // offset of the bf16 V tile in a stage
    static constexpr int bytes = kWaves * nst * stage;
};

struct AttnArgs {
    const uint16_t* q;        // [B, Hq, 128] bf16
    CSrc k, v;                // compressed caches
    const uint16_t* kb;       // bf16 caches [B, TS, Hkv, 128] (twin)
    const uint16_t* vb;
    float* part_o;            // [B*Hq, nsplit, 128]
    float* part_m;            // [B*Hq, nsplit]
    float* part_l;
    const int32_t* lens;      // per-sequence valid tokens (nullptr: T for all)
    int64_t lens_stride;
    int B, Hq, Hkv, G, HG, TS, T, nsplit, split_len;
    int HW;                   // KV heads per workgroup (gcd(Hkv, 8)); 8 / HW page phases per head
    float qk_scale;
    uint16_t* out;            // [B, Hq, 128] bf16, written by the last workgroup of each unit
    int32_t* counters;        // [gridDim.y] arrival counters (zero between calls); nullptr: no merge
};

// ---- split merge (kernels.py:33-43): M = max_s m_s, w_s = 2^(m_s - M),
// out = sum_s o_s w_s / sum_s l_s w_s. Shared by the fused merge and attn_reduce_kernel so
// both produce the same bits.
__device__ inline float fast_exp2(float x);
__device__ inline float split_max(const float* m, int ns) {
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, m[s]);
    return M;
}
__device__ inline uint32_t merge_pair(const float* po, const float* m, const float* l, int ns, float M, int dp) {
    float n0 = 0.f, n1 = 0.f, den = 0.f;
    int s = 0;
    for (; s + 8 <= ns; s += 8) {                      // 8 splits' loads in flight at once
        float2 o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = reinterpret_cast<const float2*>(po + (int64_t)(s + i) * kD)[dp];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float w = fast_exp2(m[s + i] - M);
            n0 += o[i].x * w;
            n1 += o[i].y * w;
            den += l[s + i] * w;
        }
    }
    for (; s < ns; ++s) {
        const float w = fast_exp2(m[s] - M);
        const float2 o = reinterpret_cast<const float2*>(po + (int64_t)s * kD)[dp];
        n0 += o.x * w;
        n1 += o.y * w;
        den += l[s] * w;
    }
    const __bf16 r0 = (__bf16)(n0 / den), r1 = (__bf16)(n1 / den);
    return (uint32_t)__builtin_bit_cast(uint16_t, r0) | ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
}

__device__ inline bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 u = {a, b, c, d};
    return __builtin_bit_cast(bf16x8, u);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Direct-to-LDS loads (each lane's 16 or 4 bytes land at lds + lane * size). Issued as
// inline assembly so that the compiler does not pair them with the later LDS reads (it
// would otherwise wait for every outstanding LDS load before any LDS read, which drains
// the ring); the kernel orders them itself with wait_vm. M0 carries the LDS address.
__device__ inline uint32_t lds_addr(const uint8_t* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const EXKV_LDS uint8_t*)p);
}
__device__ inline void dma16(const void* g, uint8_t* lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}
__device__ inline void dma4(const void* g, uint8_t* lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}

// Mark registers as defined here (an empty asm that reads and writes them): the compiler
// then waits for their loads at this point, once, instead of at every later use inside
// the page loop, where its vmcnt(0) would also wait for the ring's loads in flight.
template <int N>
__device__ inline void settle(uint32_t (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}

// Wait until at most n vector-memory loads of this wavefront are in flight, and keep the
// compiler from moving memory accesses across the wait.
template <int N>
__device__ inline void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}


// Per-lane parts of a page's DMA addresses (fixed for the kernel): byte offsets from the
// page's first row in each array, with the XOR swizzle of the destination applied.
struct DmaLane {
    uint32_t sm0, sm1, code, base, bf_k[4], bf_v[4];
};

template <bool COMP>
__device__ inline DmaLane dma_lane_offsets(int lane, int64_t rs) {
    DmaLane o{};
    if constexpr (COMP) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {                  // sm: 8 rows per load, 16-B segment ^= row & 7
            const int row = 8 * j + (lane >> 3);
            const uint32_t off = (uint32_t)(row * rs * 128 + ((lane & 7) ^ (row & 7)) * 16);
            (j ? o.sm1 : o.sm0) = off;
        }
        const int crow = lane >> 2;                    // code: 16 rows, segment ^= (row >> 1) & 3
        o.code = (uint32_t)(crow * rs * 64 + ((lane & 3) ^ ((crow >> 1) & 3)) * 16);
        o.base = (uint32_t)((lane & 7) * 16);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {                  // 4 rows of 256 B per load
            const int row = 4 * j + (lane >> 4);
            o.bf_k[j] = (uint32_t)(row * rs * 256 + 16 * ((lane & 15) ^ (row & 7)));
            o.bf_v[j] = (uint32_t)(row * rs * 256 + 16 * ((lane & 15) ^ ((row & 3) << 1)));
        }
    }
    return o;
}

// Issue one page's kDmaPerPage loads into stage st. row0: row index of the page's token 0
// ((b*TS + 16*pg)*Hkv + hk); page: its page index.
template <bool COMP>
__device__ inline void dma_page(const AttnArgs& a, const DmaLane& o, int64_t row0, int64_t page, uint8_t* st,
                                int lane) {
    if constexpr (COMP) {
        const uint8_t* ksm = a.k.sm + row0 * 128;
        const uint8_t* vsm = a.v.sm + row0 * 128;
        dma16(ksm + o.sm0, st + CS_KSM);
        dma16(vsm + o.sm0, st + CS_VSM);
        dma16(ksm + o.sm1, st + CS_KSM + 1024);
        dma16(vsm + o.sm1, st + CS_VSM + 1024);
        dma16(a.k.code + row0 * 64 + o.code, st + CS_KCODE);
        dma16(a.v.code + row0 * 64 + o.code, st + CS_VCODE);
        // base rows (lanes 0-7 K, 8-15 V) and meta (lanes 0-3: K rowmask, K rowoff, V rowmask,
        // V rowoff): addresses picked with bit-test selects of values already in registers
        const uint8_t* bsrc = ((lane & 8) ? a.v.base : a.k.base) + page * 128 + o.base;
        if (lane < 16) dma16(bsrc, st + CS_BASE);
        const int32_t* mk = (lane & 1) ? a.k.rowoff : a.k.rowmask;
        const int32_t* mv = (lane & 1) ? a.v.rowoff : a.v.rowmask;
        if (lane < 4) dma4(((lane & 2) ? mv : mk) + page, st + CS_META);
    } else {
        const uint8_t* kp = reinterpret_cast<const uint8_t*>(a.kb) + row0 * 256;
        const uint8_t* vp = reinterpret_cast<const uint8_t*>(a.vb) + row0 * 256;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dma16(kp + o.bf_k[j], st + BS_K + j * 1024);
            dma16(vp + o.bf_v[j], st + BS_V + j * 1024);
        }
    }
}

// ---- rebuild K or V of the staged page (lane = token r, channel group g)

__device__ inline void stage_bytes(const uint8_t* st, int sm_off, int code_off, int base_off, int r, int g,
                                   PageBytes& pb) {
    const uint8_t* smr = st + sm_off + r * 128;
    pb.sm_lo = ld16(smr + 16 * (g ^ (r & 7)));
    pb.sm_hi = ld16(smr + 16 * ((4 + g) ^ (r & 7)));
    pb.code = ld16(st + code_off + r * 64 + 16 * (g ^ ((r >> 1) & 3)));
    pb.b_lo = ld16(st + base_off + 16 * g);
    pb.b_hi = ld16(st + base_off + 64 + 16 * g);
}

__device__ inline void stage_bf16_k(const uint8_t* st, int r, int g, uint32_t out[16]) {
    const uint8_t* rp = st + BS_K + r * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = (j < 2 ? 2 * g : 8 + 2 * g) + (j & 1);
        const uint4 v = ld16(rp + 16 * (u ^ (r & 7)));
        out[4 * j] = v.x; out[4 * j + 1] = v.y; out[4 * j + 2] = v.z; out[4 * j + 3] = v.w;
    }
}

// V tile row r: logical 16-B unit u at physical unit u ^ ((r & 3) << 1)
__device__ inline void write_v_tile(uint8_t* tile, int r, int g, const uint32_t v[16]) {
    uint8_t* rp = tile + r * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = (j < 2 ? 2 * g : 8 + 2 * g) + (j & 1);
        *reinterpret_cast<u32x4*>(rp + 16 * (u ^ ((r & 3) << 1))) = u32x4{v[4 * j], v[4 * j + 1], v[4 * j + 2],
                                                                           v[4 * j + 3]};
    }
}

// After a workgroup has written its partials: count it in; the last workgroup of the unit
// (sequence b, head block hb, head group hg) merges all splits of its query heads.
__device__ inline void merge_tail(const AttnArgs& a, int b, int hb, int hg, int gh, int split) {
    if (a.counters == nullptr) return;
    __shared__ int s_last;
    __threadfence();                                   // release this workgroup's partials
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(&a.counters[blockIdx.y], 1) == a.nsplit - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();                                   // acquire the other workgroups' partials
    const int rows = a.HW * gh;
    for (int idx = threadIdx.x; idx < rows * (kD / 2); idx += kThreads) {
        const int dp = idx % (kD / 2);
        const int h = (idx / (kD / 2)) % gh, hs = (idx / (kD / 2)) / gh;
        const int64_t row = (int64_t)b * a.Hq + (int64_t)(hb * a.HW + hs) * a.G + hg * 16 + h;
        const float* m = a.part_m + row * a.nsplit;
        const float M = split_max(m, a.nsplit);
        reinterpret_cast<uint32_t*>(a.out + row * kD)[dp] =
            merge_pair(a.part_o + row * a.nsplit * kD, m, a.part_l + row * a.nsplit, a.nsplit, M, dp);
    }
    if (threadIdx.x == 0) a.counters[blockIdx.y] = 0;  // ready for the next call on this workspace
    (void)split;
}

template <bool COMP>
__global__ void __launch_bounds__(kThreads) attn_split_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[Ring<COMP>::bytes];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
    // workgroup: sequence b, token split, block of HW KV heads (all read the same tokens, so
    // the workgroup's loads cover whole token rows of the [B, T, H, D] arrays); wavefront:
    // head slot w % HW, page phase w / HW
    const int split = blockIdx.x;
    int y = blockIdx.y;
    const int hg = y % a.HG;
    y /= a.HG;
    const int nhb = a.Hkv / a.HW;
    const int hb = y % nhb;
    const int b = y / nhb;
    const int hk = hb * a.HW + wave % a.HW;
    const int phase = wave / a.HW, nphase = kWaves / a.HW;
    int len = a.lens ? a.lens[b * a.lens_stride] : a.T;
    len = min(max(len, 0), a.TS);
    const int start = split * a.split_len;
    const int end = min(start + a.split_len, len);
    const int NP = a.TS / kPage;

    // Q^T as the B operand: column = head hg*16 + r of this KV head's group, k-block kc
    // holds channels 16g + 8kc.. (kc < 2) or 64 + 16g + 8(kc-2).. (kc >= 2).
    const int hl = hg * 16 + r;
    uint32_t qw[16];
    {
        const uint16_t* qp = a.q + ((int64_t)b * a.Hq + (int64_t)hk * a.G + min(hl, a.G - 1)) * kD;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
            const int d0 = kc < 2 ? 16 * g + 8 * kc : 64 + 16 * g + 8 * (kc - 2);
            u32x4 v = {0u, 0u, 0u, 0u};
            if (hl < a.G) v = *reinterpret_cast<const u32x4*>(qp + d0);
            qw[4 * kc] = v.x; qw[4 * kc + 1] = v.y; qw[4 * kc + 2] = v.z; qw[4 * kc + 3] = v.w;
        }
    }

    float m_i = -INFINITY, l_i = 0.f;
    f32x4 acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // this wavefront's pages: p0 + phase + nphase * j, j < npw
    constexpr int NST = Ring<COMP>::nst;
    constexpr int STB = Ring<COMP>::stage;
    uint8_t* ring = lds + wave * NST * STB;
    const int p0 = start / kPage;
    const int pend = end > start ? (end + kPage - 1) / kPage : p0;
    const int npw = pend - p0 > phase ? (pend - p0 - phase + nphase - 1) / nphase : 0;
    const int64_t rs = a.Hkv;
    const DmaLane dl = dma_lane_offsets<COMP>(lane, rs);
    auto issue = [&](int j) {
        const int pg = p0 + phase + nphase * j;
        const int64_t row0 = ((int64_t)b * a.TS + (int64_t)pg * kPage) * rs + hk;
        const int64_t page = ((int64_t)b * NP + pg) * rs + hk;
        dma_page<COMP>(a, dl, row0, page, ring + (j % NST) * STB, lane);
    };
#pragma unroll
    for (int j = 0; j < NST - 1; ++j)
        if (j < npw) issue(j);
    settle(qw);                                        // q (and the first pages) arrive here
    bf16x8 qop[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) qop[kc] = as_bf16x8(qw[4 * kc], qw[4 * kc + 1], qw[4 * kc + 2], qw[4 * kc + 3]);

    for (int j = 0; j < npw; ++j) {
        // stage j is complete once only the younger pages' loads are in flight
        if (NST == 3 && j + 1 < npw)
            wait_vm<kDmaPerPage>();
        else
            wait_vm<0>();
        uint8_t* st = ring + (j % NST) * STB;
        const int pg = p0 + phase + nphase * j;
        const int t0 = pg * kPage;
        const bool row_valid = t0 + r < end;

        uint32_t kd[16], vd[16];
        uint32_t kraw[16], vraw[16];
        uint32_t rmk = 0, rmv = 0;
        if constexpr (COMP) {
            const u32x4 meta = *reinterpret_cast<const u32x4*>(st + CS_META);
            rmk = __builtin_amdgcn_readfirstlane(meta.x);
            const int rok = __builtin_amdgcn_readfirstlane(meta.y);
            rmv = __builtin_amdgcn_readfirstlane(meta.z);
            const int rov = __builtin_amdgcn_readfirstlane(meta.w);
            if ((rmk | rmv) != 0) {
                // raw rows (a few percent of pages): fetch them now and wait, before the
                // next page's loads go out, so the fixed wait counts stay exact
                if ((rmk >> r) & 1u) load_raw_values(a.k.raw, raw_slot(rmk, rok, r, a.k.raw_rows), g, kraw);
                if ((rmv >> r) & 1u) load_raw_values(a.v.raw, raw_slot(rmv, rov, r, a.v.raw_rows), g, vraw);
                wait_vm<0>();
                settle(kraw);
                settle(vraw);
            }
        }
        if (j + NST - 1 < npw) {
            // the recycled stage was last touched by this wavefront's LDS accesses of the
            // previous page: let them finish before the DMA can land there
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(j + NST - 1);
        }

        // ---- K: rebuild, scores
        if constexpr (COMP) {
            PageBytes pb;
            stage_bytes(st, CS_KSM, CS_KCODE, CS_BASE, r, g, pb);
            rebuild_values(pb, kd);
            if (rmk != 0 && ((rmk >> r) & 1u)) {       // page with raw rows (uniform test first)
#pragma unroll
                for (int i = 0; i < 16; ++i) kd[i] = kraw[i];
            }
        } else {
            stage_bf16_k(st, r, g, kd);
        }
        const bool ragged = t0 + kPage > end;          // uniform: only the last page of a split
        if (ragged && !row_valid) {
#pragma unroll
            for (int i = 0; i < 16; ++i) kd[i] = 0u;
        }
        f32x4 sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
            sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(kd[4 * kc], kd[4 * kc + 1], kd[4 * kc + 2], kd[4 * kc + 3]), qop[kc], sa, 0, 0, 0);

        // ---- online softmax: lane = head r, tokens t0 + 4g + i
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = sa[i] * a.qk_scale;
        if (ragged) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (t0 + 4 * g + i >= end) sc[i] = -INFINITY;
        }
        float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_i, mloc);
        const float alpha = fast_exp2(m_i - m_new);
        float psum = 0.f;
        bf16x4 pb4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(sc[i] - m_new);
            psum += p;
            pb4[i] = (__bf16)p;
        }
        l_i = l_i * alpha + psum;
        m_i = m_new;
        if (__ballot(alpha != 1.f) != 0) {             // rescale only when some head's max moved
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) acc[nb] *= alpha;
        }

        // ---- V: rebuild into the stage's bf16 tile (compressed) or use the staged rows
        uint8_t* tile = st + Ring<COMP>::vtile;
        if constexpr (COMP) {
            PageBytes pv;
            stage_bytes(st, CS_VSM, CS_VCODE, CS_BASE + 128, r, g, pv);
            rebuild_values(pv, vd);
            if (rmv != 0 && ((rmv >> r) & 1u)) {
#pragma unroll
                for (int i = 0; i < 16; ++i) vd[i] = vraw[i];
            }
            if (ragged && !row_valid) {
#pragma unroll
                for (int i = 0; i < 16; ++i) vd[i] = 0u;
            }
            write_v_tile(tile, r, g, vd);
        } else {
            if (ragged && !row_valid) {                // ragged last page: zero the rows past the end
#pragma unroll
                for (int i = 0; i < 16; ++i) vd[i] = 0u;
                write_v_tile(tile, r, g, vd);
            }
        }
        // ---- O^T += V^T P^T: V^T rows 4g..4g+3 of channel 16nb + r via the transpose read
        const s16x4 pop = __builtin_bit_cast(s16x4, pb4);
        const int trow = 4 * g + (r >> 2);
        const uint8_t* trp = tile + trow * 256 + 8 * (r & 1);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const int u = 2 * nb + ((r & 3) >> 1);
            const s16x4 av =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((EXKV_LDS s16x4*)(trp + 16 * (u ^ ((trow & 3) << 1))));
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, pop, acc[nb], 0, 0, 0);
        }
    }

    // ---- merge the page phases of each head (same algebra as the split merge)
    float l_t = l_i + __shfl_xor(l_i, 16);
    l_t = l_t + __shfl_xor(l_t, 32);
    const int gh = min(16, a.G - hg * 16);
    const int64_t hq0 = (int64_t)b * a.Hq + (int64_t)hk * a.G + hg * 16;     // first query head of this wave
    if (nphase == 1) {                                 // one wavefront per head: write its partial
        if (r < gh) {
            const int64_t prow = (hq0 + r) * a.nsplit + split;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb)
                *reinterpret_cast<f32x4*>(a.part_o + prow * kD + 16 * nb + 4 * g) = acc[nb];
            if (g == 0) {
                a.part_m[prow] = m_i;
                a.part_l[prow] = l_t;
            }
        }
        merge_tail(a, b, hb, hg, gh, split);
        return;
    }
    __syncthreads();
    float* mo = reinterpret_cast<float*>(lds);            // [wave][16 heads][128]
    float* mm = mo + kWaves * 16 * kD;                     // [wave][16]
    float* ml = mm + kWaves * 16;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
        *reinterpret_cast<f32x4*>(mo + (wave * 16 + r) * kD + 16 * nb + 4 * g) = acc[nb];
    if (g == 0) {
        mm[wave * 16 + r] = m_i;
        ml[wave * 16 + r] = l_t;
    }
    __syncthreads();
    // thread t merges (head slot, head, channel) items; waves of one head slot s are s, s + HW, ...
    for (int idx = threadIdx.x; idx < a.HW * gh * kD; idx += kThreads) {
        const int d = idx & (kD - 1);
        const int h = (idx >> 7) % gh;
        const int hs = (idx >> 7) / gh;
        float M = -INFINITY;
        for (int ph = 0; ph < nphase; ++ph) M = fmaxf(M, mm[(ph * a.HW + hs) * 16 + h]);
        float o = 0.f, l = 0.f;
        if (M != -INFINITY) {
            for (int ph = 0; ph < nphase; ++ph) {
                const int w = ph * a.HW + hs;
                const float wt = fast_exp2(mm[w * 16 + h] - M);
                o += wt * mo[(w * 16 + h) * kD + d];
                l += wt * ml[w * 16 + h];
            }
        }
        const int64_t prow = ((int64_t)b * a.Hq + (int64_t)(hb * a.HW + hs) * a.G + hg * 16 + h) * a.nsplit + split;
        a.part_o[prow * kD + d] = o;
        if (d == 0) {
            a.part_m[prow] = M;
            a.part_l[prow] = l;
        }
    }
    merge_tail(a, b, hb, hg, gh, split);
}

// Separate merge of the split partials, one wavefront per (sequence, query head) row.
__global__ void __launch_bounds__(64) attn_reduce_kernel(const float* po, const float* pm, const float* pl,
                                                         uint16_t* out, int ns) {
    const int64_t row = blockIdx.x;
    const float* m = pm + row * ns;
    const float M = split_max(m, ns);
    reinterpret_cast<uint32_t*>(out + row * kD)[threadIdx.x] =
        merge_pair(po + row * ns * kD, m, pl + row * ns, ns, M, threadIdx.x);
}

}  // namespace exkv

using namespace exkv;

// KV heads per workgroup: gcd(Hkv, 8) (8 wavefronts = head slots x page phases)
static int heads_per_block(int Hkv) {
    int a = Hkv, b = kWaves;
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

static int check_attn(int B, int Hq, int Hkv, int D, int T, int TS, const int32_t* lens, int nsplit,
                      int split_len) {
    EXKV_REQUIRE(D == kD, "attention: head dim must be 128 (got %d)", D);
    EXKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "attention: bad heads Hq=%d Hkv=%d (B=%d)", Hq,
                 Hkv, B);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0, "attention: TS=%d must be a positive multiple of 16", TS);
    EXKV_REQUIRE(nsplit > 0 && split_len > 0 && split_len % kPage == 0,
                 "attention: split_len=%d must be a positive multiple of 16 (nsplit=%d)", split_len, nsplit);
    if (lens == nullptr) {
        EXKV_REQUIRE(T >= 1 && T <= TS, "attention: T=%d outside [1, TS=%d]", T, TS);
        EXKV_REQUIRE((int64_t)nsplit * split_len >= T, "attention: %d splits of %d do not cover T=%d", nsplit,
                     split_len, T);
    } else {
        EXKV_REQUIRE((int64_t)nsplit * split_len >= TS,
                     "attention: with per-sequence lengths the splits must cover TS=%d", TS);
    }
    EXKV_REQUIRE((int64_t)B * (Hkv / heads_per_block(Hkv)) * ((Hq / Hkv + 15) / 16) < 65536,
                 "attention: too many (sequence, head block) units");
    return EXKV_OK;
}

static int launch_split(bool comp, const AttnArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)a.nsplit, (unsigned)(a.B * (a.Hkv / a.HW) * a.HG));
    if (comp)
        hipLaunchKernelGGL(attn_split_kernel<true>, grid, dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(attn_split_kernel<false>, grid, dim3(kThreads), 0, stream, a);
    return hip_status(hipGetLastError(), comp ? "attn_split_compressed" : "attn_split_bf16");
}

static int launch_reduce(const float* o, const float* m, const float* l, void* out, int64_t rows, int ns,
                         hipStream_t stream) {
    hipLaunchKernelGGL(attn_reduce_kernel, dim3((unsigned)rows), dim3(64), 0, stream, o, m, l, (uint16_t*)out, ns);
    return hip_status(hipGetLastError(), "attn_reduce");
}

static int fill_compressed(AttnArgs& a, const void* q, const void* k_sm, const void* k_code, const void* k_base,
                           const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw, int64_t k_raw_rows,
                           const void* v_sm, const void* v_code, const void* v_base, const int32_t* v_rowmask,
                           const int32_t* v_rowoff, const void* v_raw, int64_t v_raw_rows, float* ws_o,
                           float* ws_m, float* ws_l, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T,
                           int32_t TS, const int32_t* lens, int64_t lens_stride, int32_t nsplit,
                           int32_t split_len, float qk_scale) {
    const int rc = check_attn(B, Hq, Hkv, D, T, TS, lens, nsplit, split_len);
    if (rc) return rc;
    EXKV_REQUIRE(k_raw_rows > 0 && v_raw_rows > 0, "attn_compressed: empty raw pool");
    EXKV_REQUIRE(q && k_sm && k_code && k_base && k_rowmask && k_rowoff && k_raw && v_sm && v_code && v_base &&
                     v_rowmask && v_rowoff && v_raw && ws_o && ws_m && ws_l,
                 "attn_compressed: null pointer");
    a = AttnArgs{};
    a.q = (const uint16_t*)q;
    a.k = CSrc{(const uint8_t*)k_sm, (const uint8_t*)k_code, (const uint8_t*)k_base, k_rowmask, k_rowoff,
               (const uint16_t*)k_raw, k_raw_rows};
    a.v = CSrc{(const uint8_t*)v_sm, (const uint8_t*)v_code, (const uint8_t*)v_base, v_rowmask, v_rowoff,
               (const uint16_t*)v_raw, v_raw_rows};
    a.part_o = ws_o; a.part_m = ws_m; a.part_l = ws_l;
    a.lens = lens; a.lens_stride = lens_stride;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.HG = (a.G + 15) / 16; a.TS = TS; a.T = T;
    a.nsplit = nsplit; a.split_len = split_len; a.qk_scale = qk_scale; a.HW = heads_per_block(Hkv);
    return EXKV_OK;
}

static int fill_bf16(AttnArgs& a, const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                     float* ws_l, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                     const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len, float qk_scale) {
    const int rc = check_attn(B, Hq, Hkv, D, T, TS, lens, nsplit, split_len);
    if (rc) return rc;
    EXKV_REQUIRE(q && k && v && ws_o && ws_m && ws_l, "attn_bf16: null pointer");
    a = AttnArgs{};
    a.q = (const uint16_t*)q;
    a.kb = (const uint16_t*)k; a.vb = (const uint16_t*)v;
    a.part_o = ws_o; a.part_m = ws_m; a.part_l = ws_l;
    a.lens = lens; a.lens_stride = lens_stride;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.HG = (a.G + 15) / 16; a.TS = TS; a.T = T;
    a.nsplit = nsplit; a.split_len = split_len; a.qk_scale = qk_scale; a.HW = heads_per_block(Hkv);
    return EXKV_OK;
}

#define EXKV_C_PARAMS                                                                                    \
    const void *q, const void *k_sm, const void *k_code, const void *k_base, const int32_t *k_rowmask,         \
        const int32_t *k_rowoff, const void *k_raw, int64_t k_raw_rows, const void *v_sm, const void *v_code, \
        const void *v_base, const int32_t *v_rowmask, const int32_t *v_rowoff, const void *v_raw,            \
        int64_t v_raw_rows, float *ws_o, float *ws_m, float *ws_l
#define EXKV_C_ARGS                                                                                       \
    q, k_sm, k_code, k_base, k_rowmask, k_rowoff, k_raw, k_raw_rows, v_sm, v_code, v_base, v_rowmask, v_rowoff, \
        v_raw, v_raw_rows, ws_o, ws_m, ws_l
#define EXKV_SHAPE_PARAMS                                                                                  \
    int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS, const int32_t *lens, int64_t lens_stride, \
        int32_t nsplit, int32_t split_len, float qk_scale
#define EXKV_SHAPE_ARGS B, Hq, Hkv, D, T, TS, lens, lens_stride, nsplit, split_len, qk_scale

extern "C" int exkv_attn_compressed(EXKV_C_PARAMS, int32_t* ws_cnt, void* out, EXKV_SHAPE_PARAMS,
                                    hipStream_t stream) {
    AttnArgs a;
    int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_compressed: null output");
    if (ws_cnt) {                                      // merge fused into the split kernel
        a.out = (uint16_t*)out;
        a.counters = ws_cnt;
        return launch_split(true, a, stream);
    }
    rc = launch_split(true, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, stream);
}

extern "C" int exkv_attn_split_compressed(EXKV_C_PARAMS, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    const int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    return rc ? rc : launch_split(true, a, stream);
}

extern "C" int exkv_attn_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m, float* ws_l,
                              int32_t* ws_cnt, void* out, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    int rc = fill_bf16(a, q, k, v, ws_o, ws_m, ws_l, EXKV_SHAPE_ARGS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_bf16: null output");
    if (ws_cnt) {
        a.out = (uint16_t*)out;
        a.counters = ws_cnt;
        return launch_split(false, a, stream);
    }
    rc = launch_split(false, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, stream);
}

extern "C" int exkv_attn_split_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                                    float* ws_l, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    const int rc = fill_bf16(a, q, k, v, ws_o, ws_m, ws_l, EXKV_SHAPE_ARGS);
    return rc ? rc : launch_split(false, a, stream);
}

extern "C" int exkv_attn_reduce(const float* ws_o, const float* ws_m, const float* ws_l, void* out, int64_t rows,
                                int32_t nsplit, int32_t D, hipStream_t stream) {
    EXKV_REQUIRE(D == kD, "attn_reduce: head dim must be 128 (got %d)", D);
    EXKV_REQUIRE(rows > 0 && nsplit > 0, "attn_reduce: bad rows=%lld nsplit=%d", (long long)rows, nsplit);
    EXKV_REQUIRE(ws_o && ws_m && ws_l && out, "attn_reduce: null pointer");
    return launch_reduce(ws_o, ws_m, ws_l, out, rows, nsplit, stream);
}
