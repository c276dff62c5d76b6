// Split-K GQA decode attention for gfx950, over the compressed cache or over plain bf16.
//
// Reference: exactkv/kernels.py _split_c_kernel :142-165, _split_ref_kernel :168-194,
// _attn_block :46-59, _reduce_kernel :33-43.
//
// Grid: x = token split, y = (sequence, block of HW = min(gcd(Hkv, 8), 4) KV heads, group of
// 16 query heads); one workgroup per CU (its LDS ring, ~158 KB). A workgroup has 8 compute
// wavefronts: each KV head of the block gets 8 / HW of them ("page phases"),
// which take the split's 16-token pages round robin, each with its own online-softmax
// state, and are merged through LDS at the end (one partial per split and query head).
//
// Memory pipeline: every page is brought into its wavefront's private LDS ring by a fixed
// number of direct-to-LDS loads (global_load_lds_dwordx4 with the nontemporal hint: the
// bytes are read once per call), rows placed with XOR swizzles chosen so that the later LDS
// reads are conflict-free. The compiler does not order LDS
// reads after these loads, so a stage is read only after an explicit s_waitcnt vmcnt(N)
// of the wavefront that issued them.
//   * Compressed cache: two more wavefronts per workgroup (loaders) issue every page's 7
//     byte loads into the compute wavefronts' 3-stage rings and publish each landed page
//     through an LDS flag; a compute wavefront waits for that flag and hands the stage
//     back through another as soon as its last read of it has returned (see the kernel).
//     Compute wavefronts never stall on a full memory pipeline; the loaders do.
//   * bf16 twin: each wavefront issues its own pages' 8 loads, one page ahead (2 stages).
//
// Per page:
//   * K is rebuilt bit-exactly in VGPRs from the staged bytes (lane = token; the page's base
//     bytes reach the 16 lanes of a row through a DPP row broadcast), V straight into the
//     P.V operand layout (V^T) from transposing byte reads (ds_read_b64_tr_b8); raw rows are
//     spliced in from the wavefront's raw-row slots, which one more direct-to-LDS load per
//     page with raw rows fills (issued by the compute wavefront, which knows the page's
//     metadata).
//   * S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (tokens = rows, the G query heads of the
//     KV head = columns, padded to 16); online softmax in base 2, scores scaled by
//     D^-1/2 log2(e), p rounded to bf16 for P.V, l summed from fp32 p.
//   * V^T is the A operand of v_mfma_f32_16x16x16_bf16: the compressed kernel rebuilds it in
//     that layout (pages with raw V rows go through a bf16 row tile over the stage's K
//     bytes, already in registers), the bf16 twin reads it from its stage's V rows with
//     ds_read_b64_tr_b16; the C layout of S^T is exactly the P^T operand layout, and O^T
//     accumulates with lane = head, so the softmax rescale needs no cross-lane traffic.
// Everything after the K/V rebuild is shared by the two kernels, so the compressed and
// uncompressed results are identical bit for bit.
//
// Other head dims: 64 with an even number of KV heads runs the same structure over pairs
// of heads (attn_pair_kernel: a pair has one head-dim-128 head's bytes per token row);
// 256, and 64 with an odd count, run attn_dgen_kernel (one KV head per workgroup, each
// wavefront loading its own pages).
#include <hip/hip_ext.h>

#include "tile.hpp"
#include "stage.hpp"
#include "../../include/exactkv.h"

#define EXKV_LDS __attribute__((address_space(3)))

namespace exkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kFusedMaxSplits = 1024;   // up to this many splits the split kernel can merge in its tail
constexpr int kDmaPerPage[2] = {8, 8}; // direct-to-LDS loads per page: bf16; compressed 7 + a raw-row load (pages with raw rows)


// Raw rows travel with their page through the DMA ring when a page (K and V together)
// has at most kRawRing of them: one more load per page into the wave's raw slot of the
// page's parity. Pages with more fall back to direct loads.
constexpr int kRawRing = 2;
constexpr int kRawSlot = kRawRing * 256;

// Per wavefront: nst page stages, then (compressed) two raw slots.
template <bool COMP>
struct Ring {
    static constexpr int stage = COMP ? CS_BYTES : BS_BYTES;
    static constexpr int nst = COMP ? 3 : 2;
    static constexpr int vtile = COMP ? 0 : BS_V;    // offset of the bf16 V tile in a stage
    static constexpr int raw = COMP ? 2 * kRawSlot : 0;
    static constexpr int per_wave = nst * stage + raw;
    static constexpr int bytes = kWaves * per_wave;
};

// A wave-uniform 64-bit value the compiler cannot trace back to the kernel arguments: a
// per-lane select between two such values stays a v_cndmask instead of becoming a
// per-lane load of the chosen pointer from the argument block (and its wait for all loads).
__device__ inline uint64_t opaque_u64(uint64_t x) {
    asm("" : "+s"(x));
    return x;
}
struct PairSrc {              // K address of one array and V minus K: per-lane selects add
    uint64_t k, d;            // (cond ? d : 0), which cannot become a load of either pointer
    __device__ uint64_t pick(bool v) const { return k + (v ? d : 0ull); }
};
__device__ inline PairSrc pair_src(uint64_t k, uint64_t v) {
    const uint64_t ko = opaque_u64(k);
    return PairSrc{ko, opaque_u64(v) - ko};
}

// rowmask / rowoff of one page of the K and V caches (wave-uniform)
struct PageMeta {
    uint32_t mk, mv;
    int32_t ok, ov;
};
__device__ inline int raw_rows_of(const PageMeta& m) { return __builtin_popcount(m.mk) + __builtin_popcount(m.mv); }
__device__ inline bool raw_in_ring(const PageMeta& m) {
    const int n = raw_rows_of(m);
    return n > 0 && n <= kRawRing;
}
// Loads a compressed page takes: its 7 byte loads, plus one raw-row load when its raw rows
// travel through the ring
__device__ inline int raw_loads(const PageMeta& m) { return raw_in_ring(m) ? 1 : 0; }

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
    int window;               // > 0: attend to the last `window` tokens of each sequence only
    int HW;                   // KV heads per workgroup (min(gcd(Hkv, 8), 4)); 8 / HW page phases per head
    float qk_scale;
    uint16_t* out;            // [B, Hq, 128] bf16, written by the last workgroup of each unit
    int32_t* counters;        // [gridDim.y] arrival counters (zero between calls); nullptr: no merge
    // Paged caches: the arrays hold a pool of pool_pages pages (one sequence of
    // 16 * pool_pages tokens) and page p of sequence b is pool page block_table[b * bt_stride
    // + p]. nullptr: page p of sequence b is page b * TS / 16 + p of [B, TS, ...] arrays.
    const int32_t* block_table;
    int64_t bt_stride;
    int pool_pages;
    int D;                    // head dim: 128 (the tuned kernels), 64 or 256 (attn_dgen_kernel)
    int spin;                 // bound of every wait on another wavefront's LDS flag (polls, >= 1)
};

// ---- split merge (kernels.py:33-43): M = max_s m_s, w_s = 2^(m_s - M),
// out = sum_s o_s w_s / sum_s l_s w_s. Up to 32 splits: one wavefront per (sequence, query
// head) row with lane = channel pair, the sums over s in order with explicit fmas -- the
// order of the fused merge's one-level case, so both produce the same bits.
__device__ inline float fast_exp2(float x);
__device__ inline float wave_max(float x) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) x = fmaxf(x, __shfl_xor(x, d));
    return x;
}
__device__ inline uint32_t pack_bf16x2(float a, float b) {
    const __bf16 r0 = (__bf16)a, r1 = (__bf16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, r0) | ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
}
// ns <= N splits in one round trip: m, l and o loads issued together.
template <int N>
__device__ __attribute__((always_inline)) inline uint32_t merge_direct(const float* po, const float* m,
                                                                        const float* l, int ns, int lane) {
    const float2* po2 = reinterpret_cast<const float2*>(po);
    const float mv = lane < ns ? m[lane] : -INFINITY;
    const float lv = lane < ns ? l[lane] : 0.f;
    float2 o[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (i < ns) o[i] = po2[(int64_t)i * (kD / 2) + lane];
    const float M = wave_max(mv);
    const float ws = fast_exp2(mv - M);
    float n0 = 0.f, n1 = 0.f, den = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (i < ns) {
            const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ws), i));
            const float li = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), i));
            n0 = __builtin_fmaf(o[i].x, w, n0);
            n1 = __builtin_fmaf(o[i].y, w, n1);
            den = __builtin_fmaf(li, w, den);
        }
    return pack_bf16x2(n0 / den, n1 / den);
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
__device__ inline void dma16(const void* g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// Cache pages and raw rows: read once per call, so they stream with the nontemporal hint
// (nt: no retention in the L2 and the Infinity Cache). Measured at c2a: compressed split
// kernel 41.2 -> 37.0 us, bf16 twin 45.8 -> 42.1 us; q keeps the default policy (every
// split of a unit reads it).
__device__ inline void dma16_stream(const void* g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds) : "memory");
}
// 4-byte variant: lane L's dword lands at M0 + 4L.
__device__ inline void dma4(const void* g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

// Mark registers as defined here (an empty asm that reads and writes them): the compiler
// then waits for their loads at this point, once, instead of at every later use inside
// the page loop, where its vmcnt(0) would also wait for the ring's loads in flight.
template <int N>
__device__ inline void settle(uint32_t (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}

// Load of a wave-uniform int32 through the constant address space (an s_load_dword).
__device__ inline int32_t const_ld(const int32_t* p) {
    return *(const __attribute__((address_space(4))) int32_t*)p;
}

// Reductions over the 4 lane groups holding one head (lanes l, l^16, l^32, l^48) with the
// gfx950 row-swap permutes: with both operands = x, v_permlane16_swap returns x's even and
// odd 16-lane rows side by side (likewise v_permlane32_swap for the two halves).
__device__ inline float group_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ inline float group_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

// Wait until at most n vector-memory loads of this wavefront are in flight, and keep the
// compiler from moving memory accesses across the wait.
template <int N>
__device__ inline void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}


// wait_vm with a wave-uniform count of 0, 1, 7 or 8 loads
__device__ inline void wait_vm_n(int n) {
    if (n >= 8)
        wait_vm<8>();
    else if (n == 7)
        wait_vm<7>();
    else if (n == 1)
        wait_vm<1>();
    else
        wait_vm<0>();
}


// Issue the byte loads of one page into stage st (7 for the compressed cache, 8 for bf16).
// row0: row index of the page's token 0 ((b*TS + 16*pg)*Hkv + hk); page: its page index.
// They need no page metadata, so the first pages' loads can leave before the page table.
template <bool COMP>
__device__ inline void dma_page_bytes(const AttnArgs& a, const DmaLane& o, int64_t row0, int64_t page, uint32_t st,
                                      int lane, const PairSrc& basep) {
    if constexpr (COMP) {
        const uint8_t* ksm = a.k.sm + row0 * 128;
        const uint8_t* vsm = a.v.sm + row0 * 128;
        dma16_stream(ksm + o.sm0, st + CS_KSM);
        dma16_stream(vsm + o.sm0, st + CS_VSM);
        dma16_stream(ksm + o.sm1, st + CS_KSM + 1024);
        dma16_stream(vsm + o.sm1, st + CS_VSM + 1024);
        dma16_stream(a.k.code + row0 * 64 + o.code, st + CS_KCODE);
        dma16_stream(a.v.code + row0 * 64 + o.code, st + CS_VCODE);
        // base rows: lanes 0-7 K, 8-15 V
        const uint64_t bsrc = basep.pick((lane & 8) != 0) + (uint64_t)page * 128 + o.base;
        if (lane < 16) dma16_stream((const void*)(uintptr_t)bsrc, st + CS_BASE);
    } else {
        const uint8_t* kp = reinterpret_cast<const uint8_t*>(a.kb) + row0 * 256;
        const uint8_t* vp = reinterpret_cast<const uint8_t*>(a.vb) + row0 * 256;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dma16_stream(kp + o.bf_k[j], st + BS_K + j * 1024);
            dma16_stream(vp + o.bf_v[j], st + BS_V + j * 1024);
        }
    }
}

// The compressed page's raw-row load, issued only for a page whose raw rows travel through
// the ring (raw_loads: the waits count it); the only load that needs the page's metadata.
__device__ inline void dma_page_raw(int lane, const PageMeta& m, uint32_t raw_st, const PairSrc& rawp,
                                    const PairSrc& rawn) {
    if (!raw_in_ring(m)) return;                       // uniform
    // the slot was last read by this wavefront's splice of two pages back: those LDS reads
    // finish before the DMA can land there
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    {
        // raw rows of the page (K rows in token order, then V rows): entry e = lane / 16 of
        // at most kRawRing, 16 bytes per lane; pool index = rowoff + rank of the row
        const int nk = __builtin_popcount(m.mk);
        const int n = nk + __builtin_popcount(m.mv), e = lane >> 4;
        const bool isv = e >= nk;
        int64_t idx = isv ? (int64_t)m.ov + (e - nk) : (int64_t)m.ok + e;
        const int64_t rows = (int64_t)rawn.pick(isv);
        bool bad;
        idx = clamp_slot(idx, rows, bad);
        const uint64_t rb = rawp.pick(isv);
        if (lane < 16 * n) {
            if (bad) report_error(kErrRawSlot);
            dma16_stream((const void*)(uintptr_t)(rb + (uint64_t)idx * 256 + (uint64_t)(lane & 15) * 16), raw_st);
        }
    }
}

// q through LDS: the wavefront's query heads hg*16 .. hg*16 + gh - 1 of KV head hk, head h
// at qst + 256 h, by direct-to-LDS loads (load d: heads 4d .. 4d + 3) that are waited for
// like the page loads, so that waiting for q does not also wait for the first pages.
__device__ inline void q_dma(const AttnArgs& a, int b, int hk, int hg, int gh, int lane, uint32_t qst) {
    const int nq = (gh + 3) >> 2;
    for (int d = 0; d < nq; ++d) {
        const int h = min(4 * d + (lane >> 4), gh - 1);
        dma16(a.q + ((int64_t)b * a.Hq + (int64_t)hk * a.G + hg * 16 + h) * kD + 8 * (lane & 15),
              qst + (uint32_t)(1024 * d));
    }
}

typedef EXKV_LDS uint8_t lds_u8;
__device__ inline lds_u8* lds_ptr(uint32_t a) { return (lds_u8*)(uintptr_t)a; }
__device__ inline uint4 lds16(const lds_u8* p) {
    const u32x4 v = *reinterpret_cast<const EXKV_LDS u32x4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline void lds_st16(lds_u8* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *reinterpret_cast<EXKV_LDS u32x4*>(p) = u32x4{a, b, c, d};
}

// Keep a rarely taken, wave-uniform branch as a branch: the compiler cannot move an
// opaque volatile statement out of it, so it does not turn the block into selects that
// would run on every page.
__device__ inline void keep_branch() { asm volatile(""); }

// ---- rebuild K or V of the staged page (lane = token r, channel group g)

// ---- base bytes through a row broadcast (the head-dim-128 compressed split kernel)
//
// The 16 lanes of row g (lanes 16g .. 16g + 15, channel group g) need the same 32 base bytes
// of K and of V. Instead of every lane reading them (four 16-byte LDS reads of a page, most
// of the page's LDS read traffic), lane r of the row reads one dword (LdsLane::bw) -- r =
// 0-3 and 4-7: dwords 0-3 of its group's low and high K runs, 8-11 and 12-15: the same of V
// -- and the rebuild takes dword i of a run from lane i of its own row with a DPP row
// broadcast (row_newbcast), which the compiler folds into the exponent add.
__device__ inline void stage_sm_code(uint32_t sb, const LdsLane& o, int sm_off, int code_off, StageSC& sc) {
    sc.sm_lo = lds16(lds_ptr(sb + o.sml) + sm_off);
    sc.sm_hi = lds16(lds_ptr(sb + o.smh) + sm_off);
    sc.code = lds16(lds_ptr(sb + o.code) + code_off);
}
__device__ inline uint32_t stage_base_word(uint32_t sb, uint32_t off) {
    return *reinterpret_cast<const EXKV_LDS uint32_t*>(lds_ptr(sb + off));
}
__device__ inline uint32_t stage_base_word(uint32_t sb, const LdsLane& o) { return stage_base_word(sb, o.bw); }

template <int L>                       // lane L of the row, to every lane of the row
__device__ __forceinline__ uint32_t row_bcast(uint32_t x) {
    return __builtin_amdgcn_update_dpp(0u, x, 0x150 + L, 0xf, 0xf, false);
}
template <bool Z, int L>
__device__ __forceinline__ void rebuild4_bc(uint32_t s, uint32_t cn, uint32_t bw, uint32_t& o01, uint32_t& o23) {
    bf16_pairs(s, Z ? exponents(cn, row_bcast<L>(bw)) : cn + row_bcast<L>(bw), o01, o23);
}
// The DPP row broadcast as the base-dword source of the stage's rebuild (stage.hpp)
struct RowBcast {
    uint32_t bw;
    template <int L>
    __device__ __forceinline__ uint32_t get() const { return row_bcast<L>(bw); }
};
// K (V = false) or V values of the lane from its staged bytes (stage.hpp rebuild_values_from)
template <bool V>
__device__ __forceinline__ void rebuild_values_bc(const StageSC& sc, uint32_t bw, uint64_t zf, uint32_t out[16]) {
    rebuild_values_from<V>(sc, RowBcast{bw}, zf, out);
}

// The same for runs of W dwords (head dim 256: W = 8, lanes L .. L + 7 of the row holding
// the run's base dwords).
template <bool Z, bool HIGH, int L, int I, int W>
__device__ __forceinline__ void rebuild_run_bcw(const uint32_t* sm, const uint32_t* code, uint32_t bw, uint32_t* out) {
    if constexpr (I < W) {
        rebuild4_bc<Z, L + I>(sm[I], (HIGH ? code[I] >> 4 : code[I]) & 0x0F0F0F0Fu, bw, out[2 * I], out[2 * I + 1]);
        rebuild_run_bcw<Z, HIGH, L, I + 1, W>(sm, code, bw, out);
    }
}

// ---- V^T straight from the staged bytes (the head-dim-128 compressed split kernel; the
// lane offsets, the read's layout and the rebuild arithmetic are in stage.hpp)
__device__ inline uint2 lds_tr8(uint32_t a) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((EXKV_LDS v2i*)lds_ptr(a));
    return make_uint2((uint32_t)v.x, (uint32_t)v.y);
}
__device__ inline void stage_vt_bytes(uint32_t sb, const VtLane& o, VtBytes& vb) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        const uint2 s = lds_tr8(sb + o.sm[nb]);
        vb.sm[nb] = s.x;
        vb.sm[nb + 4] = s.y;
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint2 s = lds_tr8(sb + o.code[c]);
        vb.code[2 * c] = s.x;
        vb.code[2 * c + 1] = s.y;
    }
    const uint2 b = lds_tr8(sb + o.base);
    vb.base[0] = b.x;
    vb.base[1] = b.y;
}
// The zero-group fix-up per run of blocks (0-3, 4-7; their base bytes are base[0], base[1]),
// decided for the wavefront.
template <bool PAIR = false>
__device__ __forceinline__ void rebuild_vt(const VtBytes& vb, s16x4 (&vt)[8]) {
    if (__ballot((vb.base[0] & 0x80808080u) != 0u) != 0)
        rebuild_vt_run<true, 0, PAIR>(vb, vt);
    else
        rebuild_vt_run<false, 0, PAIR>(vb, vt);
    if (__ballot((vb.base[1] & 0x80808080u) != 0u) != 0)
        rebuild_vt_run<true, 4, PAIR>(vb, vt);
    else
        rebuild_vt_run<false, 4, PAIR>(vb, vt);
}
// Tokens of a ragged page past the split's end or before the window read as zero.
template <int NB>
__device__ __forceinline__ void vt_zero_invalid(s16x4 (&vt)[NB], int tok0, int end, int wlo) {
    uint32_t m[2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const int t = tok0 + 2 * d;
        m[d] = (t < end && t >= wlo ? 0x0000FFFFu : 0u) | (t + 1 < end && t + 1 >= wlo ? 0xFFFF0000u : 0u);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const uint2 d = __builtin_bit_cast(uint2, vt[nb]);
        vt[nb] = __builtin_bit_cast(s16x4, make_uint2(d.x & m[0], d.y & m[1]));
    }
}

__device__ inline void stage_bf16_k(uint32_t sb, const LdsLane& o, uint32_t out[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 v = lds16(lds_ptr(sb + o.bk[j]) + BS_K);
        out[4 * j] = v.x; out[4 * j + 1] = v.y; out[4 * j + 2] = v.z; out[4 * j + 3] = v.w;
    }
}

// The lane's 32 values of raw row q of a ring slot (channels 16g.. and 64+16g..)
__device__ inline void lds_raw_values(uint32_t slot, int q, int g, uint32_t out[16]) {
    const lds_u8* p = lds_ptr(slot + (uint32_t)(q * 256 + 32 * g));
    const uint4 a0 = lds16(p), a1 = lds16(p + 16), h0 = lds16(p + 128), h1 = lds16(p + 144);
    out[0] = a0.x; out[1] = a0.y; out[2] = a0.z; out[3] = a0.w;
    out[4] = a1.x; out[5] = a1.y; out[6] = a1.z; out[7] = a1.w;
    out[8] = h0.x; out[9] = h0.y; out[10] = h0.z; out[11] = h0.w;
    out[12] = h1.x; out[13] = h1.y; out[14] = h1.z; out[15] = h1.w;
}

// Splice the page's raw K (V = false) or V rows into the lane's rebuilt row (lane = token
// r): from the page's raw slot when they came through the ring (entry = rank of the row,
// K rows first), else straight from the pool (rare; this waits for every load in flight).
template <bool V>
__device__ inline void splice_raw(const AttnArgs& a, const PageMeta& m, uint32_t slot, int r, int g,
                                  uint32_t d[16]) {
    const uint32_t mask = V ? m.mv : m.mk;
    const uint32_t below = (1u << r) - 1u;
    uint32_t x[16];
    if (raw_in_ring(m)) {
        const int e = (V ? __builtin_popcount(m.mk) : 0) + __builtin_popcount(mask & below);
        lds_raw_values(slot, min(e, kRawRing - 1), g, x);
    } else {
        const CSrc& c = V ? a.v : a.k;
        load_raw_values(c.raw, raw_slot(mask, V ? m.ov : m.ok, r, c.raw_rows), g, x);
        wait_vm<0>();
        settle(x);
    }
    const bool take = ((mask >> r) & 1u) != 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = take ? x[i] : d[i];
}

// V tile row r (32 values of the lane) at the tile offset toff of the stage
__device__ inline void write_v_tile(uint32_t sb, const LdsLane& o, int toff, const uint32_t v[16]) {
    lds_u8* p = lds_ptr(sb + o.tw) + toff;
    lds_st16(p, v[0], v[1], v[2], v[3]);
    lds_st16(p + 16, v[4], v[5], v[6], v[7]);
    lds_st16(p + 128, v[8], v[9], v[10], v[11]);
    lds_st16(p + 144, v[12], v[13], v[14], v[15]);
}

// ---- the merge in the split kernel's tail (counters != nullptr)
//
// Partials are written with device-scope stores, which go through the L2 of the writer's
// XCD to memory, and read with device-scope loads; a workgroup counts itself in only once
// its own stores are complete (s_waitcnt vmcnt(0) before the counter's atomic add). So the
// last workgroup of a group sees every partial of the group without an L2 write-back or
// invalidate (a device-scope release / acquire, which on a multi-XCD part writes back the
// XCD's whole L2: measured slower than a second kernel at every grid size).
//
// Up to 32 splits the last workgroup of a unit merges them all (one level: the separate
// merge's arithmetic, so its bits). More splits take two levels, each short: the splits of
// a unit form groups of merge_group(ns) consecutive splits; the last workgroup to finish a
// group merges it into the group's first split slot (un-normalised o, max m, sum l), and
// the last group merger of the unit merges the groups into the output. Counters:
// [unit][group] then [unit][ngroups] for the second level, all zero between calls (each
// merger resets the one it consumed). Partial values move as 8-byte device-scope
// atomics (a channel pair per access).
__device__ inline void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float ld_dev(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void st_dev2(float* p, float x, float y) {       // p 8-byte aligned
    const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float2 ld_dev2(const float* p) {
    const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
// 16 bytes with the device-scope stores' cache policy (sc1: through the writer's L2 to
// memory), in one access: HIP has no 16-byte atomic store, and two 8-byte ones from lanes
// holding every other channel pair would each fill only half of every 64-byte sector.
// Completion is waited for with the other stores (arrive_last's s_waitcnt vmcnt(0)).
__device__ inline void st_dev4(float* p, const f32x4& v) {    // p 16-byte aligned
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}

__host__ __device__ inline int merge_group(int ns) {
    if (ns <= 32) return ns;                           // one level (the separate merge's bits)
    int g = 1;
    while (g * g < ns) ++g;                            // ceil(sqrt(ns)): both levels about as long
    return g;
}
__host__ __device__ inline int merge_groups(int ns) { return (ns + merge_group(ns) - 1) / merge_group(ns); }

// One row (sequence, query head): merge splits s0, s0 + step, ... (n <= 32 of them, all
// loads in flight together), lane = channel pair. Returns the un-normalised sums and the
// common maximum; a row whose splits are all empty gives m = -inf, l = 0, o = 0.
struct RowMerge {
    float n0, n1, den, M;
};
__device__ inline RowMerge merge_row_dev(const AttnArgs& a, int64_t row, int s0, int step, int n, int lane) {
    const float* po = a.part_o + row * a.nsplit * kD;
    const float* pm = a.part_m + row * a.nsplit;
    const float* pl = a.part_l + row * a.nsplit;
    const float mv = lane < n ? ld_dev(pm + s0 + lane * step) : -INFINITY;
    const float lv = lane < n ? ld_dev(pl + s0 + lane * step) : 0.f;
    float ox[32], oy[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
        if (i < n) {
            const float2 v = ld_dev2(po + (int64_t)(s0 + i * step) * kD + 2 * lane);
            ox[i] = v.x;
            oy[i] = v.y;
        }
    const float M = wave_max(mv);
    const float ws = M == -INFINITY ? 0.f : fast_exp2(mv - M);
    RowMerge r{0.f, 0.f, 0.f, M};
#pragma unroll
    for (int i = 0; i < 32; ++i)
        if (i < n) {
            const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ws), i));
            const float li = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), i));
            r.n0 = __builtin_fmaf(ox[i], w, r.n0);
            r.n1 = __builtin_fmaf(oy[i], w, r.n1);
            r.den = __builtin_fmaf(li, w, r.den);
        }
    return r;
}

// Count this workgroup in at counter c (after every wave's stores are complete); true for
// the workgroup that completes a count of n, which also resets the counter.
__device__ inline bool arrive_last(int32_t* c, int n) {
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's partial stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == n - 1;
        if (old == n - 1) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return s_last != 0;
}

// After a workgroup has written its partials (rows of heads hb*HW .. of sequence b, query
// group hg, split `split`): the two-level merge above.
__device__ inline void merge_tail(const AttnArgs& a, int b, int hb, int hg, int gh, int split) {
    if (a.counters == nullptr) return;
    const int G1 = merge_group(a.nsplit), ng = merge_groups(a.nsplit);
    const int grp = split / G1, g0 = grp * G1, gn = min(G1, a.nsplit - g0);
    int32_t* cnt = a.counters + (int64_t)blockIdx.y * (ng + 1);
    if (!arrive_last(cnt + grp, gn)) return;
    const int rows = a.HW * gh, lane = threadIdx.x & 63;
    auto row_of = [&](int i) {
        return (int64_t)b * a.Hq + (int64_t)(hb * a.HW + i / gh) * a.G + hg * 16 + i % gh;
    };
    if (ng > 1) {                                      // level 1: the group into its first split slot
        for (int i = threadIdx.x >> 6; i < rows; i += blockDim.x >> 6) {
            const int64_t row = row_of(i);
            const RowMerge r = merge_row_dev(a, row, g0, 1, gn, lane);
            st_dev2(a.part_o + (row * a.nsplit + g0) * kD + 2 * lane, r.n0, r.n1);
            if (lane == 0) {
                st_dev(a.part_m + row * a.nsplit + g0, r.M);
                st_dev(a.part_l + row * a.nsplit + g0, r.den);
            }
        }
        if (!arrive_last(cnt + ng, ng)) return;
    }
    const int step = ng > 1 ? G1 : 1, n2 = ng > 1 ? ng : a.nsplit;
    for (int i = threadIdx.x >> 6; i < rows; i += blockDim.x >> 6) {   // level 2: the groups (or splits) into the output
        const int64_t row = row_of(i);
        const RowMerge r = merge_row_dev(a, row, 0, step, n2, lane);
        reinterpret_cast<uint32_t*>(a.out + row * kD)[lane] = pack_bf16x2(r.n0 / r.den, r.n1 / r.den);
    }
}

// ---- pieces shared by the two split kernels

// Page-phase partials through LDS (split_epilogue): rows of 128 channels padded to kMoRow
// floats, so that the 16 heads of one write land in different banks (a 512-byte row
// stride put them all in the same ones).
constexpr int kMoRow = kD + 4;
constexpr int kMoBytes = (16 * kMoRow + 2 * 16) * 4;    // one wavefront's partial
static_assert(Ring<true>::per_wave >= kMoBytes && Ring<false>::per_wave >= kMoBytes,
              "a page phase's partial must fit its wavefront's ring");

// Workgroup coordinates of a split-kernel launch: sequence b, token split, block hb of HW
// KV heads, group hg of 16 query heads (gh of them real); the split's tokens [start, end)
// (pages p0 .. pend - 1) and the window's first token wlo. Page phase ph (wavefronts ph*HW
// .. ph*HW + HW - 1) takes pages p0 + ph + nphase * j, j < npw(ph).
struct SplitCoords {
    int split, hg, hb, b, hw_sh, nphase, wlo, start, end, NP, p0, pend, gh;
    __device__ int npw(int ph) const { return pend - p0 > ph ? (pend - p0 - ph + nphase - 1) / nphase : 0; }
};
__device__ inline SplitCoords split_coords(const AttnArgs& a) {
    SplitCoords c;
    c.split = blockIdx.x;
    int y = blockIdx.y;
    c.hg = y % a.HG;
    y /= a.HG;
    const int nhb = a.Hkv / a.HW;
    c.hb = y % nhb;
    c.b = y / nhb;
    c.hw_sh = __builtin_ctz(a.HW);                    // HW: a power of two
    c.nphase = kWaves >> c.hw_sh;
    int len = a.lens ? a.lens[c.b * a.lens_stride] : a.T;
    len = min(max(len, 0), a.TS);
    // sliding window: tokens [wlo, len) only; the splits start at wlo's page
    c.wlo = a.window > 0 ? max(len - a.window, 0) : 0;
    c.start = (c.wlo & ~(kPage - 1)) + c.split * a.split_len;
    c.end = min(c.start + a.split_len, len);
    c.NP = a.TS / kPage;
    c.p0 = c.start / kPage;
    c.pend = c.end > c.start ? (c.end + kPage - 1) / kPage : c.p0;
    c.gh = min(16, a.G - c.hg * 16);
    return c;
}

// Array page of page lp of sequence b: contiguous, or pool page block_table[b * bt_stride +
// lp] clamped to the pool (a bad entry cannot read out of bounds). e: that table entry.
__device__ inline int64_t array_page(const AttnArgs& a, const SplitCoords& c, int lp, int32_t e) {
    if (a.block_table == nullptr) return (int64_t)c.b * c.NP + lp;
    return (int64_t)min((uint32_t)e, (uint32_t)(a.pool_pages - 1));
}

// Q^T as the B operand of the score MFMAs, from q staged at qst (head h at qst + 256 h):
// column = head hg*16 + r of this KV head's group, k-block kc holds channels 16g + 8kc..
// (kc < 2) or 64 + 16g + 8(kc-2).. (kc >= 2); heads past the group are zero.
__device__ inline void load_qop(uint32_t qst, int r, int g, int gh, bf16x8 (&qop)[4]) {
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        const int d0 = kc < 2 ? 16 * g + 8 * kc : 64 + 16 * g + 8 * (kc - 2);
        uint4 v = lds16(lds_ptr(qst + (uint32_t)(r * 256 + 2 * d0)));
        if (r >= gh) v = make_uint4(0u, 0u, 0u, 0u);
        qop[kc] = as_bf16x8(v.x, v.y, v.z, v.w);
        // pin the masked operand: left alone, the compiler re-applies the mask (16 selects)
        // before every page's score MFMAs instead of keeping the result
        asm volatile("" : "+v"(qop[kc]));
    }
}

// Score MFMAs of one page: S^T = K Q^T (tokens = rows, the group's query heads = columns)
__device__ inline f32x4 page_scores(const uint32_t (&kd)[16], const bf16x8 (&qop)[4]) {
    f32x4 sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
        sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kd[4 * kc], kd[4 * kc + 1], kd[4 * kc + 2], kd[4 * kc + 3]),
                                                     qop[kc], sa, 0, 0, 0);
    return sa;
}

// V^T operands of the P.V MFMAs out of the page's bf16 V tile (at sb + toff)
__device__ inline void read_vt(uint32_t sb, const LdsLane& lo, int toff, s16x4 (&vt)[8]) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        const lds_u8* tp = lds_ptr(sb + lo.tr[nb & 3]) + toff + (nb >= 4 ? 128 : 0);
        vt[nb] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EXKV_LDS s16x4*)tp);
    }
}

// Rows of a ragged page (past the split's end or before the window) read as zero
__device__ inline void zero_invalid_rows(bool valid, uint32_t (&d)[16]) {
    if (!valid) {
#pragma unroll
        for (int i = 0; i < 16; ++i) d[i] = 0u;
    }
}

// One page's online softmax and P.V, the same code in both kernels (so that their results
// agree bit for bit). Lane = head r, tokens t0 + 4g + i; m_i in scaled (log2) units.
// max(s) * scale == max(s * scale) (rounding is monotone), and the scale goes into the
// exponent's fma: p = 2^(s * scale - m). Tokens outside the split or the window score
// -inf; only a ragged page has any. p is rounded to bf16 for P.V, l sums the fp32 p.
template <int NB>
__device__ __forceinline__ void page_softmax_pv(f32x4 sa, const s16x4 (&vt)[NB], bool ragged, int t0, int end, int wlo,
                                                int g, float qk_scale, float& m_i, float& l_i, f32x4 (&acc)[NB]) {
    // The score MFMAs' result is read below after branches whose opaque asm the compiler's
    // hazard tracking has counted as wait states (reads then saw stale accumulators). Pass
    // it through 16 explicit wait states instead: the asm defines sa, so every later read
    // follows it.
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(sa));
    float sc[4] = {sa[0], sa[1], sa[2], sa[3]};
    if (ragged) {
        keep_branch();
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (t0 + 4 * g + i >= end || t0 + 4 * g + i < wlo) sc[i] = -INFINITY;
    }
    float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mloc = group_max(mloc) * qk_scale;
    const float m_new = fmaxf(m_i, mloc);
    const float alpha = fast_exp2(m_i - m_new);
    float psum = 0.f;
    bf16x4 pb4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(__builtin_fmaf(sc[i], qk_scale, -m_new));
        psum += p;
        pb4[i] = (__bf16)p;
    }
    l_i = l_i * alpha + psum;
    m_i = m_new;
    if (__ballot(alpha != 1.f) != 0) {                 // rescale only when some head's max moved
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb] *= alpha;
    }
    // O^T += V^T P^T: V^T rows 4g..4g+3 of channel 16nb + r; the C layout of S^T is exactly
    // the P^T operand layout, and O^T accumulates with lane = head
    const s16x4 pop = __builtin_bit_cast(s16x4, pb4);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt[nb], pop, acc[nb], 0, 0, 0);
}

// Wavefronts w and w ^ 4 share a SIMD, whose issue arbiter favours the older one: left
// alone it runs ahead and its partner finishes last. The one that is behind takes the
// higher priority (the partner's page count is an unsynchronised hint: either value is
// fine).
__device__ inline void balance_priority(int j, int other) {
    if (j > 0) {
        if (j < other)
            __builtin_amdgcn_s_setprio(2);
        else
            __builtin_amdgcn_s_setprio(0);
    }
}

// Flags between the wavefronts of a workgroup: LDS words, read and written as relaxed
// atomics (the waits order the data accesses around them); every wait on one is bounded
// (AttnArgs::spin polls; a correct run never reaches the bound) and a wait that reaches its
// bound is reported (kErrWait) before the kernel goes on with whatever the LDS holds.
constexpr int kSpinMax = 1 << 22;                  // the default bound
__device__ inline int lds_flag_ld(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ inline void lds_flag_st(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }

// Store one partial row (m, l, o) of a (split, query head): lane (head r, channel group g)
// holds o for channels 16 nb + 4 g .. + 3; plain stores, or device-scope ones when the
// split kernel merges in its tail.
__device__ inline void store_partial(const AttnArgs& a, int64_t prow, int g, const f32x4 (&o)[8], float m, float l) {
    if (a.counters == nullptr) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) *reinterpret_cast<f32x4*>(a.part_o + prow * kD + 16 * nb + 4 * g) = o[nb];
        if (g == 0) {
            a.part_m[prow] = m;
            a.part_l[prow] = l;
        }
    } else {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) st_dev4(a.part_o + prow * kD + 16 * nb + 4 * g, o[nb]);
        if (g == 0) {
            st_dev(a.part_m + prow, m);
            st_dev(a.part_l + prow, l);
        }
    }
}

// One split per row: the output itself, with the merge's arithmetic for a single term
// (w = 2^(m - m), n = fma(o, w, 0), d = fma(l, w, 0), out = n / d; merge_direct at ns = 1),
// so the bits are those of the separate merge and no second launch is needed.
__device__ inline void store_direct(const AttnArgs& a, int64_t orow, int g, const f32x4 (&o)[8], float m, float l) {
    const float w = fast_exp2(m - m);
    const float den = __builtin_fmaf(l, w, 0.f);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        float n[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) n[k] = __builtin_fmaf(o[nb][k], w, 0.f);
        *reinterpret_cast<uint2*>(a.out + orow * kD + 16 * nb + 4 * g) =
            make_uint2(pack_bf16x2(n[0] / den, n[1] / den), pack_bf16x2(n[2] / den, n[3] / den));
    }
}

// After the page loop: one partial per (split, query head). With page phases (fewer than 8
// KV heads per workgroup), the wavefront of phase p > 0 leaves its (o, m, l) in its own
// ring -- free once its pages are consumed: o as [16 heads][kMoRow] floats (rows padded so
// that the 16 heads of one write fall in different banks), then m[16], l[16] -- and raises
// done[wave]; the phase-0 wavefront of the head slot waits for its partners (bounded),
// merges in phase order with the split merge's algebra (M = max m, o = sum o 2^(m - M),
// l likewise) and writes the partial. Then the fused merge when asked for: every
// wavefront of the workgroup calls this (merge_tail's barriers count them all); active ==
// false (loader wavefronts) contributes nothing. ring0: the workgroup's first ring (LDS
// address), ring_stride: bytes from one wavefront's ring to the next.
__device__ __forceinline__ void split_epilogue(const AttnArgs& a, const SplitCoords& c, uint32_t ring0,
                                               uint32_t ring_stride, int* done, int wave, int lane, bool active,
                                               int hk, const f32x4 (&acc)[8], float m_i, float l_i) {
    const int r = lane & 15, g = lane >> 4;
    // the accumulators were last written by MFMAs, possibly across inline assembly that the
    // hazard tracking may count as wait states: pad explicitly before the first reads
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    const float l_t = group_sum(l_i);
    const int phase = wave >> c.hw_sh;
    auto mo = [&](int w) { return ring0 + (uint32_t)w * ring_stride; };   // wavefront w's partial
    auto ld_ml = [&](int w, int k) {                                     // k = 0: m, 1: l of head r
        return *reinterpret_cast<const EXKV_LDS float*>(lds_ptr(mo(w) + 4u * (16 * kMoRow + 16 * k + r)));
    };
    if (active && phase > 0) {                         // hand the partial to the phase-0 wavefront
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
            *reinterpret_cast<EXKV_LDS f32x4*>(lds_ptr(mo(wave) + 4u * (r * kMoRow + 16 * nb + 4 * g))) = acc[nb];
        if (g == 0) {
            *reinterpret_cast<EXKV_LDS float*>(lds_ptr(mo(wave) + 4u * (16 * kMoRow + r))) = m_i;
            *reinterpret_cast<EXKV_LDS float*>(lds_ptr(mo(wave) + 4u * (16 * kMoRow + 16 + r))) = l_t;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_flag_st(&done[wave], 1);
    } else if (active && r < c.gh) {
        const int64_t orow = (int64_t)c.b * a.Hq + (int64_t)hk * a.G + c.hg * 16 + r;
        const int64_t prow = orow * a.nsplit + c.split;
        {
            float M = fmaxf(-INFINITY, m_i);
            for (int ph = 1; ph < c.nphase; ++ph) {
                const int w = ph * a.HW + wave;
                int s = 0;
                for (; s < a.spin && lds_flag_ld(&done[w]) == 0; ++s) __builtin_amdgcn_s_sleep(1);
                if (s == a.spin) report_error(kErrWait);
                asm volatile("" ::: "memory");
                M = fmaxf(M, ld_ml(w, 0));
            }
            f32x4 o[8];
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            float l = 0.f;
            if (M != -INFINITY) {
                const float wt = fast_exp2(m_i - M);
#pragma unroll
                for (int nb = 0; nb < 8; ++nb)
#pragma unroll
                    for (int k = 0; k < 4; ++k) o[nb][k] += wt * acc[nb][k];
                l += wt * l_t;
                for (int ph = 1; ph < c.nphase; ++ph) {
                    const int w = ph * a.HW + wave;
                    const float wp = fast_exp2(ld_ml(w, 0) - M);
#pragma unroll
                    for (int nb = 0; nb < 8; ++nb) {
                        const f32x4 v = *reinterpret_cast<const EXKV_LDS f32x4*>(
                            lds_ptr(mo(w) + 4u * (r * kMoRow + 16 * nb + 4 * g)));
#pragma unroll
                        for (int k = 0; k < 4; ++k) o[nb][k] += wp * v[k];
                    }
                    l += wp * ld_ml(w, 1);
                }
            }
            if (a.nsplit == 1 && a.out != nullptr)
                store_direct(a, orow, g, o, M, l);
            else
                store_partial(a, prow, g, o, M, l);
        }
    }
    if (a.nsplit > 1) merge_tail(a, c.b, c.hb, c.hg, c.gh, c.split);
}

template <bool COMP>
__global__ void attn_split_kernel(AttnArgs a);

// ---- compressed split kernel: 8 compute wavefronts (head slots x page phases) and
// kLoaders loader wavefronts.
//
// Loader l issues every byte load of the pages of compute wavefronts kWpl*l .. kWpl*l +
// kWpl - 1 into their rings, in rounds (page j of each of them, in order), keeps kLoadAhead
// + 1 pages in flight, and publishes a page (ready[w] = pages of w landed) once its loads
// are complete (its own s_waitcnt vmcnt: loads complete in order). It issues page j of w
// only once avail[w] > j, i.e. once w has handed back the stage that page j reuses. A
// compute wavefront waits for ready[w] > j, reads the page, and hands the stage back as
// soon as its last LDS read of it has returned. So the compute wavefronts never stall on a
// full memory pipeline (the loaders do), and the CU's loads stay in flight while they
// compute. The flags live in LDS; every wait on them is bounded (AttnArgs::spin).
constexpr int kLoaders = 2;
constexpr int kWpl = kWaves / kLoaders;          // compute wavefronts per loader
constexpr int kCompThreads = 64 * (kWaves + kLoaders);
constexpr int kLoadAhead = 3;                    // pages a loader keeps in flight besides the newest
constexpr int kBytesLoads = kDmaPerPage[1] - 1;  // byte loads per compressed page
static_assert((kLoadAhead + 1) * kBytesLoads <= 63, "a loader's loads in flight must fit vmcnt");
static_assert(kLoadAhead == 3, "loader_wait_pages covers 0 to kLoadAhead newer pages");

// Wait until a loader's oldest page in flight has landed, k pages (each kBytesLoads loads)
// being newer than it: the loads of one wavefront land in order.
__device__ inline void loader_wait_pages(int k) {
    if (k >= 3)
        wait_vm<3 * kBytesLoads>();
    else if (k == 2)
        wait_vm<2 * kBytesLoads>();
    else if (k == 1)
        wait_vm<kBytesLoads>();
    else
        wait_vm<0>();
}


// Loader wavefront l (see above)
__device__ __forceinline__ void comp_loader(const AttnArgs& a, const SplitCoords& c, uint32_t lds0, int* ready,
                                            const int* avail, int l, int lane) {
    constexpr int NST = Ring<true>::nst, STB = Ring<true>::stage;
    __builtin_amdgcn_s_setprio(3);                     // issue as soon as the memory pipeline takes it
    const int64_t rs = a.Hkv;
    const DmaLane dl = dma_lane_offsets<true>(lane, rs);
    const PairSrc basep = pair_src((uint64_t)(uintptr_t)a.k.base, (uint64_t)(uintptr_t)a.v.base);
    const int w0 = kWpl * l;
    auto lpage = [&](int i, int j) { return c.p0 + ((w0 + i) >> c.hw_sh) + c.nphase * j; };
    const int jmax = c.npw(w0 >> c.hw_sh);             // wavefront w0 has the lowest phase: the most pages
    // paged: the block-table entries of pages p0 .. p0 + 63 (lane k: page p0 + k), read once
    int32_t vbt = 0;
    if (a.block_table != nullptr) {
        vbt = a.block_table[c.b * a.bt_stride + min(c.p0 + lane, c.NP - 1)];
        asm volatile("" : "+v"(vbt));                  // waited for here, once, before any page load
    }
    int inflight = 0, pi = 0, pj = 0;                  // the oldest page in flight: wavefront w0 + pi, page pj
    auto publish = [&]() {
        lds_flag_st(&ready[w0 + pi], pj + 1);
        do {
            if (++pi == kWpl) {
                pi = 0;
                ++pj;
            }
        } while (pj < jmax && lpage(pi, pj) >= c.pend);
        --inflight;
    };
    for (int j = 0; j < jmax; ++j) {
        for (int i = 0; i < kWpl; ++i) {
            const int lp = lpage(i, j);
            if (lp >= c.pend) continue;
            const int w = w0 + i;
            if (lds_flag_ld(&avail[w]) <= j) {         // its stage is still in use: publish all, then wait
                while (inflight > 0) {                 // each page as soon as its own loads have landed
                    loader_wait_pages(inflight - 1);
                    publish();
                }
                int s = 0;
                for (; s < a.spin && lds_flag_ld(&avail[w]) <= j; ++s) __builtin_amdgcn_s_sleep(1);
                if (s == a.spin) report_error(kErrWait);
            }
            int32_t e = 0;
            if (a.block_table != nullptr)
                e = lp - c.p0 < 64 ? __builtin_amdgcn_readlane(vbt, lp - c.p0)
                                   : const_ld(a.block_table + c.b * a.bt_stride + lp);
            const int64_t gp = array_page(a, c, lp, e);
            const int hk = c.hb * a.HW + (w & (a.HW - 1));
            const uint32_t sb = lds0 + (uint32_t)(w * Ring<true>::per_wave + (j % NST) * STB);
            dma_page_bytes<true>(a, dl, gp * kPage * rs + hk, gp * rs + hk, sb, lane, basep);
            if (++inflight > kLoadAhead) {
                wait_vm<kLoadAhead * kBytesLoads>();
                publish();
            }
        }
    }
    while (inflight > 0) {                             // the last pages, each as soon as it has landed
        loader_wait_pages(inflight - 1);
        publish();
    }
}

template <>
__global__ void __launch_bounds__(kCompThreads) attn_split_kernel<true>(AttnArgs a) {
    constexpr int NST = Ring<true>::nst, STB = Ring<true>::stage;
    __shared__ __attribute__((aligned(16))) uint8_t lds[Ring<true>::bytes];
    __shared__ int progress[kWaves];                   // pages done per compute wavefront (priority hint)
    __shared__ int ready[kWaves];                      // pages of wavefront w in its ring (loader -> w)
    __shared__ int avail[kWaves];                      // pages of w its loader may issue (w -> loader)
    __shared__ int done[kWaves];                       // page phase p > 0: partial left in the ring
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);    // uniform: scalar addressing
    const SplitCoords c = split_coords(a);
    const int hk = c.hb * a.HW + (wave & (a.HW - 1));
    if (threadIdx.x < kWaves) {
        ready[threadIdx.x] = 0;
        avail[threadIdx.x] = NST - 1;                  // the last stage holds q and the page table at first
        done[threadIdx.x] = 0;
    }
    __syncthreads();

    float m_i = -INFINITY, l_i = 0.f;
    f32x4 acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (wave >= kWaves) {
        comp_loader(a, c, lds_addr(lds), ready, avail, wave - kWaves, lane);
    } else {
        const int phase = wave >> c.hw_sh;
        const int npw = c.npw(phase);
        const int64_t rs = a.Hkv;
        const uint32_t ring = lds_addr(lds) + (uint32_t)(wave * Ring<true>::per_wave);   // this wave's (uniform)
        const uint32_t raw_ring = ring + (uint32_t)(NST * STB);
        const LdsLane lo = lds_lane_offsets(r, g);
        const VtLane vto = vt_lane_offsets(lane);
        const PairSrc rawp = pair_src((uint64_t)(uintptr_t)a.k.raw, (uint64_t)(uintptr_t)a.v.raw);
        const PairSrc rawn = pair_src((uint64_t)a.k.raw_rows, (uint64_t)a.v.raw_rows);

        // rowmask / rowoff of the wavefront's pages. Lane i holds page i's (i < 64): loaded
        // once, with q, by direct-to-LDS loads, then read into VGPRs, so that a page's values
        // are v_readlane of its index (scalar loads for pages past 64). The same for the
        // block-table entries of the wavefront's pages (paged caches).
        int32_t vbt = 0;
        auto gpage = [&](int j) -> int64_t {
            const int lp = c.p0 + phase + c.nphase * j;
            int32_t e = 0;
            if (a.block_table != nullptr)
                e = j < 64 ? __builtin_amdgcn_readlane(vbt, j) : const_ld(a.block_table + c.b * a.bt_stride + lp);
            return array_page(a, c, lp, e);
        };
        auto meta_s = [&](int j) {
            const int64_t page = gpage(j) * rs + hk;
            return PageMeta{(uint32_t)const_ld(a.k.rowmask + page), (uint32_t)const_ld(a.v.rowmask + page),
                            const_ld(a.k.rowoff + page), const_ld(a.v.rowoff + page)};
        };
        uint32_t vmk = 0u, vmv = 0u;
        int32_t vok = 0, vov = 0;
        auto meta = [&](int j) {
            if (j >= 64) return meta_s(j);
            return PageMeta{(uint32_t)__builtin_amdgcn_readlane((int)vmk, j),
                            (uint32_t)__builtin_amdgcn_readlane((int)vmv, j), __builtin_amdgcn_readlane(vok, j),
                            __builtin_amdgcn_readlane(vov, j)};
        };
        auto issue_raw = [&](int j, const PageMeta& m) {
            dma_page_raw(lane, m, raw_ring + (uint32_t)((j & 1) * kRawSlot), rawp, rawn);
        };
        // q and the page table through the last stage, which no page uses before the
        // wavefront hands it over (avail = NST below)
        const uint32_t qst = ring + (uint32_t)((NST - 1) * STB);
        const uint32_t mst = qst + 4096u;              // rowmask K | rowoff K | rowmask V | rowoff V
        const int i_pg = min(lane, max(npw - 1, 0));   // per lane: the wavefront's page i
        if (a.block_table != nullptr) {                // the block-table entries first: every address needs them
            const uint32_t bst = mst + 1024u;
            dma4(a.block_table + c.b * a.bt_stride + min(c.p0 + phase + c.nphase * i_pg, c.NP - 1), bst);
            wait_vm<0>();
            vbt = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(bst + 4u * lane));
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        q_dma(a, c.b, hk, c.hg, c.gh, lane, qst);
        {
            const int64_t gp = a.block_table == nullptr ? (int64_t)c.b * c.NP + min(c.p0 + phase + c.nphase * i_pg, c.NP - 1)
                                                        : array_page(a, c, 0, vbt);
            const int64_t page = gp * rs + hk;
            dma4(a.k.rowmask + page, mst);
            dma4(a.k.rowoff + page, mst + 256u);
            dma4(a.v.rowmask + page, mst + 512u);
            dma4(a.v.rowoff + page, mst + 768u);
        }
        wait_vm<0>();
        bf16x8 qop[4];
        load_qop(qst, r, g, c.gh, qop);
        vmk = *reinterpret_cast<const EXKV_LDS uint32_t*>(lds_ptr(mst + 4u * lane));
        vok = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(mst + 256u + 4u * lane));
        vmv = *reinterpret_cast<const EXKV_LDS uint32_t*>(lds_ptr(mst + 512u + 4u * lane));
        vov = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(mst + 768u + 4u * lane));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // q and the page table are in registers
        lds_flag_st(&avail[wave], NST);
        // raw rows of a page travel through the wavefront's two raw slots (page parity),
        // issued two pages ahead by the wavefront itself
        if (npw > 0) issue_raw(0, meta(0));
        if (npw > 1) issue_raw(1, meta(1));

        lds_flag_st(&progress[wave], 0);
        int stg = 0;                                   // stage of page j (j % NST)
        for (int j = 0; j < npw; ++j) {
            // page j's raw rows have landed once only page j + 1's are in flight
            if (j + 1 < npw)
                wait_vm_n(raw_loads(meta(j + 1)));
            else
                wait_vm<0>();
            if (lds_flag_ld(&ready[wave]) <= j) {      // page j's bytes: published by the loader
                int s = 0;
                for (; s < a.spin && lds_flag_ld(&ready[wave]) <= j; ++s) __builtin_amdgcn_s_sleep(0);
                if (s == a.spin) report_error(kErrWait);
            }
            asm volatile("" ::: "memory");
            const uint32_t sb = ring + (uint32_t)(stg * STB);
            stg = stg == NST - 1 ? 0 : stg + 1;
            const int t0 = (c.p0 + phase + c.nphase * j) * kPage;
            const bool ragged = t0 + kPage > c.end || t0 < c.wlo;   // uniform: a split's last page, or the window's first
            const bool valid = t0 + r < c.end && t0 + r >= c.wlo;
            const PageMeta mc = meta(j);
            const PageMeta mn = j + NST - 1 < npw ? meta(j + NST - 1) : PageMeta{0u, 0u, 0, 0};
            const int other = lds_flag_ld(&progress[wave ^ 4]);   // the partner's count: a hint, read unsynchronised
            lds_flag_st(&progress[wave], j);

            // every read of the stage up front: V^T by transposing byte reads, K by rows; the
            // stage goes back to the loader once they have returned (after the score MFMAs)
            VtBytes vb;
            stage_vt_bytes(sb, vto, vb);
            StageSC pk;
            stage_sm_code(sb, lo, CS_KSM, CS_KCODE, pk);
            const uint32_t bw = stage_base_word(sb, lo);
            balance_priority(j, other);
            const uint32_t slot = raw_ring + (uint32_t)((j & 1) * kRawSlot);
            s16x4 vt[8];
            const uint64_t zf = __ballot((bw & 0x80808080u) != 0u);
            if (mc.mv == 0) {
                rebuild_vt(vb, vt);
                if (ragged) {
                    keep_branch();
                    vt_zero_invalid(vt, t0 + 4 * g, c.end, c.wlo);
                }
            } else {                                   // a page with raw V rows (rare): V by token
                keep_branch();                         // rows, its raw rows spliced in, transposed
                StageSC pv;                            // through a bf16 tile over the K bytes
                stage_sm_code(sb, lo, CS_VSM, CS_VCODE, pv);   // (already in registers)
                uint32_t vd[16];
                rebuild_values_bc<true>(pv, bw, zf, vd);
                splice_raw<true>(a, mc, slot, r, g, vd);
                if (ragged) {
                    keep_branch();
                    zero_invalid_rows(valid, vd);
                }
                write_v_tile(sb, lo, Ring<true>::vtile, vd);
                read_vt(sb, lo, Ring<true>::vtile, vt);
            }
            uint32_t kd[16];
            rebuild_values_bc<false>(pk, bw, zf, kd);
            if (mc.mk != 0) {
                keep_branch();
                splice_raw<false>(a, mc, slot, r, g, kd);
            }
            if (ragged) {
                keep_branch();
                zero_invalid_rows(valid, kd);
            }
            const f32x4 sa = page_scores(kd, qop);
            // this page's raw rows are out of their slot: page j + 2's go there
            if (j + NST - 1 < npw) issue_raw(j + NST - 1, mn);
            // every LDS read of the stage (bytes, V^T operands) has returned: hand it back
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            lds_flag_st(&avail[wave], j + NST + 1);
            page_softmax_pv(sa, vt, ragged, t0, c.end, c.wlo, g, a.qk_scale, m_i, l_i, acc);
        }
    }
    split_epilogue(a, c, lds_addr(lds), Ring<true>::per_wave, done, wave, lane, wave < kWaves, hk, acc, m_i, l_i);
}

// ---- bf16 twin: 8 wavefronts, each issuing its own pages' loads into a 2-stage ring (one
// page ahead); the same softmax / P.V code and epilogue as the compressed kernel.
template <>
__global__ void __launch_bounds__(kThreads) attn_split_kernel<false>(AttnArgs a) {
    constexpr int NST = Ring<false>::nst, STB = Ring<false>::stage;
    __shared__ __attribute__((aligned(16))) uint8_t lds[Ring<false>::bytes];
    __shared__ int progress[kWaves];
    __shared__ int done[kWaves];                       // page phase p > 0: partial left in the ring
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const SplitCoords c = split_coords(a);
    if (threadIdx.x < kWaves) done[threadIdx.x] = 0;
    __syncthreads();
    const int hk = c.hb * a.HW + (wave & (a.HW - 1));
    const int phase = wave >> c.hw_sh;
    const int npw = c.npw(phase);
    const int64_t rs = a.Hkv;
    float m_i = -INFINITY, l_i = 0.f;
    f32x4 acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t ring = lds_addr(lds) + (uint32_t)(wave * Ring<false>::per_wave);
    const LdsLane lo = lds_lane_offsets(r, g);
    const DmaLane dl = dma_lane_offsets<false>(lane, rs);
    const PairSrc nobase{0ull, 0ull};
    int32_t vbt = 0;
    auto gpage = [&](int j) -> int64_t {
        const int lp = c.p0 + phase + c.nphase * j;
        int32_t e = 0;
        if (a.block_table != nullptr)
            e = j < 64 ? __builtin_amdgcn_readlane(vbt, j) : const_ld(a.block_table + c.b * a.bt_stride + lp);
        return array_page(a, c, lp, e);
    };
    auto issue = [&](int j, uint32_t sb) {
        const int64_t gp = gpage(j);
        dma_page_bytes<false>(a, dl, gp * kPage * rs + hk, gp * rs + hk, sb, lane, nobase);
    };
    // q through the last stage, which no page uses before page NST - 1 is issued
    const uint32_t qst = ring + (uint32_t)((NST - 1) * STB);
    if (a.block_table != nullptr) {
        const uint32_t bst = qst + 5120u;
        const int i_pg = min(lane, max(npw - 1, 0));
        dma4(a.block_table + c.b * a.bt_stride + min(c.p0 + phase + c.nphase * i_pg, c.NP - 1), bst);
        wait_vm<0>();
        vbt = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(bst + 4u * lane));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    q_dma(a, c.b, hk, c.hg, c.gh, lane, qst);
    if (npw > 0) {
        issue(0, ring);
        wait_vm<kDmaPerPage[0]>();                     // q has landed once only page 0's loads are in flight
    } else {
        wait_vm<0>();
    }
    bf16x8 qop[4];
    load_qop(qst, r, g, c.gh, qop);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // q is in registers before its stage is reused

    lds_flag_st(&progress[wave], 0);
    int stg = 0;
    for (int j = 0; j < npw; ++j) {
        wait_vm<0>();                                  // page j has landed (the only page in flight)
        const uint32_t sb = ring + (uint32_t)(stg * STB);
        const int stn = stg == 0 ? NST - 1 : stg - 1;  // stage of page j + 1
        stg = stg == NST - 1 ? 0 : stg + 1;
        const int t0 = (c.p0 + phase + c.nphase * j) * kPage;
        const bool ragged = t0 + kPage > c.end || t0 < c.wlo;
        const bool valid = t0 + r < c.end && t0 + r >= c.wlo;
        // the next page's loads go out at once, into the stage the previous page used (its
        // last LDS reads are waited for first)
        if (j + NST - 1 < npw) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(j + NST - 1, ring + (uint32_t)(stn * STB));
        }
        const int other = lds_flag_ld(&progress[wave ^ 4]);   // the partner's count: a hint, read unsynchronised
        lds_flag_st(&progress[wave], j);
        uint32_t kd[16];
        stage_bf16_k(sb, lo, kd);
        balance_priority(j, other);
        if (ragged) {
            keep_branch();
            zero_invalid_rows(valid, kd);
        }
        const f32x4 sa = page_scores(kd, qop);
        if (ragged) {                                  // ragged page: zero the staged V rows past the end
            keep_branch();
            if (!valid) {
                uint32_t vd[16];
                zero_invalid_rows(false, vd);
                write_v_tile(sb, lo, Ring<false>::vtile, vd);
            }
        }
        s16x4 vt[8];
        read_vt(sb, lo, Ring<false>::vtile, vt);
        page_softmax_pv(sa, vt, ragged, t0, c.end, c.wlo, g, a.qk_scale, m_i, l_i, acc);
    }
    split_epilogue(a, c, lds_addr(lds), Ring<false>::per_wave, done, wave, lane, true, hk, acc, m_i, l_i);
}

// Separate merge of up to 32 splits: one wavefront per (sequence, query head) row, every
// load of the row in flight at once (the fused merge's code, so both give the same bits).
__global__ void __launch_bounds__(64) attn_reduce_kernel(const float* po, const float* pm, const float* pl,
                                                         uint16_t* out, int ns) {
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x & 63;
    reinterpret_cast<uint32_t*>(out + row * kD)[lane] =
        merge_direct<32>(po + row * ns * kD, pm + row * ns, pl + row * ns, ns, lane);
}

// Separate merge of more than 32 splits: workgroup (row, 16-channel chunk) of four
// wavefronts, so that a row's loads spread over eight workgroups (rows x 8 of them fill
// the chip where rows alone would use a few CUs). Lane (split group sg = lane / 8, channel
// pair cp = lane % 8); wavefront w takes a contiguous quarter of the splits, 64 at a time
// with every load of a batch (o, m and l) in flight together, in one pass: its sums are
// kept relative to the largest m it has seen, rescaled when a batch raises it, so no load
// waits for a first pass over m. Empty splits (m = -inf) weigh 0, and a wavefront whose
// splits are all empty adds 0. The sums combine over sg by shuffles, then over the
// wavefronts in order through LDS, each rescaled to the row's largest m. Deterministic,
// so the compressed call and its twin still agree bit for bit.
constexpr int kWideWaves = 4, kWideChunk = 16;
__global__ void __launch_bounds__(64 * kWideWaves) attn_reduce_wide_kernel(const float* po, const float* pm,
                                                                            const float* pl, uint16_t* out, int ns) {
    const int64_t row = blockIdx.x;
    const int c0 = kWideChunk * (int)blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sg = lane >> 3, cp = lane & 7;
    const float* o = po + row * ns * kD + c0 + 2 * cp;
    const float* m = pm + row * ns;
    const float* l = pl + row * ns;
    __shared__ float part[kWideWaves][4][8];
    const int per = (ns + kWideWaves - 1) / kWideWaves;
    const int s0 = min(ns, wave * per), s1 = min(ns, s0 + per);
    float n0 = 0.f, n1 = 0.f, den = 0.f, mw = -INFINITY;
    for (int b0 = s0; b0 < s1; b0 += 64) {
        float2 v[8];
        float mv[8], lv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int s = min(b0 + 8 * i + sg, s1 - 1);           // past the range: a valid split, weight 0
            v[i] = *reinterpret_cast<const float2*>(o + (int64_t)s * kD);
            mv[i] = m[s];
            lv[i] = l[s];
        }
        float mb = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (b0 + 8 * i + sg >= s1) mv[i] = -INFINITY;
            mb = fmaxf(mb, mv[i]);
        }
        const float mn = fmaxf(mw, wave_max(mb));
        if (mn != mw) {                                           // uniform; mn > -inf here
            const float r = fast_exp2(mw - mn);                   // 0 while mw is -inf
            n0 *= r;
            n1 *= r;
            den *= r;
            mw = mn;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float w = mv[i] == -INFINITY ? 0.f : fast_exp2(mv[i] - mw);
            n0 = __builtin_fmaf(v[i].x, w, n0);
            n1 = __builtin_fmaf(v[i].y, w, n1);
            den = __builtin_fmaf(lv[i], w, den);
        }
    }
#pragma unroll
    for (int d = 8; d < 64; d <<= 1) {
        n0 += __shfl_xor(n0, d);
        n1 += __shfl_xor(n1, d);
        den += __shfl_xor(den, d);
    }
    if (sg == 0) {
        part[wave][0][cp] = n0;
        part[wave][1][cp] = n1;
        part[wave][2][cp] = den;
        part[wave][3][cp] = mw;
    }
    __syncthreads();
    if (wave == 0 && sg == 0) {
        float M = part[0][3][cp];
#pragma unroll
        for (int w = 1; w < kWideWaves; ++w) M = fmaxf(M, part[w][3][cp]);
        float a0 = 0.f, a1 = 0.f, dn = 0.f;
#pragma unroll
        for (int w = 0; w < kWideWaves; ++w) {
            const float mwv = part[w][3][cp];
            const float f = mwv == -INFINITY ? 0.f : fast_exp2(mwv - M);
            a0 = __builtin_fmaf(part[w][0][cp], f, a0);
            a1 = __builtin_fmaf(part[w][1][cp], f, a1);
            dn = __builtin_fmaf(part[w][2][cp], f, dn);
        }
        reinterpret_cast<uint32_t*>(out + row * kD + c0)[cp] = pack_bf16x2(a0 / dn, a1 / dn);
    }
}


// ---- split kernel for head dims 64 and 256 (the reference builds head dim 128 only,
// cache.py:21; its kernels.py:142-194 at other head sizes)
//
// Grid: one workgroup per (sequence, split, group of 16 query heads, KV head), numbered so
// that the KV heads of one (sequence, split) run together on one XCD (see the kernel).
// NPH wavefronts per workgroup (page phases: 4 for D = 64, 2 for D = 256) take the
// split's pages round robin and are merged through LDS at the end, one partial per
// (split, query head), so the workspace and the merge are those of the D = 128 kernels.
//
// Memory pipeline: each wavefront brings its pages into its own NS-stage LDS ring with
// direct-to-LDS loads (global_load_lds_dwordx4, 16 bytes per lane: one load per KiB of the
// page's image), so that a page in flight costs no registers; a stage is read only after
// the wavefront's own s_waitcnt vmcnt(n) for it (n = the loads issued after it). Row pieces
// land XOR-swizzled (16-byte chunk c of row r at chunk c ^ key(r)), which keeps the later
// reads of one chunk across 16 rows at the minimum of two LDS passes. A compressed page
// with one or two raw rows (K and V together) brings them along with one more load into
// the stage's raw slot; pages with more (rare) read them from the pool directly.
//
// Per page: lane (token r, channel group g) reads its bytes from the stage in the rebuild
// layout (tile.hpp, any head dim), rebuilds K and V, splices raw rows, and runs the MFMA
// formulation of the D = 128 kernels: S^T = K Q^T with v_mfma_f32_16x16x32_bf16 over D/32
// k-blocks, and P.V from V^T read with ds_read_b64_tr_b16 (lane (r, g) supplies row
// 4g + r/4, channels 16nb + 4(r & 3) .. + 3, and receives channel 16nb + r of rows 4g ..
// 4g + 3) -- out of a per-wavefront tile of the rebuilt V (rows of 2D + 32 bytes, so each
// bank serves two of a read's lanes), or, in the bf16 twin, straight out of its stage.
// Both run the same arithmetic on the same values, so they agree bit for bit.
template <int D, bool COMP>
struct DGen {
    static constexpr int NPH = D >= 256 ? 2 : 4;     // page phases (wavefronts) per workgroup
    static constexpr int R = Run<D>::R;             // channels per lane run
    static constexpr int V = Run<D>::V;             // value dwords per lane (K or V of a page)
    static constexpr int KC = D / 32;               // score MFMA k-blocks
    static constexpr int NB = D / 16;               // 16-channel blocks of V and O
    // page stage: compressed sm K [16][D] | sm V | code K [16][D/2] | code V | base K [D] |
    // base V [D]; bf16 twin: K rows [16][2D] | V rows
    static constexpr int SMK = 0, SMV = 16 * D, CODE = 32 * D, BASE = 48 * D;
    static constexpr int BK = 0, BV = 32 * D;
    static constexpr int STAGE = COMP ? 50 * D : 64 * D;
    static constexpr int NDMA = COMP ? 3 * D / 64 + 1 : D / 16;   // 16-byte loads per lane and page
    static constexpr int NS = COMP && D == 64 ? 3 : 2;             // ring stages per wavefront
    static constexpr int NRAW = 2;                                // raw rows per page through the ring
    static constexpr int RAWB = COMP ? NRAW * 2 * D : 0;          // a stage's raw slot
    static constexpr int RING = NS * (STAGE + RAWB);
    static constexpr int TROW = 2 * D + 32;                       // V tile row (bytes)
    static constexpr int TILE = COMP ? kPage * TROW : 0;
    static constexpr int PER_WAVE = RING + TILE;
    static constexpr int LDS = NPH * PER_WAVE;
    static constexpr int MROW = D + 4;                            // one head's partial in the merge (floats)
    static constexpr int MBYTES = (16 * MROW + 32) * 4;
    static constexpr int MAXWAIT = (NS - 1) * (NDMA + 1);          // loads a stage's wait lets stay in flight
    static_assert(RING >= MBYTES, "a wavefront's ring holds its partial for the merge");
    static_assert(NDMA * 1024 >= STAGE && (NDMA - 1) * 1024 < STAGE, "one load per KiB of the stage");
    static_assert(MAXWAIT <= 63, "the waits must fit vmcnt");
};

// Physical 16-byte chunk of logical chunk c in row r of an LDS image with rows of LB bytes:
// c XOR the row's index among the rows that start on the same bank (rows LB apart cycle
// through the 256 bytes of banks every 256 / LB rows).
template <int LB>
__device__ constexpr int dswz(int r, int c) {
    constexpr int C = LB / 16, RPB = LB >= 256 ? 1 : 256 / LB;
    return c ^ ((r / RPB) % C);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ inline uint2 lds8(const lds_u8* p) {
    const u32x2 v = *reinterpret_cast<const EXKV_LDS u32x2*>(p);
    return make_uint2(v.x, v.y);
}

// N bytes (8, 16, 32 or 64) of row r of a swizzled image at img, from logical byte b0
// (8-aligned for N = 8, 16-aligned otherwise), as dwords.
template <int LB, int N>
__device__ inline void dread(uint32_t img, int r, int b0, uint32_t* out) {
    if constexpr (N == 8) {
        const uint2 v = lds8(lds_ptr(img + (uint32_t)(r * LB + dswz<LB>(r, b0 >> 4) * 16 + (b0 & 8))));
        out[0] = v.x;
        out[1] = v.y;
    } else {
#pragma unroll
        for (int i = 0; i < N / 16; ++i) {
            const uint4 v = lds16(lds_ptr(img + (uint32_t)(r * LB + dswz<LB>(r, (b0 >> 4) + i) * 16)));
            out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
        }
    }
}

// A lane's loads of a page (fixed for the kernel): load i takes 16 bytes at off[i] from the
// page's first row in its array (the K or the V array: bit i of vmask), lands them at stage
// byte 1024 i + 16 lane, and is issued when bit i of act is set.
template <int D, bool COMP>
struct DLanes {
    uint32_t off[DGen<D, COMP>::NDMA];
    uint32_t vmask, act;
};

template <int D, bool COMP>
__device__ inline DLanes<D, COMP> dgen_lanes(int Hkv, int lane) {
    using G = DGen<D, COMP>;
    DLanes<D, COMP> o{};
#pragma unroll
    for (int i = 0; i < G::NDMA; ++i) {
        const int byte = 1024 * i + 16 * lane;         // in the stage image
        bool v = false, on = true;
        uint32_t off = 0;
        if constexpr (COMP) {
            if (byte < G::CODE) {                      // sm rows of D bytes
                v = byte >= G::SMV;
                const int b = byte - (v ? G::SMV : 0), row = b / D;
                off = (uint32_t)(row * Hkv * D + dswz<D>(row, (b % D) >> 4) * 16);
            } else if (byte < G::BASE) {               // code rows of D/2 bytes
                v = byte >= G::CODE + 8 * D;
                const int b = byte - G::CODE - (v ? 8 * D : 0), row = b / (D / 2);
                off = (uint32_t)(row * Hkv * (D / 2) + dswz<D / 2>(row, (b % (D / 2)) >> 4) * 16);
            } else {                                   // base rows of the page: K, then V
                on = byte < G::STAGE;
                v = byte >= G::BASE + D;
                off = (uint32_t)((byte - G::BASE) % D);
            }
        } else {                                       // bf16 rows of 2D bytes
            v = byte >= G::BV;
            const int b = byte - (v ? G::BV : 0), row = b / (2 * D);
            off = (uint32_t)(row * Hkv * 2 * D + dswz<2 * D>(row, (b % (2 * D)) >> 4) * 16);
        }
        o.off[i] = off;
        o.vmask |= (v ? 1u : 0u) << i;
        o.act |= (on ? 1u : 0u) << i;
    }
    return o;
}

struct DMeta {              // rowmask / rowoff of a page of the K and V caches (uniform)
    uint32_t mk, mv;
    int32_t ok, ov;
};
__device__ inline bool draw_in_ring(const DMeta& m) {
    const int n = __builtin_popcount(m.mk) + __builtin_popcount(m.mv);
    return n > 0 && n <= 2;
}

// Pool page of page p of sequence b (uniform): contiguous, or through the block table.
__device__ inline int64_t dgen_pidx(const AttnArgs& a, int b, int NP, int p) {
    if (a.block_table == nullptr) return (int64_t)b * NP + p;
    return (int64_t)min((uint32_t)const_ld(a.block_table + b * a.bt_stride + p), (uint32_t)(a.pool_pages - 1));
}

template <bool COMP>
__device__ inline DMeta dgen_meta(const AttnArgs& a, int64_t page) {
    DMeta m{0u, 0u, 0, 0};
    if constexpr (COMP) {
        m.mk = (uint32_t)const_ld(a.k.rowmask + page);
        m.mv = (uint32_t)const_ld(a.v.rowmask + page);
        m.ok = const_ld(a.k.rowoff + page);
        m.ov = const_ld(a.v.rowoff + page);
    }
    return m;
}

// Issue a page's loads into stage st (and, compressed, its raw rows into raw_st when they
// travel through the ring). Returns the number of loads issued.
template <int D, bool COMP>
__device__ inline int dgen_issue(const AttnArgs& a, const DLanes<D, COMP>& o, int64_t pidx, int hk, const DMeta& m,
                                 uint32_t st, uint32_t raw_st, int lane) {
    using G = DGen<D, COMP>;
    const int64_t row0 = pidx * kPage * a.Hkv + hk, page = pidx * a.Hkv + hk;
    // the stage (and its raw slot) was last read by this wavefront NS pages ago: those LDS
    // reads complete before the loads can land there
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // the page's first row in each array, K and V (uniform; per-lane selects stay selects)
    auto u64 = [](const void* p) { return (uint64_t)(uintptr_t)p; };
    PairSrc sm{}, code{}, base{}, bf{};
    if constexpr (COMP) {
        sm = pair_src(u64(a.k.sm) + (uint64_t)row0 * D, u64(a.v.sm) + (uint64_t)row0 * D);
        code = pair_src(u64(a.k.code) + (uint64_t)row0 * (D / 2), u64(a.v.code) + (uint64_t)row0 * (D / 2));
        base = pair_src(u64(a.k.base) + (uint64_t)page * D, u64(a.v.base) + (uint64_t)page * D);
    } else {
        bf = pair_src(u64(a.kb) + (uint64_t)row0 * (2 * D), u64(a.vb) + (uint64_t)row0 * (2 * D));
    }
#pragma unroll
    for (int i = 0; i < G::NDMA; ++i) {
        const bool v = (o.vmask >> i) & 1u;
        const int byte = 1024 * i;                     // the load's array is fixed by its position
        const PairSrc& ps = !COMP ? bf : (byte < G::CODE ? sm : (byte < G::BASE ? code : base));
        if ((o.act >> i) & 1u) dma16_stream((const void*)(uintptr_t)(ps.pick(v) + o.off[i]), st + 1024u * i);
    }
    int n = G::NDMA;
    if constexpr (COMP) {
        if (draw_in_ring(m)) {                         // uniform
            // raw rows of the page (K rows in token order, then V rows): entry e = lane /
            // (D/8), 16 bytes per lane; pool slot = rowoff + rank of the row
            constexpr int LPR = D / 8;                 // lanes per raw row
            const int nk = __builtin_popcount(m.mk), nr = nk + __builtin_popcount(m.mv), e = lane / LPR;
            const bool isv = e >= nk;
            int64_t idx = isv ? (int64_t)m.ov + (e - nk) : (int64_t)m.ok + e;
            const int64_t rows = isv ? a.v.raw_rows : a.k.raw_rows;
            bool bad;
            idx = clamp_slot(idx, rows, bad);
            const uint8_t* rb = reinterpret_cast<const uint8_t*>(isv ? a.v.raw : a.k.raw);
            if (lane < LPR * nr) {
                if (bad) report_error(kErrRawSlot);
                dma16_stream(rb + idx * (2 * D) + (lane % LPR) * 16, raw_st);
            }
            ++n;
        }
    }
    return n;
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, N]
template <int N>
__device__ inline void dwait(int n) {
    if constexpr (N > 0) {
        if (n >= N) {
            wait_vm<N>();
            return;
        }
        dwait<N - 1>(n);
    } else {
        wait_vm<0>();
    }
}

// The lane's values of one raw row of the stage's raw slot (entry e: 2D bytes, unswizzled)
template <int D>
__device__ inline void draw_values(uint32_t raw_st, int e, int g, uint32_t (&out)[Run<D>::V]) {
    constexpr int R = Run<D>::R;
    const uint32_t p = raw_st + (uint32_t)(e * 2 * D + 2 * g * R);
#pragma unroll
    for (int i = 0; i < R / 8; ++i) {
        const uint4 lo = lds16(lds_ptr(p) + 16 * i), hi = lds16(lds_ptr(p) + D + 16 * i);
        out[4 * i] = lo.x; out[4 * i + 1] = lo.y; out[4 * i + 2] = lo.z; out[4 * i + 3] = lo.w;
        out[R / 2 + 4 * i] = hi.x; out[R / 2 + 4 * i + 1] = hi.y; out[R / 2 + 4 * i + 2] = hi.z;
        out[R / 2 + 4 * i + 3] = hi.w;
    }
}

// K (V = false) or V of the stage's compressed page for lane (r, g): its bytes in the
// rebuild layout, the rebuild, and its raw row spliced in (from the raw slot when the
// page's raw rows came through the ring, else from the pool: rare, and it waits for every
// load in flight).
template <int D, bool V>
__device__ inline void dgen_rebuild(const AttnArgs& a, uint32_t st, uint32_t raw_st, const DMeta& m, int r, int g,
                                    uint32_t (&d)[Run<D>::V]) {
    using G = DGen<D, true>;
    constexpr int R = Run<D>::R;
    PageBytesD<D> pb;
    const uint32_t sm = st + (V ? G::SMV : G::SMK), code = st + G::CODE + (V ? 8 * D : 0);
    dread<D, R>(sm, r, g * R, pb.sm_lo);
    dread<D, R>(sm, r, D / 2 + g * R, pb.sm_hi);
    dread<D / 2, R>(code, r, g * R, pb.code);
    dread<D, R>(st + G::BASE + (V ? D : 0), 0, g * R, pb.b_lo);     // one row: no swizzle
    dread<D, R>(st + G::BASE + (V ? D : 0), 0, D / 2 + g * R, pb.b_hi);
    rebuild_values_d<D>(pb, d);
    const uint32_t mask = V ? m.mv : m.mk;
    if (mask != 0u) {                                  // uniform
        keep_branch();
        const bool take = ((mask >> r) & 1u) != 0;
        uint32_t x[Run<D>::V];
        if (draw_in_ring(m)) {
            const int e = (V ? __builtin_popcount(m.mk) : 0) + __builtin_popcount(mask & ((1u << r) - 1u));
            draw_values<D>(raw_st, min(e, G::NRAW - 1), g, x);
        } else {
            const CSrc& c = V ? a.v : a.k;
            load_row_values_d<D>(c.raw + raw_slot(mask, V ? m.ov : m.ok, r, c.raw_rows) * D, g, x);
            wait_vm<0>();
            settle(x);
        }
#pragma unroll
        for (int i = 0; i < Run<D>::V; ++i) d[i] = take ? x[i] : d[i];
    }
}

// K of a head-dim-256 page with its base bytes through the row broadcast: lane r of row g
// reads base dword r of its row's runs (r = 0-7: channels 32g + 4r .., 8-15: 128 + 32g +
// 4(r - 8) ..), and the rebuild takes dword i of a run from lane i (low run) or 8 + i.
__device__ inline void dgen256_rebuild_k(const AttnArgs& a, uint32_t st, uint32_t raw_st, const DMeta& m, int r,
                                         int g, uint32_t (&d)[Run<256>::V]) {
    using G = DGen<256, true>;
    constexpr int D = 256, R = Run<D>::R, W = Run<D>::W;
    uint32_t sm_lo[W], sm_hi[W], code[W];
    dread<D, R>(st + G::SMK, r, g * R, sm_lo);
    dread<D, R>(st + G::SMK, r, D / 2 + g * R, sm_hi);
    dread<D / 2, R>(st + G::CODE, r, g * R, code);
    const uint32_t bw = stage_base_word(st, (uint32_t)(G::BASE + 128 * (r >> 3) + 32 * g + 4 * (r & 7)));
    const uint64_t zf = __ballot((bw & 0x80808080u) != 0u);
    constexpr uint64_t lo_lanes = 0x00FF00FF00FF00FFull;
    if ((zf & lo_lanes) != 0)
        rebuild_run_bcw<true, false, 0, 0, W>(sm_lo, code, bw, d);
    else
        rebuild_run_bcw<false, false, 0, 0, W>(sm_lo, code, bw, d);
    if ((zf & (lo_lanes << 8)) != 0)
        rebuild_run_bcw<true, true, 8, 0, W>(sm_hi, code, bw, d + 2 * W);
    else
        rebuild_run_bcw<false, true, 8, 0, W>(sm_hi, code, bw, d + 2 * W);
    if (m.mk != 0u) {                                  // uniform: raw K rows (dgen_rebuild's splice)
        keep_branch();
        const bool take = ((m.mk >> r) & 1u) != 0;
        uint32_t x[Run<D>::V];
        if (draw_in_ring(m)) {
            draw_values<D>(raw_st, min(__builtin_popcount(m.mk & ((1u << r) - 1u)), G::NRAW - 1), g, x);
        } else {
            load_row_values_d<D>(a.k.raw + raw_slot(m.mk, m.ok, r, a.k.raw_rows) * D, g, x);
            wait_vm<0>();
            settle(x);
        }
#pragma unroll
        for (int i = 0; i < Run<D>::V; ++i) d[i] = take ? x[i] : d[i];
    }
}

// V^T of a head-dim-256 page straight from the stage, as in the head-dim-128 kernels
// (ds_read_b64_tr_b8: rows 0-3 of a read = the lane's 4 tokens in one 16-byte chunk, rows 4-7
// the same tokens in another). Block nb (channels 16nb .. 16nb + 15) is sm chunk nb, the low
// (nb < 8) or high nibbles of code chunk nb & 7 (code byte j: channels j and j + 128), and
// byte nb of the lane's slice of the base row. 8 sm reads (chunks q and q + 8), 4 code reads
// (chunks 2c and 2c + 1) and 2 base reads (bytes 128b + 16k + i) of 8 bytes per lane.
struct Vt256Lane {
    uint32_t sm[8], code[4], base[2];
};
struct Vt256Bytes {
    uint32_t sm[16], code[8], base[4];   // sm[nb], code[nb & 7], base[nb >> 2] byte nb & 3
};
__device__ inline Vt256Lane vt256_lane_offsets(int lane) {
    using G = DGen<256, true>;
    const int L = lane & 15, kb = lane >> 4, k = L >> 1, h = L & 1, t = 4 * kb + (k & 3);
    Vt256Lane o;
#pragma unroll
    for (int q = 0; q < 8; ++q)
        o.sm[q] = (uint32_t)(G::SMV + t * 256 + dswz<256>(t, q + 8 * (k >> 2)) * 16 + 8 * h);
#pragma unroll
    for (int c = 0; c < 4; ++c)
        o.code[c] = (uint32_t)(G::CODE + 8 * 256 + t * 128 + dswz<128>(t, 2 * c + (k >> 2)) * 16 + 8 * h);
#pragma unroll
    for (int b = 0; b < 2; ++b) o.base[b] = (uint32_t)(G::BASE + 256 + 128 * b + 16 * k + 8 * h);
    return o;
}
__device__ inline void stage_vt256_bytes(uint32_t st, const Vt256Lane& o, Vt256Bytes& vb) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const uint2 v = lds_tr8(st + o.sm[q]);
        vb.sm[q] = v.x;
        vb.sm[q + 8] = v.y;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint2 v = lds_tr8(st + o.code[c]);
        vb.code[2 * c] = v.x;
        vb.code[2 * c + 1] = v.y;
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const uint2 v = lds_tr8(st + o.base[b]);
        vb.base[2 * b] = v.x;
        vb.base[2 * b + 1] = v.y;
    }
}
template <bool Z, int NB>
__device__ __forceinline__ void rebuild_vt256_block(const Vt256Bytes& vb, s16x4& out) {
    const uint32_t cd = vb.code[NB & 7];
    const uint32_t cn = (NB < 8 ? cd : cd >> 4) & 0x0F0F0F0Fu;
    const uint32_t b4 = perm_b32(vb.base[NB >> 2], vb.base[NB >> 2], (NB & 3) * 0x01010101u);
    uint32_t o01, o23;
    bf16_pairs(vb.sm[NB], Z ? exponents(cn, b4) : cn + b4, o01, o23);
    out = __builtin_bit_cast(s16x4, make_uint2(o01, o23));
}
template <bool Z, int NB0>
__device__ __forceinline__ void rebuild_vt256_run(const Vt256Bytes& vb, s16x4 (&vt)[16]) {
    rebuild_vt256_block<Z, NB0 + 0>(vb, vt[NB0 + 0]);
    rebuild_vt256_block<Z, NB0 + 1>(vb, vt[NB0 + 1]);
    rebuild_vt256_block<Z, NB0 + 2>(vb, vt[NB0 + 2]);
    rebuild_vt256_block<Z, NB0 + 3>(vb, vt[NB0 + 3]);
    rebuild_vt256_block<Z, NB0 + 4>(vb, vt[NB0 + 4]);
    rebuild_vt256_block<Z, NB0 + 5>(vb, vt[NB0 + 5]);
    rebuild_vt256_block<Z, NB0 + 6>(vb, vt[NB0 + 6]);
    rebuild_vt256_block<Z, NB0 + 7>(vb, vt[NB0 + 7]);
}
// The zero-group fix-up per run (blocks 0-7: channels 0-127, 8-15: 128-255), for the wavefront.
__device__ __forceinline__ void rebuild_vt256(const Vt256Bytes& vb, s16x4 (&vt)[16]) {
    if (__ballot(((vb.base[0] | vb.base[1]) & 0x80808080u) != 0u) != 0)
        rebuild_vt256_run<true, 0>(vb, vt);
    else
        rebuild_vt256_run<false, 0>(vb, vt);
    if (__ballot(((vb.base[2] | vb.base[3]) & 0x80808080u) != 0u) != 0)
        rebuild_vt256_run<true, 8>(vb, vt);
    else
        rebuild_vt256_run<false, 8>(vb, vt);
}

template <int D, bool COMP>
__global__ void __launch_bounds__(64 * (D >= 256 ? 2 : 4)) attn_dgen_kernel(AttnArgs a) {
    using G = DGen<D, COMP>;
    static_assert(64 * G::NPH == 64 * (D >= 256 ? 2 : 4), "launch bounds");
    constexpr int R = G::R, NS = G::NS;
    __shared__ __attribute__((aligned(16))) uint8_t lds[G::LDS];
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));   // uniform, in an SGPR
    // XCD-aware order: workgroups go to the 8 XCDs round robin (linear id mod 8), and a
    // workgroup reads only its KV head's share of each token row (64 / 32-byte pieces at
    // D = 64), so the KV heads of one (sequence, split) are given consecutive ids on one
    // XCD, where they run together and share the L2 lines of their rows.
    int item;
    {
        const int L = blockIdx.x, N = gridDim.x, q = N >> 3, rem = N & 7, x = L & 7, pos = L >> 3;
        item = x < rem ? x * (q + 1) + pos : rem * (q + 1) + (x - rem) * q + pos;
    }
    const int hk = item % a.Hkv;
    item /= a.Hkv;
    const int hg = item % a.HG;
    item /= a.HG;
    const int split = item % a.nsplit, b = item / a.nsplit;
    int len = a.lens ? const_ld(a.lens + b * a.lens_stride) : a.T;
    len = min(max(len, 0), a.TS);
    const int wlo = a.window > 0 ? max(len - a.window, 0) : 0;   // sliding window: tokens [wlo, len)
    const int start = (wlo & ~(kPage - 1)) + split * a.split_len;
    const int end = min(start + a.split_len, len);
    const int NP = a.TS / kPage, p0 = start / kPage, pend = end > start ? (end + kPage - 1) / kPage : p0;
    const int gh = min(16, a.G - hg * 16);

    const uint32_t ring = lds_addr(lds) + (uint32_t)(wave * G::PER_WAVE);   // this wavefront's (uniform)
    auto stage = [&](int s) { return ring + (uint32_t)(s * G::STAGE); };
    auto raw_slot_of = [&](int s) { return ring + (uint32_t)(NS * G::STAGE + s * G::RAWB); };
    const DLanes<D, COMP> dl = dgen_lanes<D, COMP>(a.Hkv, lane);

    // the first NS pages' loads leave before anything else
    const int pfirst = p0 + wave;
    DMeta meta[NS];
    int cnt[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int p = pfirst + s * G::NPH;
        cnt[s] = 0;
        meta[s] = DMeta{0u, 0u, 0, 0};
        if (p < pend) {
            const int64_t pidx = dgen_pidx(a, b, NP, p);
            meta[s] = dgen_meta<COMP>(a, pidx * a.Hkv + hk);
            cnt[s] = dgen_issue<D, COMP>(a, dl, pidx, hk, meta[s], stage(s), raw_slot_of(s), lane);
        }
    }

    // Q^T operand: column = head hg*16 + r, k-block kc = channels of dwords 4kc.. of a lane's values
    bf16x8 qop[G::KC];
    {
        const uint16_t* qr = a.q + ((int64_t)b * a.Hq + (int64_t)hk * a.G + hg * 16 + min(r, gh - 1)) * D;
#pragma unroll
        for (int kc = 0; kc < G::KC; ++kc) {
            const int d0 = kc < G::KC / 2 ? g * R + 8 * kc : D / 2 + g * R + 8 * (kc - G::KC / 2);
            uint4 v = *reinterpret_cast<const uint4*>(qr + d0);
            if (r >= gh) v = make_uint4(0u, 0u, 0u, 0u);
            qop[kc] = as_bf16x8(v.x, v.y, v.z, v.w);
            asm volatile("" : "+v"(qop[kc]));
        }
    }
    f32x4 acc[G::NB];
#pragma unroll
    for (int nb = 0; nb < G::NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_i = -INFINITY, l_i = 0.f;
    const uint32_t tile = ring + (uint32_t)G::RING;
    const uint32_t tw = tile + (uint32_t)(r * G::TROW + 2 * g * R);                     // V tile row r, low run
    const uint32_t tr = tile + (uint32_t)((4 * g + (r >> 2)) * G::TROW + 8 * (r & 3));  // transposed reads
    const int trow = 4 * g + (r >> 2);                 // twin: the row this lane's transposed reads supply
    [[maybe_unused]] Vt256Lane vto{};
    if constexpr (COMP && D == 256) vto = vt256_lane_offsets(lane);

    for (int p = pfirst; p < pend; p += NS * G::NPH) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int pi = p + s * G::NPH;
            if (pi >= pend) break;
            const int pn = pi + NS * G::NPH;
            int64_t pidx_n = 0;
            DMeta mn{0u, 0u, 0, 0};
            if (pn < pend) {                           // the refill's metadata, early
                pidx_n = dgen_pidx(a, b, NP, pn);
                mn = dgen_meta<COMP>(a, pidx_n * a.Hkv + hk);
            }
            int after = 0;                             // loads issued after this stage's page
#pragma unroll
            for (int t = 0; t < NS; ++t)
                if (t != s) after += cnt[t];
            dwait<G::MAXWAIT>(after);
            const uint32_t st = stage(s);
            const int t0 = pi * kPage;
            const bool ragged = t0 < wlo || t0 + kPage > end;
            const bool valid = t0 + r >= wlo && t0 + r < end;
            uint32_t kd[G::V];
            s16x4 vt[G::NB];
            if constexpr (COMP) {
                bool tiled = true;                     // V through the bf16 tile
                if constexpr (D == 256) {
                    if (meta[s].mv == 0u) {            // uniform: V^T from transposing byte reads
                        Vt256Bytes vb;
                        stage_vt256_bytes(st, vto, vb);
                        rebuild_vt256(vb, vt);
                        if (ragged) {
                            keep_branch();
                            vt_zero_invalid(vt, t0 + 4 * g, end, wlo);
                        }
                        tiled = false;
                    }
                }
                if (tiled) {                           // head dim 64, and pages with raw V rows
                    uint32_t vd[G::V];
                    dgen_rebuild<D, true>(a, st, raw_slot_of(s), meta[s], r, g, vd);
                    if (ragged && !valid) {            // rows outside [wlo, end) read as zero V
#pragma unroll
                        for (int i = 0; i < G::V; ++i) vd[i] = 0u;
                    }
#pragma unroll
                    for (int i = 0; i < R / 8; ++i) {  // the two runs of row r into the V tile
                        lds_st16(lds_ptr(tw) + 16 * i, vd[4 * i], vd[4 * i + 1], vd[4 * i + 2], vd[4 * i + 3]);
                        lds_st16(lds_ptr(tw) + D + 16 * i, vd[R / 2 + 4 * i], vd[R / 2 + 4 * i + 1],
                                 vd[R / 2 + 4 * i + 2], vd[R / 2 + 4 * i + 3]);
                    }
                }
                if constexpr (D == 256)
                    dgen256_rebuild_k(a, st, raw_slot_of(s), meta[s], r, g, kd);
                else
                    dgen_rebuild<D, false>(a, st, raw_slot_of(s), meta[s], r, g, kd);
                if (tiled) {
#pragma unroll
                    for (int nb = 0; nb < G::NB; ++nb)
                        vt[nb] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EXKV_LDS s16x4*)lds_ptr(tr + 32 * nb));
                }
            } else {
                dread<2 * D, 2 * R>(st + G::BK, r, 2 * g * R, kd);
                dread<2 * D, 2 * R>(st + G::BK, r, D + 2 * g * R, kd + R / 2);
                const uint32_t vs = st + G::BV;
                if (ragged) {                          // rows outside [wlo, end) read as zero V
                    keep_branch();
                    if (!valid) {
#pragma unroll
                        for (int i = 0; i < 2 * R / 16; ++i) {
                            lds_st16(lds_ptr(vs + (uint32_t)(r * 2 * D + dswz<2 * D>(r, (2 * g * R >> 4) + i) * 16)),
                                     0u, 0u, 0u, 0u);
                            lds_st16(lds_ptr(vs + (uint32_t)(r * 2 * D + dswz<2 * D>(r, ((D + 2 * g * R) >> 4) + i) * 16)),
                                     0u, 0u, 0u, 0u);
                        }
                    }
                }
#pragma unroll
                for (int nb = 0; nb < G::NB; ++nb) {
                    const int c = 2 * nb + ((r & 3) >> 1);    // logical chunk of channels 16nb + 4(r & 3) ..
                    const uint32_t ad = vs + (uint32_t)(trow * 2 * D + dswz<2 * D>(trow, c) * 16 + 8 * (r & 1));
                    vt[nb] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EXKV_LDS s16x4*)lds_ptr(ad));
                }
            }
            f32x4 sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < G::KC; ++kc)
                sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(kd[4 * kc], kd[4 * kc + 1], kd[4 * kc + 2], kd[4 * kc + 3]), qop[kc], sa, 0, 0, 0);
            page_softmax_pv<G::NB>(sa, vt, ragged, t0, end, wlo, g, a.qk_scale, m_i, l_i, acc);
            // refill the stage with page pn
            cnt[s] = 0;
            if (pn < pend) {
                meta[s] = mn;
                cnt[s] = dgen_issue<D, COMP>(a, dl, pidx_n, hk, mn, st, raw_slot_of(s), lane);
            }
        }
    }

    // page phases -> one partial per (split, query head): phase w > 0 leaves (o, m, l) in
    // its own ring (no loads are in flight: every issued page was consumed), phase 0
    // merges them in order (M = max m, o = sum o 2^(m - M), l alike)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    const float l_t = group_sum(l_i);
    auto mo = [&](int w) { return lds_addr(lds) + (uint32_t)(w * G::PER_WAVE); };
    if (wave > 0) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int nb = 0; nb < G::NB; ++nb)
            *reinterpret_cast<EXKV_LDS f32x4*>(lds_ptr(mo(wave) + 4u * (r * G::MROW + 16 * nb + 4 * g))) = acc[nb];
        if (g == 0) {
            *reinterpret_cast<EXKV_LDS float*>(lds_ptr(mo(wave) + 4u * (16 * G::MROW + r))) = m_i;
            *reinterpret_cast<EXKV_LDS float*>(lds_ptr(mo(wave) + 4u * (16 * G::MROW + 16 + r))) = l_t;
        }
    }
    __syncthreads();
    if (wave == 0 && r < gh) {
        auto ld_ml = [&](int w, int k) {
            return *reinterpret_cast<const EXKV_LDS float*>(lds_ptr(mo(w) + 4u * (16 * G::MROW + 16 * k + r)));
        };
        float M = fmaxf(-INFINITY, m_i);
        for (int w = 1; w < G::NPH; ++w) M = fmaxf(M, ld_ml(w, 0));
        f32x4 o[G::NB];
#pragma unroll
        for (int nb = 0; nb < G::NB; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        float l = 0.f;
        if (M != -INFINITY) {
            const float wt = fast_exp2(m_i - M);
#pragma unroll
            for (int nb = 0; nb < G::NB; ++nb)
#pragma unroll
                for (int k = 0; k < 4; ++k) o[nb][k] += wt * acc[nb][k];
            l += wt * l_t;
            for (int w = 1; w < G::NPH; ++w) {
                const float wp = fast_exp2(ld_ml(w, 0) - M);
#pragma unroll
                for (int nb = 0; nb < G::NB; ++nb) {
                    const f32x4 v = *reinterpret_cast<const EXKV_LDS f32x4*>(
                        lds_ptr(mo(w) + 4u * (r * G::MROW + 16 * nb + 4 * g)));
#pragma unroll
                    for (int k = 0; k < 4; ++k) o[nb][k] += wp * v[k];
                }
                l += wp * ld_ml(w, 1);
            }
        }
        const int64_t prow = ((int64_t)b * a.Hq + (int64_t)hk * a.G + hg * 16 + r) * a.nsplit + split;
#pragma unroll
        for (int nb = 0; nb < G::NB; ++nb) *reinterpret_cast<f32x4*>(a.part_o + prow * D + 16 * nb + 4 * g) = o[nb];
        if (g == 0) {
            a.part_m[prow] = M;
            a.part_l[prow] = l;
        }
    }
}

// Split merge for head dims 64 and 256: one wavefront per (sequence, query head) row, lane
// = D/64 consecutive channels. The splits go in batches of 32 with every load of a batch in
// flight (lane s of the batch reads m and l of split s, every lane its channels of each
// split's o); the sums run over s in order with fmas (out = sum o_s w_s / sum l_s w_s, w_s
// = 2^(m_s - max m)). Used by the compressed call and its twin alike.
template <int D>
__global__ void __launch_bounds__(64) attn_reduce_d_kernel(const float* po, const float* pm, const float* pl,
                                                           uint16_t* out, int ns) {
    constexpr int C = D / 64;
    constexpr int NBATCH = 32;
    typedef float fC __attribute__((ext_vector_type(C)));
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const float* m = pm + row * ns;
    const float* l = pl + row * ns;
    const float* o = po + row * ns * D + lane * C;
    float M = -INFINITY;
    for (int s = lane; s < ns; s += 64) M = fmaxf(M, m[s]);
    M = wave_max(M);
    fC n;
#pragma unroll
    for (int c = 0; c < C; ++c) n[c] = 0.f;
    float den = 0.f;
    for (int s0 = 0; s0 < ns; s0 += NBATCH) {
        const int nb = min(NBATCH, ns - s0);
        const float mv = lane < nb ? m[s0 + lane] : -INFINITY;
        const float lv = lane < nb ? l[s0 + lane] : 0.f;
        fC v[NBATCH];
#pragma unroll
        for (int i = 0; i < NBATCH; ++i)
            if (i < nb) v[i] = *reinterpret_cast<const fC*>(o + (int64_t)(s0 + i) * D);
        const float ws = fast_exp2(mv - M);
#pragma unroll
        for (int i = 0; i < NBATCH; ++i)
            if (i < nb) {
                const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ws), i));
                const float li = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), i));
#pragma unroll
                for (int c = 0; c < C; ++c) n[c] = __builtin_fmaf(v[i][c], w, n[c]);
                den = __builtin_fmaf(li, w, den);
            }
    }
    uint16_t* dst = out + row * D + lane * C;
    if constexpr (C == 1) {
        const __bf16 r = (__bf16)(n[0] / den);
        dst[0] = __builtin_bit_cast(uint16_t, r);
    } else {
#pragma unroll
        for (int c = 0; c < C; c += 2) reinterpret_cast<uint32_t*>(dst)[c / 2] = pack_bf16x2(n[c] / den, n[c + 1] / den);
    }
}

// ---- head dim 64 as pairs of KV heads (attn_pair_kernel)
//
// KV heads 2v and 2v + 1 of a token row are 64 + 64 contiguous bytes of sm, 32 + 32 of
// codes (64 + 64 of base per page, 128 + 128 bytes of a bf16 row): "virtual head" v has
// the byte layout of one head-dim-128 head. The head-dim-128 split kernels' workgroup
// structure, loader wavefronts, DMA pattern, ring and flags serve the pairs as they are,
// with Hkv / 2 virtual heads (a workgroup covers HW of them: min(gcd(Hkv / 2, 8), 4)), so
// every load moves the pair's 128-byte sm and 64-byte code rows; what differs is the
// compute side:
//   * lane (token r, channel group g) takes channels 8g..8g+7 and 32+8g..32+8g+7 of both
//     heads: its PageBytes hold head 2v's 8 bytes, then head 2v+1's, so rebuild_values
//     gives out[0..3] = head 2v channels 8g.., out[4..7] = head 2v+1's, out[8..11] = head
//     2v channels 32+8g.., out[12..15] = head 2v+1's;
//   * a head's scores are two MFMA k-blocks of its own channels (no product crosses the
//     heads), with its own group of query heads as the columns; one online softmax each;
//   * the V tile holds the pair in virtual-channel order (head 2v, then 2v+1), so the
//     V^T reads of the head-dim-128 kernels give channel blocks 0-3 of head 2v and 4-7 of
//     head 2v+1;
//   * metadata and raw rows per real head: up to kRawPair raw rows (128 bytes each) of a
//     page travel through the wavefront's raw slot, in the order 2v K, 2v V, 2v+1 K, 2v+1 V;
//   * partials per real head (64 channels), merged by attn_reduce_d_kernel<64>, or the
//     output itself for one split.
// The compressed kernel and its bf16 twin share the per-page arithmetic: same bits.
constexpr int kDp = 64;
constexpr int kRawPair = 4;
static_assert(kRawPair * 2 * kDp <= kRawSlot, "a raw slot holds kRawPair head-dim-64 rows");

struct PairMeta {
    PageMeta h[2];
};
__device__ inline int pair_raw_rows(const PairMeta& m) { return raw_rows_of(m.h[0]) + raw_rows_of(m.h[1]); }
__device__ inline bool pair_raw_in_ring(const PairMeta& m) {
    const int n = pair_raw_rows(m);
    return n > 0 && n <= kRawPair;
}
__device__ inline int pair_raw_loads(const PairMeta& m) { return pair_raw_in_ring(m) ? 1 : 0; }

__device__ inline void stage_bytes_pair(uint32_t sb, const PairLane& o, int sm_off, int code_off, int base_off,
                                        PageBytes& pb) {
    const uint2 s0 = lds8(lds_ptr(sb + o.sm[0]) + sm_off), s1 = lds8(lds_ptr(sb + o.sm[1]) + sm_off);
    const uint2 s2 = lds8(lds_ptr(sb + o.sm[2]) + sm_off), s3 = lds8(lds_ptr(sb + o.sm[3]) + sm_off);
    const uint2 c0 = lds8(lds_ptr(sb + o.code[0]) + code_off), c1 = lds8(lds_ptr(sb + o.code[1]) + code_off);
    const lds_u8* bp = lds_ptr(sb) + base_off;
    const uint2 b0 = lds8(bp + o.base[0]), b1 = lds8(bp + o.base[1]), b2 = lds8(bp + o.base[2]),
                b3 = lds8(bp + o.base[3]);
    pb.sm_lo = make_uint4(s0.x, s0.y, s1.x, s1.y);
    pb.sm_hi = make_uint4(s2.x, s2.y, s3.x, s3.y);
    pb.code = make_uint4(c0.x, c0.y, c1.x, c1.y);
    pb.b_lo = make_uint4(b0.x, b0.y, b1.x, b1.y);
    pb.b_hi = make_uint4(b2.x, b2.y, b3.x, b3.y);
}

__device__ inline void stage_sm_code_pair(uint32_t sb, const PairLane& o, int sm_off, int code_off, StageSC& sc) {
    stage_sm_code_pair_from([&](uint32_t off, int arr) { return lds8(lds_ptr(sb + off) + arr); }, o, sm_off, code_off, sc);
}

__device__ inline void stage_bf16_k_pair(uint32_t sb, const PairLane& o, uint32_t out[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 v = lds16(lds_ptr(sb + o.bk[j]) + BS_K);
        out[4 * j] = v.x; out[4 * j + 1] = v.y; out[4 * j + 2] = v.z; out[4 * j + 3] = v.w;
    }
}

__device__ inline void write_v_tile_pair(uint32_t sb, const PairLane& o, int toff, const uint32_t v[16]) {
    lds_u8* p0 = lds_ptr(sb + o.tw[0]) + toff;         // head 2v channels 8g.. (+128: head 2v+1's)
    lds_u8* p1 = lds_ptr(sb + o.tw[1]) + toff;         // head 2v channels 32+8g.. (+128: head 2v+1's)
    lds_st16(p0, v[0], v[1], v[2], v[3]);
    lds_st16(p1, v[8], v[9], v[10], v[11]);
    lds_st16(p0 + 128, v[4], v[5], v[6], v[7]);
    lds_st16(p1 + 128, v[12], v[13], v[14], v[15]);
}

// The page pair's raw rows into raw_st when they travel through the ring: entry e = lane /
// 8 (8 lanes x 16 bytes per 128-byte row), K rows of head 2v, its V rows, then head 2v+1's.
__device__ inline void dma_pair_raw(int lane, const PairMeta& m, uint32_t raw_st, const PairSrc& rawp,
                                    const PairSrc& rawn) {
    if (!pair_raw_in_ring(m)) return;                  // uniform
    // the slot was last read by this wavefront's splice of two pages back
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int e = lane >> 3;
    const int n0k = __builtin_popcount(m.h[0].mk), n0 = n0k + __builtin_popcount(m.h[0].mv);
    const int n1k = n0 + __builtin_popcount(m.h[1].mk), n = n1k + __builtin_popcount(m.h[1].mv);
    const bool isv = (e >= n0k && e < n0) || e >= n1k;
    const int32_t off = e < n0k ? m.h[0].ok + e
                      : e < n0  ? m.h[0].ov + (e - n0k)
                      : e < n1k ? m.h[1].ok + (e - n0)
                                : m.h[1].ov + (e - n1k);
    bool bad;
    const int64_t idx = clamp_slot((int64_t)off, (int64_t)rawn.pick(isv), bad);
    if (lane < 8 * n) {
        if (bad) report_error(kErrRawSlot);
        dma16_stream((const void*)(uintptr_t)(rawp.pick(isv) + (uint64_t)idx * (2 * kDp) + (uint64_t)(lane & 7) * 16), raw_st);
    }
}

// Splice the pair's raw K (V = false) or V rows into the lane's values: head k's are
// d[4k..4k+3] (channels 8g..) and d[8+4k..] (32+8g..). From the raw slot when the page's
// rows came through the ring, else straight from the pool (rare; waits for every load).
template <bool V>
__device__ inline void splice_pair(const AttnArgs& a, const PairMeta& m, uint32_t slot, int r, int g,
                                   uint32_t d[16]) {
    const uint32_t below = (1u << r) - 1u;
    const bool ring = pair_raw_in_ring(m);
    int e0 = 0;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const PageMeta& mh = m.h[k];
        const uint32_t mask = V ? mh.mv : mh.mk;
        if (mask != 0u) {                              // uniform
            uint32_t x[8];
            if (ring) {
                const int e = e0 + (V ? __builtin_popcount(mh.mk) : 0) + __builtin_popcount(mask & below);
                const lds_u8* p = lds_ptr(slot + (uint32_t)(min(e, kRawPair - 1) * 2 * kDp));
                const uint4 lo = lds16(p + 16 * g), hi = lds16(p + 64 + 16 * g);
                x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
                x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
            } else {
                const CSrc& c = V ? a.v : a.k;
                const int64_t sl = raw_slot(mask, V ? mh.ov : mh.ok, r, c.raw_rows);
                const uint8_t* rp = reinterpret_cast<const uint8_t*>(c.raw + sl * kDp);
                const uint4 lo = ld16(rp + 16 * g), hi = ld16(rp + 64 + 16 * g);
                x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
                x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
                wait_vm<0>();
                settle(x);
            }
            const bool take = ((mask >> r) & 1u) != 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                d[4 * k + i] = take ? x[i] : d[4 * k + i];
                d[8 + 4 * k + i] = take ? x[4 + i] : d[8 + 4 * k + i];
            }
        }
        e0 += raw_rows_of(mh);
    }
}

// q of the pair's query heads through LDS: head 2v + k's (k = 0, 1) query heads hg*16 + i,
// i < gh, at qst + 2048 k + 128 i (64 channels), by direct-to-LDS loads of 8 rows each.
__device__ inline void q_dma_pair(const AttnArgs& a, int b, int hk0, int hg, int gh, int lane, uint32_t qst) {
    const int nq = (gh + 7) >> 3;
    for (int k = 0; k < 2; ++k)
        for (int d = 0; d < nq; ++d) {
            const int i = min(8 * d + (lane >> 3), gh - 1);
            dma16(a.q + ((int64_t)b * a.Hq + (int64_t)(hk0 + k) * a.G + hg * 16 + i) * kDp + 8 * (lane & 7),
                  qst + (uint32_t)(2048 * k + 1024 * d));
        }
}

// Q^T operands: qop[2k + j] = head 2v + k's query head r (column), channels 8g + 32j ..
// 8g + 32j + 7 (the k-elements lane group g supplies); heads past the group are zero.
__device__ inline void load_qop_pair(uint32_t qst, int r, int g, int gh, bf16x8 (&qop)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = i >> 1, j = i & 1;
        uint4 v = lds16(lds_ptr(qst + (uint32_t)(2048 * k + r * 128 + 2 * (8 * g + 32 * j))));
        if (r >= gh) v = make_uint4(0u, 0u, 0u, 0u);
        qop[i] = as_bf16x8(v.x, v.y, v.z, v.w);
        asm volatile("" : "+v"(qop[i]));
    }
}

// Each head's score MFMAs, over its own channels: head 2v's k-blocks are out[0..3] and
// out[8..11], head 2v+1's out[4..7] and out[12..15]
__device__ inline void pair_scores(const uint32_t (&kd)[16], const bf16x8 (&qop)[4], f32x4& s0, f32x4& s1) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kd[0], kd[1], kd[2], kd[3]), qop[0], z, 0, 0, 0);
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kd[8], kd[9], kd[10], kd[11]), qop[1], s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kd[4], kd[5], kd[6], kd[7]), qop[2], z, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kd[12], kd[13], kd[14], kd[15]), qop[3], s1, 0, 0, 0);
}

// One page of the pair after its scores: V^T operands of both heads, then each head's
// online softmax and P.V (head 2v, then 2v+1)
__device__ __forceinline__ void pair_softmax_pv(const f32x4& s0, const f32x4& s1, const s16x4 (&vt)[8], bool ragged,
                                                int t0, const SplitCoords& c, int g, float qk_scale, float (&m_i)[2],
                                                float (&l_i)[2], f32x4 (&acc0)[4], f32x4 (&acc1)[4]) {
    const s16x4 v0[4] = {vt[0], vt[1], vt[2], vt[3]}, v1[4] = {vt[4], vt[5], vt[6], vt[7]};
    page_softmax_pv<4>(s0, v0, ragged, t0, c.end, c.wlo, g, qk_scale, m_i[0], l_i[0], acc0);
    page_softmax_pv<4>(s1, v1, ragged, t0, c.end, c.wlo, g, qk_scale, m_i[1], l_i[1], acc1);
}

// Partials of the pair: a head's row in LDS is kMoRowP floats (64 channels, padded)
constexpr int kMoRowP = kDp + 4;
constexpr int kMoHeadP = (16 * kMoRowP + 32) * 4;      // bytes of one head's partial (o, then m[16], l[16])
static_assert(Ring<true>::per_wave >= 2 * kMoHeadP && Ring<false>::per_wave >= 2 * kMoHeadP,
              "a page phase's partials of both heads fit its wavefront's ring");

// One split per row: the output with the merge's arithmetic for a single term (as
// store_direct; attn_reduce_d_kernel<64> at ns = 1 gives the same bits)
__device__ inline void store_direct_d64(const AttnArgs& a, int64_t orow, int g, const f32x4 (&o)[4], float m,
                                        float l) {
    const float w = fast_exp2(m - m);
    const float den = __builtin_fmaf(l, w, 0.f);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        float n[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) n[k] = __builtin_fmaf(o[nb][k], w, 0.f);
        *reinterpret_cast<uint2*>(a.out + orow * kDp + 16 * nb + 4 * g) =
            make_uint2(pack_bf16x2(n[0] / den, n[1] / den), pack_bf16x2(n[2] / den, n[3] / den));
    }
}

// After the page loop: both heads' partials per (split, query head), page phases merged as
// in split_epilogue (phase p > 0 leaves its partials in its ring and raises done[wave];
// phase 0 waits, bounded, and merges in phase order).
__device__ __forceinline__ void pair_epilogue(const AttnArgs& a, const SplitCoords& c, int HWv, uint32_t ring0,
                                              uint32_t ring_stride, int* done, int wave, int lane, bool active,
                                              int hk0, int gh, const f32x4 (&acc0)[4], const f32x4 (&acc1)[4],
                                              const float (&m_i)[2], const float (&l_i)[2]) {
    const int r = lane & 15, g = lane >> 4;
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    const float lt[2] = {group_sum(l_i[0]), group_sum(l_i[1])};
    const int phase = wave >> c.hw_sh;
    auto mo = [&](int w, int k) { return ring0 + (uint32_t)w * ring_stride + (uint32_t)(k * kMoHeadP); };
    auto ld_ml = [&](int w, int k, int which) {
        return *reinterpret_cast<const EXKV_LDS float*>(lds_ptr(mo(w, k) + 4u * (16 * kMoRowP + 16 * which + r)));
    };
    if (active && phase > 0) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const f32x4(&acc)[4] = k ? acc1 : acc0;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
                *reinterpret_cast<EXKV_LDS f32x4*>(lds_ptr(mo(wave, k) + 4u * (r * kMoRowP + 16 * nb + 4 * g))) = acc[nb];
            if (g == 0) {
                *reinterpret_cast<EXKV_LDS float*>(lds_ptr(mo(wave, k) + 4u * (16 * kMoRowP + r))) = m_i[k];
                *reinterpret_cast<EXKV_LDS float*>(lds_ptr(mo(wave, k) + 4u * (16 * kMoRowP + 16 + r))) = lt[k];
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_flag_st(&done[wave], 1);
    } else if (active && r < gh) {
        for (int ph = 1; ph < c.nphase; ++ph) {
            const int w = ph * HWv + wave;
            int s = 0;
            for (; s < a.spin && lds_flag_ld(&done[w]) == 0; ++s) __builtin_amdgcn_s_sleep(1);
            if (s == a.spin) report_error(kErrWait);
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const f32x4(&acc)[4] = k ? acc1 : acc0;
            float M = fmaxf(-INFINITY, m_i[k]);
            for (int ph = 1; ph < c.nphase; ++ph) M = fmaxf(M, ld_ml(ph * HWv + wave, k, 0));
            f32x4 o[4];
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            float l = 0.f;
            if (M != -INFINITY) {
                const float wt = fast_exp2(m_i[k] - M);
#pragma unroll
                for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                    for (int q = 0; q < 4; ++q) o[nb][q] += wt * acc[nb][q];
                l += wt * lt[k];
                for (int ph = 1; ph < c.nphase; ++ph) {
                    const int w = ph * HWv + wave;
                    const float wp = fast_exp2(ld_ml(w, k, 0) - M);
#pragma unroll
                    for (int nb = 0; nb < 4; ++nb) {
                        const f32x4 v = *reinterpret_cast<const EXKV_LDS f32x4*>(
                            lds_ptr(mo(w, k) + 4u * (r * kMoRowP + 16 * nb + 4 * g)));
#pragma unroll
                        for (int q = 0; q < 4; ++q) o[nb][q] += wp * v[q];
                    }
                    l += wp * ld_ml(w, k, 1);
                }
            }
            const int64_t orow = (int64_t)c.b * a.Hq + (int64_t)(hk0 + k) * a.G + c.hg * 16 + r;
            if (a.nsplit == 1 && a.out != nullptr) {
                store_direct_d64(a, orow, g, o, M, l);
            } else {
                const int64_t prow = orow * a.nsplit + c.split;
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) *reinterpret_cast<f32x4*>(a.part_o + prow * kDp + 16 * nb + 4 * g) = o[nb];
                if (g == 0) {
                    a.part_m[prow] = M;
                    a.part_l[prow] = l;
                }
            }
        }
    }
}

template <bool COMP>
__global__ void attn_pair_kernel(AttnArgs a);

// Compressed: the structure of attn_split_kernel<true> (8 compute + 2 loader wavefronts)
template <>
__global__ void __launch_bounds__(kCompThreads) attn_pair_kernel<true>(AttnArgs ar) {
    constexpr int NST = Ring<true>::nst, STB = Ring<true>::stage;
    __shared__ __attribute__((aligned(16))) uint8_t lds[Ring<true>::bytes];
    __shared__ int progress[kWaves];                   // pages done per compute wavefront (priority hint)
    __shared__ int ready[kWaves];                      // pages of wavefront w in its ring (loader -> w)
    __shared__ int avail[kWaves];                      // pages of w its loader may issue (w -> loader)
    __shared__ int done[kWaves];                       // page phase p > 0: partials left in the ring
    AttnArgs a = ar;                                   // virtual heads: the loader and coordinates see pairs
    a.Hkv = ar.Hkv / 2;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);    // uniform: scalar addressing
    const SplitCoords c = split_coords(a);
    const int hv = c.hb * a.HW + (wave & (a.HW - 1));  // virtual head: KV heads 2hv, 2hv + 1
    const int hk0 = 2 * hv;
    const int gh = min(16, ar.G - c.hg * 16);
    if (threadIdx.x < kWaves) {
        ready[threadIdx.x] = 0;
        avail[threadIdx.x] = NST - 1;                  // the last stage holds q and the page table at first
        done[threadIdx.x] = 0;
    }
    __syncthreads();

    float m_i[2] = {-INFINITY, -INFINITY}, l_i[2] = {0.f, 0.f};
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc0[nb] = acc1[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (wave >= kWaves) {
        comp_loader(a, c, lds_addr(lds), ready, avail, wave - kWaves, lane);
    } else {
        const int phase = wave >> c.hw_sh;
        const int npw = c.npw(phase);
        const uint32_t ring = lds_addr(lds) + (uint32_t)(wave * Ring<true>::per_wave);   // this wave's (uniform)
        const uint32_t raw_ring = ring + (uint32_t)(NST * STB);
        const PairLane po = pair_lane_offsets(r, g);
        const LdsLane lo = lds_lane_offsets(r, g);     // the V^T reads of pages with raw V rows
        const VtLane vto = vt_lane_offsets(lane);
        const PairSrc rawp = pair_src((uint64_t)(uintptr_t)ar.k.raw, (uint64_t)(uintptr_t)ar.v.raw);
        const PairSrc rawn = pair_src((uint64_t)ar.k.raw_rows, (uint64_t)ar.v.raw_rows);

        // metadata of both heads of the wavefront's pages: lane i holds page i's (i < 64),
        // loaded once with q by direct-to-LDS loads, then v_readlane per page (scalar loads
        // past 64); the same for the block-table entries of a paged cache
        int32_t vbt = 0;
        auto gpage = [&](int j) -> int64_t {
            const int lp = c.p0 + phase + c.nphase * j;
            int32_t e = 0;
            if (ar.block_table != nullptr)
                e = j < 64 ? __builtin_amdgcn_readlane(vbt, j) : const_ld(ar.block_table + c.b * ar.bt_stride + lp);
            return array_page(a, c, lp, e);
        };
        uint32_t vmk[2] = {0u, 0u}, vmv[2] = {0u, 0u};
        int32_t vok[2] = {0, 0}, vov[2] = {0, 0};
        auto meta = [&](int j) {
            PairMeta m;
            if (j >= 64) {
                const int64_t gp = gpage(j);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int64_t page = gp * ar.Hkv + hk0 + k;
                    m.h[k] = PageMeta{(uint32_t)const_ld(ar.k.rowmask + page), (uint32_t)const_ld(ar.v.rowmask + page),
                                      const_ld(ar.k.rowoff + page), const_ld(ar.v.rowoff + page)};
                }
                return m;
            }
#pragma unroll
            for (int k = 0; k < 2; ++k)
                m.h[k] = PageMeta{(uint32_t)__builtin_amdgcn_readlane((int)vmk[k], j),
                                  (uint32_t)__builtin_amdgcn_readlane((int)vmv[k], j),
                                  __builtin_amdgcn_readlane(vok[k], j), __builtin_amdgcn_readlane(vov[k], j)};
            return m;
        };
        auto issue_raw = [&](int j, const PairMeta& m) {
            dma_pair_raw(lane, m, raw_ring + (uint32_t)((j & 1) * kRawSlot), rawp, rawn);
        };
        // q (4 KiB) and the metadata (2 KiB) through the last stage, which no page uses before
        // the wavefront hands it over (avail = NST below)
        const uint32_t qst = ring + (uint32_t)((NST - 1) * STB);
        const uint32_t mst = qst + 4096u;              // per head (+1024): rowmask K | rowoff K | rowmask V | rowoff V
        const int i_pg = min(lane, max(npw - 1, 0));   // per lane: the wavefront's page i
        if (ar.block_table != nullptr) {               // the block-table entries first: every address needs them
            const uint32_t bst = mst + 2048u;
            dma4(ar.block_table + c.b * ar.bt_stride + min(c.p0 + phase + c.nphase * i_pg, c.NP - 1), bst);
            wait_vm<0>();
            vbt = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(bst + 4u * lane));
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        q_dma_pair(ar, c.b, hk0, c.hg, gh, lane, qst);
        {
            const int64_t gp = ar.block_table == nullptr ? (int64_t)c.b * c.NP + min(c.p0 + phase + c.nphase * i_pg, c.NP - 1)
                                                         : array_page(a, c, 0, vbt);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int64_t page = gp * ar.Hkv + hk0 + k;
                const uint32_t mk = mst + 1024u * k;
                dma4(ar.k.rowmask + page, mk);
                dma4(ar.k.rowoff + page, mk + 256u);
                dma4(ar.v.rowmask + page, mk + 512u);
                dma4(ar.v.rowoff + page, mk + 768u);
            }
        }
        wait_vm<0>();
        bf16x8 qop[4];
        load_qop_pair(qst, r, g, gh, qop);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t mk = mst + 1024u * k + 4u * lane;
            vmk[k] = *reinterpret_cast<const EXKV_LDS uint32_t*>(lds_ptr(mk));
            vok[k] = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(mk + 256u));
            vmv[k] = *reinterpret_cast<const EXKV_LDS uint32_t*>(lds_ptr(mk + 512u));
            vov[k] = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(mk + 768u));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // q and the page table are in registers
        lds_flag_st(&avail[wave], NST);
        if (npw > 0) issue_raw(0, meta(0));
        if (npw > 1) issue_raw(1, meta(1));

        lds_flag_st(&progress[wave], 0);
        int stg = 0;                                   // stage of page j (j % NST)
        for (int j = 0; j < npw; ++j) {
            // page j's raw rows have landed once only page j + 1's are in flight
            if (j + 1 < npw)
                wait_vm_n(pair_raw_loads(meta(j + 1)));
            else
                wait_vm<0>();
            if (lds_flag_ld(&ready[wave]) <= j) {      // page j's bytes: published by the loader
                int s = 0;
                for (; s < a.spin && lds_flag_ld(&ready[wave]) <= j; ++s) __builtin_amdgcn_s_sleep(0);
                if (s == a.spin) report_error(kErrWait);
            }
            asm volatile("" ::: "memory");
            const uint32_t sb = ring + (uint32_t)(stg * STB);
            stg = stg == NST - 1 ? 0 : stg + 1;
            const int t0 = (c.p0 + phase + c.nphase * j) * kPage;
            const bool ragged = t0 + kPage > c.end || t0 < c.wlo;   // uniform: a split's last page, or the window's first
            const bool valid = t0 + r < c.end && t0 + r >= c.wlo;
            const PairMeta mc = meta(j);
            const PairMeta mn = j + NST - 1 < npw ? meta(j + NST - 1) : PairMeta{};
            const int other = lds_flag_ld(&progress[wave ^ 4]);   // the partner's count: a hint, read unsynchronised
            lds_flag_st(&progress[wave], j);

            // every read of the stage up front: V^T by transposing byte reads, K by rows (base
            // bytes through the row broadcast); the stage goes back after the score MFMAs
            VtBytes vb;
            stage_vt_bytes(sb, vto, vb);
            StageSC pk;
            stage_sm_code_pair(sb, po, CS_KSM, CS_KCODE, pk);
            const uint32_t bw = stage_base_word(sb, po.bw);
            balance_priority(j, other);
            const uint32_t slot = raw_ring + (uint32_t)((j & 1) * kRawSlot);
            s16x4 vt[8];
            const uint64_t zf = __ballot((bw & 0x80808080u) != 0u);
            if ((mc.h[0].mv | mc.h[1].mv) == 0u) {
                rebuild_vt<true>(vb, vt);
                if (ragged) {
                    keep_branch();
                    vt_zero_invalid(vt, t0 + 4 * g, c.end, c.wlo);
                }
            } else {                                   // a page with raw V rows (rare): V by token
                keep_branch();                         // rows, its raw rows spliced in, transposed
                PageBytes pv;                          // through a bf16 tile over the K bytes
                stage_bytes_pair(sb, po, CS_VSM, CS_VCODE, CS_BASE + 128, pv);   // (already in registers)
                uint32_t vd[16];
                rebuild_values(pv, vd);
                splice_pair<true>(ar, mc, slot, r, g, vd);
                if (ragged) {
                    keep_branch();
                    zero_invalid_rows(valid, vd);
                }
                write_v_tile_pair(sb, po, Ring<true>::vtile, vd);
                read_vt(sb, lo, Ring<true>::vtile, vt);
            }
            uint32_t kd[16];
            rebuild_values_bc<false>(pk, bw, zf, kd);
            if ((mc.h[0].mk | mc.h[1].mk) != 0u) {
                keep_branch();
                splice_pair<false>(ar, mc, slot, r, g, kd);
            }
            if (ragged) {
                keep_branch();
                zero_invalid_rows(valid, kd);
            }
            f32x4 s0, s1;
            pair_scores(kd, qop, s0, s1);
            // this page's raw rows are out of their slot: page j + 2's go there
            if (j + NST - 1 < npw) issue_raw(j + NST - 1, mn);
            // every LDS read of the stage (bytes, V^T operands) has returned: hand it back
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            lds_flag_st(&avail[wave], j + NST + 1);
            pair_softmax_pv(s0, s1, vt, ragged, t0, c, g, a.qk_scale, m_i, l_i, acc0, acc1);
        }
    }
    pair_epilogue(ar, c, a.HW, lds_addr(lds), Ring<true>::per_wave, done, wave, lane, wave < kWaves, hk0, gh, acc0,
                  acc1, m_i, l_i);
}

// bf16 twin: the structure of attn_split_kernel<false> (8 wavefronts issuing their own pages)
template <>
__global__ void __launch_bounds__(kThreads) attn_pair_kernel<false>(AttnArgs ar) {
    constexpr int NST = Ring<false>::nst, STB = Ring<false>::stage;
    __shared__ __attribute__((aligned(16))) uint8_t lds[Ring<false>::bytes];
    __shared__ int progress[kWaves];
    __shared__ int done[kWaves];                       // page phase p > 0: partials left in the ring
    AttnArgs a = ar;
    a.Hkv = ar.Hkv / 2;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const SplitCoords c = split_coords(a);
    if (threadIdx.x < kWaves) done[threadIdx.x] = 0;
    __syncthreads();
    const int hv = c.hb * a.HW + (wave & (a.HW - 1));
    const int hk0 = 2 * hv;
    const int gh = min(16, ar.G - c.hg * 16);
    const int phase = wave >> c.hw_sh;
    const int npw = c.npw(phase);
    const int64_t rs = a.Hkv;
    float m_i[2] = {-INFINITY, -INFINITY}, l_i[2] = {0.f, 0.f};
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc0[nb] = acc1[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t ring = lds_addr(lds) + (uint32_t)(wave * Ring<false>::per_wave);
    const LdsLane lo = lds_lane_offsets(r, g);
    const PairLane po = pair_lane_offsets(r, g);
    const DmaLane dl = dma_lane_offsets<false>(lane, rs);
    const PairSrc nobase{0ull, 0ull};
    int32_t vbt = 0;
    auto gpage = [&](int j) -> int64_t {
        const int lp = c.p0 + phase + c.nphase * j;
        int32_t e = 0;
        if (ar.block_table != nullptr)
            e = j < 64 ? __builtin_amdgcn_readlane(vbt, j) : const_ld(ar.block_table + c.b * ar.bt_stride + lp);
        return array_page(a, c, lp, e);
    };
    auto issue = [&](int j, uint32_t sb) {
        const int64_t gp = gpage(j);
        dma_page_bytes<false>(a, dl, gp * kPage * rs + hv, gp * rs + hv, sb, lane, nobase);
    };
    // q through the last stage, which no page uses before page NST - 1 is issued
    const uint32_t qst = ring + (uint32_t)((NST - 1) * STB);
    if (ar.block_table != nullptr) {
        const uint32_t bst = qst + 5120u;
        const int i_pg = min(lane, max(npw - 1, 0));
        dma4(ar.block_table + c.b * ar.bt_stride + min(c.p0 + phase + c.nphase * i_pg, c.NP - 1), bst);
        wait_vm<0>();
        vbt = *reinterpret_cast<const EXKV_LDS int32_t*>(lds_ptr(bst + 4u * lane));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    q_dma_pair(ar, c.b, hk0, c.hg, gh, lane, qst);
    if (npw > 0) {
        issue(0, ring);
        wait_vm<kDmaPerPage[0]>();                     // q has landed once only page 0's loads are in flight
    } else {
        wait_vm<0>();
    }
    bf16x8 qop[4];
    load_qop_pair(qst, r, g, gh, qop);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // q is in registers before its stage is reused

    lds_flag_st(&progress[wave], 0);
    int stg = 0;
    for (int j = 0; j < npw; ++j) {
        wait_vm<0>();                                  // page j has landed (the only page in flight)
        const uint32_t sb = ring + (uint32_t)(stg * STB);
        const int stn = stg == 0 ? NST - 1 : stg - 1;  // stage of page j + 1
        stg = stg == NST - 1 ? 0 : stg + 1;
        const int t0 = (c.p0 + phase + c.nphase * j) * kPage;
        const bool ragged = t0 + kPage > c.end || t0 < c.wlo;
        const bool valid = t0 + r < c.end && t0 + r >= c.wlo;
        if (j + NST - 1 < npw) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(j + NST - 1, ring + (uint32_t)(stn * STB));
        }
        const int other = lds_flag_ld(&progress[wave ^ 4]);   // the partner's count: a hint, read unsynchronised
        lds_flag_st(&progress[wave], j);
        uint32_t kd[16];
        stage_bf16_k_pair(sb, po, kd);
        balance_priority(j, other);
        if (ragged) {
            keep_branch();
            zero_invalid_rows(valid, kd);
        }
        f32x4 s0, s1;
        pair_scores(kd, qop, s0, s1);
        if (ragged) {                                  // ragged page: zero the staged V rows past the end
            keep_branch();
            if (!valid) {
                uint32_t vd[16];
                zero_invalid_rows(false, vd);
                write_v_tile(sb, lo, Ring<false>::vtile, vd);
            }
        }
        s16x4 vt[8];
        read_vt(sb, lo, Ring<false>::vtile, vt);
        pair_softmax_pv(s0, s1, vt, ragged, t0, c, g, a.qk_scale, m_i, l_i, acc0, acc1);
    }
    pair_epilogue(ar, c, a.HW, lds_addr(lds), Ring<false>::per_wave, done, wave, lane, true, hk0, gh, acc0, acc1,
                  m_i, l_i);
}

}  // namespace exkv

using namespace exkv;

// KV heads per workgroup: gcd(Hkv, 8), at most 4 (8 wavefronts = head slots x page phases,
// so every head gets at least two phases). At 8 KV heads four per workgroup halves the
// partials a call merges and is never slower: measured (split kernel / call, 8 against 4
// heads per workgroup) c2a 40.5 / 44.7 against 40.5 / 44.2 us, c2a with a partial last
// page 41.8 / 46.0 against 41.7 / 45.3, B1 x 128K 77.3 / 79.8 against 75.6 / 79.0, B32 x
// 4096 77.6 / 79.7 against 77-80 / 79-80, B128 x 4352 302.8 / 307.9 against 301.6 / 305.8.
static int heads_per_block(int Hkv) {
    int a = Hkv, b = kWaves;
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a < 4 ? a : 4;
}

// Head dim 64 with an even number of KV heads runs as pairs of heads (attn_pair_kernel);
// odd counts and head dim 256 run attn_dgen_kernel.
static bool pair_heads(int D, int Hkv) { return D == 64 && Hkv % 2 == 0; }

// KV heads (virtual heads of two, for pairs) per workgroup of the split kernels
static int block_heads(int D, int Hkv) { return pair_heads(D, Hkv) ? heads_per_block(Hkv / 2) : heads_per_block(Hkv); }

// Workgroup units (sequence, head block, query group) of the split kernels' 2-D grid
static int64_t grid_units(int B, int Hq, int Hkv, int D) {
    const int64_t hg = (Hq / Hkv + 15) / 16;
    if (D == kD) return (int64_t)B * (Hkv / block_heads(D, Hkv)) * hg;
    if (pair_heads(D, Hkv)) return (int64_t)B * (Hkv / 2 / block_heads(D, Hkv)) * hg;
    return (int64_t)B * Hkv * hg;                      // the generic kernel's one-dimensional units
}

// One launch: one split (the split kernel writes the output), or the merge in the split
// kernel's tail (head dim 128, with arrival counters)
static bool one_launch(int D, int Hkv, int nsplit, const int32_t* ws_cnt) {
    if (D == kD) return nsplit == 1 || (ws_cnt && nsplit <= kFusedMaxSplits);
    return pair_heads(D, Hkv) && nsplit == 1;
}

static int check_attn(int B, int Hq, int Hkv, int D, int T, int TS, const int32_t* lens, int nsplit,
                      int split_len, int window) {
    EXKV_REQUIRE(head_dim_ok(D), "attention: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "attention: bad heads Hq=%d Hkv=%d (B=%d)", Hq,
                 Hkv, B);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0, "attention: TS=%d must be a positive multiple of 16", TS);
    EXKV_REQUIRE(nsplit > 0 && split_len > 0 && split_len % kPage == 0,
                 "attention: split_len=%d must be a positive multiple of 16 (nsplit=%d)", split_len, nsplit);
    EXKV_REQUIRE(window >= 0, "attention: negative window %d", window);
    // a sequence's splits cover [lo's page, len): at most window + 15 tokens with a window
    const int64_t reach = window > 0 ? (int64_t)window + kPage - 1 : INT64_MAX;
    if (lens == nullptr) {
        EXKV_REQUIRE(T >= 1 && T <= TS, "attention: T=%d outside [1, TS=%d]", T, TS);
        EXKV_REQUIRE((int64_t)nsplit * split_len >= min((int64_t)T, reach),
                     "attention: %d splits of %d do not cover T=%d (window %d)", nsplit, split_len, T, window);
    } else {
        EXKV_REQUIRE((int64_t)nsplit * split_len >= min((int64_t)TS, reach),
                     "attention: with per-sequence lengths the splits must cover TS=%d (window %d)", TS, window);
    }
    EXKV_REQUIRE(grid_units(B, Hq, Hkv, D) < 65536, "attention: too many (sequence, head block) units");
    // a launch's grid is 32-bit in work-items: x = splits (head dim 128 and pairs of head-dim-64
    // heads; the compressed kernel's workgroups are the larger) or every workgroup (the
    // one-dimensional grid of the generic kernel, DGen<D, *>::NPH wavefronts each)
    const bool two_d = D == kD || pair_heads(D, Hkv);
    const int64_t wg_x = two_d ? (int64_t)nsplit : (int64_t)nsplit * grid_units(B, Hq, Hkv, D);
    const int64_t wg_threads = two_d ? kCompThreads : 64 * (D >= 256 ? 2 : 4);
    EXKV_REQUIRE(wg_x * wg_threads <= (int64_t)UINT32_MAX, "attention: too many workgroups (%d splits)", nsplit);
    return EXKV_OK;
}

// Timing hook: events that the next split-kernel launch on this thread records at its start
// and end (hipExtLaunchKernelGGL), consumed by that launch.
static thread_local hipEvent_t t_split_start = nullptr, t_split_stop = nullptr;

// Test hook: the bound of the split kernels' flag waits for launches on this thread.
static thread_local int t_wait_limit = kSpinMax;

template <int D>
static void launch_dgen(bool comp, const AttnArgs& a, hipEvent_t e0, hipEvent_t e1, hipStream_t stream) {
    // one-dimensional: the kernel orders (sequence, split, head group, KV head) itself
    const dim3 grid((unsigned)((int64_t)a.nsplit * a.B * a.Hkv * a.HG)), block(64 * DGen<D, true>::NPH);
    auto k = comp ? attn_dgen_kernel<D, true> : attn_dgen_kernel<D, false>;
    if (e0 || e1)
        hipExtLaunchKernelGGL(k, grid, block, 0, stream, e0, e1, 0, a);
    else
        hipLaunchKernelGGL(k, grid, block, 0, stream, a);
}

static int launch_split(bool comp, const AttnArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)a.nsplit, (unsigned)(a.B * (a.Hkv / a.HW) * a.HG));
    hipEvent_t e0 = t_split_start, e1 = t_split_stop;
    t_split_start = t_split_stop = nullptr;
    if (pair_heads(a.D, a.Hkv)) {
        const dim3 pgrid((unsigned)a.nsplit, (unsigned)(a.B * (a.Hkv / 2 / a.HW) * a.HG));
        auto k = comp ? attn_pair_kernel<true> : attn_pair_kernel<false>;
        const dim3 block(comp ? kCompThreads : kThreads);
        if (e0 || e1)
            hipExtLaunchKernelGGL(k, pgrid, block, 0, stream, e0, e1, 0, a);
        else
            hipLaunchKernelGGL(k, pgrid, block, 0, stream, a);
        return hip_status(hipGetLastError(), comp ? "attn_split_compressed" : "attn_split_bf16");
    }
    if (a.D != kD) {
        if (a.D == 64)
            launch_dgen<64>(comp, a, e0, e1, stream);
        else
            launch_dgen<256>(comp, a, e0, e1, stream);
        return hip_status(hipGetLastError(), comp ? "attn_split_compressed" : "attn_split_bf16");
    }
    if (e0 || e1) {
        if (comp)
            hipExtLaunchKernelGGL(attn_split_kernel<true>, grid, dim3(kCompThreads), 0, stream, e0, e1, 0, a);
        else
            hipExtLaunchKernelGGL(attn_split_kernel<false>, grid, dim3(kThreads), 0, stream, e0, e1, 0, a);
    } else if (comp) {
        hipLaunchKernelGGL(attn_split_kernel<true>, grid, dim3(kCompThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL(attn_split_kernel<false>, grid, dim3(kThreads), 0, stream, a);
    }
    return hip_status(hipGetLastError(), comp ? "attn_split_compressed" : "attn_split_bf16");
}

extern "C" int64_t exkv_merge_counters(int32_t B, int32_t Hq, int32_t Hkv, int32_t nsplit) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || nsplit <= 0 || nsplit > kFusedMaxSplits) return -1;
    const int64_t units = (int64_t)B * (Hkv / heads_per_block(Hkv)) * ((Hq / Hkv + 15) / 16);
    return units * (merge_groups(nsplit) + 1);
}

extern "C" int exkv_set_wait_limit(int32_t polls) {
    t_wait_limit = polls > 0 ? polls : kSpinMax;
    return EXKV_OK;
}

namespace exkv {
hipError_t fetch_errors_attention(uint32_t* out, int first, int clear, hipStream_t stream) {
    return fetch_file_errors(out, first, clear, stream);
}
}  // namespace exkv

extern "C" int exkv_time_next_split(hipEvent_t start, hipEvent_t stop) {
    t_split_start = start;
    t_split_stop = stop;
    return EXKV_OK;
}

static int launch_reduce(const float* o, const float* m, const float* l, void* out, int64_t rows, int ns, int D,
                         hipStream_t stream) {
    if (D == 64)
        hipLaunchKernelGGL(attn_reduce_d_kernel<64>, dim3((unsigned)rows), dim3(64), 0, stream, o, m, l, (uint16_t*)out, ns);
    else if (D == 256)
        hipLaunchKernelGGL(attn_reduce_d_kernel<256>, dim3((unsigned)rows), dim3(64), 0, stream, o, m, l, (uint16_t*)out, ns);
    else if (ns <= 32)
        hipLaunchKernelGGL(attn_reduce_kernel, dim3((unsigned)rows), dim3(64), 0, stream, o, m, l, (uint16_t*)out, ns);
    else
        hipLaunchKernelGGL(attn_reduce_wide_kernel, dim3((unsigned)rows, kD / kWideChunk), dim3(64 * kWideWaves), 0,
                           stream, o, m, l, (uint16_t*)out, ns);
    return hip_status(hipGetLastError(), "attn_reduce");
}

static int fill_compressed(AttnArgs& a, const void* q, const void* k_sm, const void* k_code, const void* k_base,
                           const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw, int64_t k_raw_rows,
                           const void* v_sm, const void* v_code, const void* v_base, const int32_t* v_rowmask,
                           const int32_t* v_rowoff, const void* v_raw, int64_t v_raw_rows, float* ws_o,
                           float* ws_m, float* ws_l, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T,
                           int32_t TS, const int32_t* lens, int64_t lens_stride, int32_t nsplit,
                           int32_t split_len, int32_t window, float qk_scale) {
    const int rc = check_attn(B, Hq, Hkv, D, T, TS, lens, nsplit, split_len, window);
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
    a.nsplit = nsplit; a.split_len = split_len; a.window = window; a.qk_scale = qk_scale;
    a.HW = block_heads(D, Hkv);
    a.D = D;
    a.spin = t_wait_limit;
    return EXKV_OK;
}

static int fill_bf16(AttnArgs& a, const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                     float* ws_l, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                     const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len, int32_t window,
                     float qk_scale) {
    const int rc = check_attn(B, Hq, Hkv, D, T, TS, lens, nsplit, split_len, window);
    if (rc) return rc;
    EXKV_REQUIRE(q && k && v && ws_o && ws_m && ws_l, "attn_bf16: null pointer");
    a = AttnArgs{};
    a.q = (const uint16_t*)q;
    a.kb = (const uint16_t*)k; a.vb = (const uint16_t*)v;
    a.part_o = ws_o; a.part_m = ws_m; a.part_l = ws_l;
    a.lens = lens; a.lens_stride = lens_stride;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.HG = (a.G + 15) / 16; a.TS = TS; a.T = T;
    a.nsplit = nsplit; a.split_len = split_len; a.window = window; a.qk_scale = qk_scale;
    a.HW = block_heads(D, Hkv);
    a.D = D;
    a.spin = t_wait_limit;
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
        int32_t nsplit, int32_t split_len, int32_t window, float qk_scale
#define EXKV_SHAPE_ARGS B, Hq, Hkv, D, T, TS, lens, lens_stride, nsplit, split_len, window, qk_scale

extern "C" int exkv_attn_compressed(EXKV_C_PARAMS, int32_t* ws_cnt, void* out, EXKV_SHAPE_PARAMS,
                                    hipStream_t stream) {
    AttnArgs a;
    int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_compressed: null output");
    if (one_launch(D, Hkv, nsplit, ws_cnt)) {
        // one launch: one split (the output directly), or the merge in the split kernel's tail
        a.out = (uint16_t*)out;
        a.counters = nsplit > 1 ? ws_cnt : nullptr;
        return launch_split(true, a, stream);
    }
    rc = launch_split(true, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, D, stream);
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
    if (one_launch(D, Hkv, nsplit, ws_cnt)) {
        // one launch: one split (the output directly), or the merge in the split kernel's tail
        a.out = (uint16_t*)out;
        a.counters = nsplit > 1 ? ws_cnt : nullptr;
        return launch_split(false, a, stream);
    }
    rc = launch_split(false, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, D, stream);
}

extern "C" int exkv_attn_split_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                                    float* ws_l, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    const int rc = fill_bf16(a, q, k, v, ws_o, ws_m, ws_l, EXKV_SHAPE_ARGS);
    return rc ? rc : launch_split(false, a, stream);
}

// Paged caches: the compressed (or bf16) arrays hold pool_pages pages of 16 tokens (shape
// [1, 16 * pool_pages, Hkv, ...]); page p of sequence b is pool page block_table[b *
// bt_stride + p] (entries clamped to the pool). TS is the sequences' capacity in tokens
// (at most 16 * bt_stride).
static int set_paged(AttnArgs& a, const int32_t* block_table, int64_t bt_stride, int32_t pool_pages, int32_t TS) {
    EXKV_REQUIRE(block_table, "attention (paged): null block table");
    EXKV_REQUIRE(pool_pages > 0, "attention (paged): pool_pages=%d", pool_pages);
    EXKV_REQUIRE(bt_stride > 0 && (int64_t)TS <= 16 * bt_stride,
                 "attention (paged): TS=%d exceeds the block table's %lld pages", TS, (long long)bt_stride);
    a.block_table = block_table;
    a.bt_stride = bt_stride;
    a.pool_pages = pool_pages;
    return EXKV_OK;
}

extern "C" int exkv_attn_compressed_paged(EXKV_C_PARAMS, int32_t* ws_cnt, void* out, const int32_t* block_table,
                                          int64_t bt_stride, int32_t pool_pages, EXKV_SHAPE_PARAMS,
                                          hipStream_t stream) {
    AttnArgs a;
    int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    if (!rc) rc = set_paged(a, block_table, bt_stride, pool_pages, TS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_compressed_paged: null output");
    if (one_launch(D, Hkv, nsplit, ws_cnt)) {
        // one launch: one split (the output directly), or the merge in the split kernel's tail
        a.out = (uint16_t*)out;
        a.counters = nsplit > 1 ? ws_cnt : nullptr;
        return launch_split(true, a, stream);
    }
    rc = launch_split(true, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, D, stream);
}

extern "C" int exkv_attn_split_compressed_paged(EXKV_C_PARAMS, const int32_t* block_table, int64_t bt_stride,
                                                int32_t pool_pages, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    if (!rc) rc = set_paged(a, block_table, bt_stride, pool_pages, TS);
    return rc ? rc : launch_split(true, a, stream);
}

extern "C" int exkv_attn_bf16_paged(const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                                    float* ws_l, int32_t* ws_cnt, void* out, const int32_t* block_table,
                                    int64_t bt_stride, int32_t pool_pages, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    int rc = fill_bf16(a, q, k, v, ws_o, ws_m, ws_l, EXKV_SHAPE_ARGS);
    if (!rc) rc = set_paged(a, block_table, bt_stride, pool_pages, TS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_bf16_paged: null output");
    if (one_launch(D, Hkv, nsplit, ws_cnt)) {
        // one launch: one split (the output directly), or the merge in the split kernel's tail
        a.out = (uint16_t*)out;
        a.counters = nsplit > 1 ? ws_cnt : nullptr;
        return launch_split(false, a, stream);
    }
    rc = launch_split(false, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, D, stream);
}

extern "C" int exkv_attn_reduce(const float* ws_o, const float* ws_m, const float* ws_l, void* out, int64_t rows,
                                int32_t nsplit, int32_t D, hipStream_t stream) {
    EXKV_REQUIRE(head_dim_ok(D), "attn_reduce: head dim must be 64, 128 or 256 (got %d)", D);
    EXKV_REQUIRE(rows > 0 && nsplit > 0, "attn_reduce: bad rows=%lld nsplit=%d", (long long)rows, nsplit);
    EXKV_REQUIRE(ws_o && ws_m && ws_l && out, "attn_reduce: null pointer");
    return launch_reduce(ws_o, ws_m, ws_l, out, rows, nsplit, D, stream);
}
