// Page loader and bit-exact rebuild shared by decode attention and decode_to_bf16.
//
// First the head-dim-128 forms (the row rebuild that pages with raw V rows take in the
// head-dim-64 pair kernel, raw-row slots and loads), then templates for every head dim
// (decode_to_bf16 and the generic-head-dim kernel).
// Lane layout (one wavefront of 64 lanes covers one 16-token page of one KV head):
//   r = lane % 16   token within the page
//   g = lane / 16   channel group: channels [16g, 16g+16) and [64+16g, 64+16g+16)
// With this split a lane's 16 code bytes (channels 16g..16g+15) carry the codes of both
// of its channel runs (low and high nibbles), so every load is a 16-byte vector.
// Output: 16 dwords of bf16 pairs; out[0..7] = channels 16g.., out[8..15] = 64+16g..
// This is also the A-operand layout of v_mfma_f32_16x16x32_bf16 with tokens as rows:
// k-block kc of the MFMA takes out[4kc .. 4kc+3].
#pragma once

#include "common.hpp"
#include "errors.hpp"

namespace exkv {

struct CSrc {                 // one compressed cache (reference cache.py:24-32)
    const uint8_t* sm;        // [B, TS, H, D]
    const uint8_t* code;      // [B, TS, H, D/2]
    const uint8_t* base;      // [B, TS/16, H, D]
    const int32_t* rowmask;   // [B, TS/16, H]
    const int32_t* rowoff;    // [B, TS/16, H]
    const uint16_t* raw;      // [raw_rows, D] bf16
    int64_t raw_rows;
};

struct PageBytes {
    uint4 sm_lo, sm_hi, code, b_lo, b_hi;
    int32_t rmask, roff;
};

__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// One of the lane's two channel runs: 16 values from four dwords of sm, code and base bytes
// (codes in the low nibbles for the run 16g.., high nibbles for 64+16g..).
template <bool Z, bool HIGH>
__device__ inline void rebuild_run(const uint4& sm, const uint4& code, const uint4& base, uint32_t out[8]) {
    const uint32_t S[4] = {sm.x, sm.y, sm.z, sm.w};
    const uint32_t C[4] = {code.x, code.y, code.z, code.w};
    const uint32_t B[4] = {base.x, base.y, base.z, base.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t cn = (HIGH ? C[i] >> 4 : C[i]) & 0x0F0F0F0Fu;
        rebuild4<Z>(S[i], cn, B[i], out[2 * i], out[2 * i + 1]);
    }
}

// Rebuild the lane's 32 values. The zero-group fix-up runs per channel run (channels 0-63
// and 64-127 of the page) and only when some group of that run carries the zero flag,
// decided for the whole wavefront (a page flags a run far less often than it flags one of
// its two runs).
__device__ inline void rebuild_values(const PageBytes& pb, uint32_t out[16]) {
    const uint32_t flo = (pb.b_lo.x | pb.b_lo.y | pb.b_lo.z | pb.b_lo.w) & 0x80808080u;
    const uint32_t fhi = (pb.b_hi.x | pb.b_hi.y | pb.b_hi.z | pb.b_hi.w) & 0x80808080u;
    if (__ballot(flo != 0) != 0)
        rebuild_run<true, false>(pb.sm_lo, pb.code, pb.b_lo, out);
    else
        rebuild_run<false, false>(pb.sm_lo, pb.code, pb.b_lo, out);
    if (__ballot(fhi != 0) != 0)
        rebuild_run<true, true>(pb.sm_hi, pb.code, pb.b_hi, out + 8);
    else
        rebuild_run<false, true>(pb.sm_hi, pb.code, pb.b_hi, out + 8);
}

// Slot of token r's raw row: rowoff + popcount(rowmask & ((1 << r) - 1)) (reference
// kernels.py:119-123), clamped to the pool so that a page whose metadata is broken (say,
// read before the host repaired an overflow) cannot read out of bounds; a clamp of a row
// that token r really has is reported (kErrRawSlot).
// raw_slot_checked: the same with the report as a flag (host-callable, for the CPU build's
// test): bad is set when token r has a raw row and its slot had to be clamped.
__host__ __device__ inline int64_t raw_slot_checked(uint32_t rmask, int32_t roff, int r, int64_t raw_rows,
                                                    bool& bad) {
    const int64_t slot = clamp_slot((int64_t)roff + __builtin_popcount(rmask & ((1u << r) - 1u)), raw_rows, bad);
    bad = bad && ((rmask >> r) & 1u);
    return slot;
}
__device__ inline int64_t raw_slot(uint32_t rmask, int32_t roff, int r, int64_t raw_rows) {
    bool bad;
    const int64_t slot = raw_slot_checked(rmask, roff, r, raw_rows, bad);
    if (bad) report_error(kErrRawSlot);
    return slot;
}

// The lane's 32 values of a raw row (channels 16g.. and 64+16g..).
__device__ inline void load_raw_values(const uint16_t* raw, int64_t slot, int g, uint32_t out[16]) {
    const uint8_t* rp = reinterpret_cast<const uint8_t*>(raw + slot * 128) + 32 * g;
    const uint4 a0 = ld16(rp), a1 = ld16(rp + 16), h0 = ld16(rp + 128), h1 = ld16(rp + 144);
    out[0] = a0.x; out[1] = a0.y; out[2] = a0.z; out[3] = a0.w;
    out[4] = a1.x; out[5] = a1.y; out[6] = a1.z; out[7] = a1.w;
    out[8] = h0.x; out[9] = h0.y; out[10] = h0.z; out[11] = h0.w;
    out[12] = h1.x; out[13] = h1.y; out[14] = h1.z; out[15] = h1.w;
}

// ---------------------------------------------------------------- any head dim D
//
// The same lane layout for D = 64, 128 or 256: lane (r = token, g = lane / 16) holds the
// channel runs [g R, g R + R) and [D/2 + g R, D/2 + g R + R), R = D / 8, whose codes share
// the R code bytes g R .. (low and high nibbles). Values: D / 8 dwords of bf16 pairs, the
// low run first; k-block kc of the score MFMAs takes dwords 4kc .. 4kc + 3.
template <int D>
struct Run {
    static_assert(D == 64 || D == 128 || D == 256, "head dim 64, 128 or 256");
    static constexpr int R = D / 8;        // channels per run
    static constexpr int W = R / 4;        // dwords of bytes per run
    static constexpr int V = D / 8;        // dwords of values per lane (two runs)
};

// n dwords from p (8- or 16-byte aligned for n = 2, n >= 4)
template <int N>
__device__ inline void ld_words(const void* p, uint32_t* out) {
    if constexpr (N == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        out[0] = v.x; out[1] = v.y;
    } else {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const uint4 v = reinterpret_cast<const uint4*>(p)[i];
            out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
        }
    }
}
template <int N>
__device__ inline void st_words(void* p, const uint32_t* in) {
    if constexpr (N == 2) {
        *reinterpret_cast<uint2*>(p) = make_uint2(in[0], in[1]);
    } else {
#pragma unroll
        for (int i = 0; i < N / 4; ++i)
            reinterpret_cast<uint4*>(p)[i] = make_uint4(in[4 * i], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]);
    }
}

template <int D>
struct PageBytesD {
    uint32_t sm_lo[Run<D>::W], sm_hi[Run<D>::W], code[Run<D>::W], b_lo[Run<D>::W], b_hi[Run<D>::W];
};

// row: the lane's token row ((page * 16 + r) * H + h in the arrays); page: page * H + h.
template <int D>
__device__ inline void load_page_d(const CSrc& c, int64_t row, int64_t page, int g, PageBytesD<D>& pb) {
    constexpr int R = Run<D>::R, W = Run<D>::W;
    const uint8_t* s = c.sm + row * D + g * R;
    ld_words<W>(s, pb.sm_lo);
    ld_words<W>(s + D / 2, pb.sm_hi);
    ld_words<W>(c.code + row * (D / 2) + g * R, pb.code);
    const uint8_t* bp = c.base + page * D + g * R;
    ld_words<W>(bp, pb.b_lo);
    ld_words<W>(bp + D / 2, pb.b_hi);
}

template <int D, bool Z, bool HIGH>
__device__ inline void rebuild_run_d(const uint32_t* sm, const uint32_t* code, const uint32_t* base, uint32_t* out) {
#pragma unroll
    for (int i = 0; i < Run<D>::W; ++i) {
        const uint32_t cn = (HIGH ? code[i] >> 4 : code[i]) & 0x0F0F0F0Fu;
        rebuild4<Z>(sm[i], cn, base[i], out[2 * i], out[2 * i + 1]);
    }
}

// The lane's D / 4 values; the zero-group fix-up per run, decided for the wavefront.
template <int D>
__device__ inline void rebuild_values_d(const PageBytesD<D>& pb, uint32_t (&out)[Run<D>::V]) {
    constexpr int W = Run<D>::W;
    uint32_t flo = 0, fhi = 0;
#pragma unroll
    for (int i = 0; i < W; ++i) {
        flo |= pb.b_lo[i];
        fhi |= pb.b_hi[i];
    }
    if (__ballot((flo & 0x80808080u) != 0) != 0)
        rebuild_run_d<D, true, false>(pb.sm_lo, pb.code, pb.b_lo, out);
    else
        rebuild_run_d<D, false, false>(pb.sm_lo, pb.code, pb.b_lo, out);
    if (__ballot((fhi & 0x80808080u) != 0) != 0)
        rebuild_run_d<D, true, true>(pb.sm_hi, pb.code, pb.b_hi, out + 2 * W);
    else
        rebuild_run_d<D, false, true>(pb.sm_hi, pb.code, pb.b_hi, out + 2 * W);
}

// The lane's values of a bf16 row of D channels (a raw row, or a row of the bf16 twin).
template <int D>
__device__ inline void load_row_values_d(const uint16_t* rowp, int g, uint32_t (&out)[Run<D>::V]) {
    constexpr int R = Run<D>::R;
    ld_words<R / 2>(rowp + g * R, out);
    ld_words<R / 2>(rowp + D / 2 + g * R, out + R / 2);
}

// Rebuild one page row of D channels, raw rows spliced in from the pool.
template <int D>
__device__ inline void rebuild_page_d(const CSrc& c, const PageBytesD<D>& pb, uint32_t rmask, int32_t roff, int r,
                                      int g, uint32_t (&out)[Run<D>::V]) {
    rebuild_values_d<D>(pb, out);
    if (rmask != 0 && ((rmask >> r) & 1u))
        load_row_values_d<D>(c.raw + raw_slot(rmask, roff, r, c.raw_rows) * D, g, out);
}

}  // namespace exkv
