// Page loader and bit-exact rebuild shared by decode attention and decode_to_bf16.
//
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

namespace exkv {

struct CSrc {                 // one compressed cache (reference cache.py:24-32)
    const uint8_t* sm;        // [B, TS, H, 128]
    const uint8_t* code;      // [B, TS, H, 64]
    const uint8_t* base;      // [B, TS/16, H, 128]
    const int32_t* rowmask;   // [B, TS/16, H]
    const int32_t* rowoff;    // [B, TS/16, H]
    const uint16_t* raw;      // [raw_rows, 128] bf16
    int64_t raw_rows;
};

struct PageBytes {
    uint4 sm_lo, sm_hi, code, b_lo, b_hi;
    int32_t rmask, roff;
};

__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// row: this lane's token row index ((b*TS + t)*H + hk); page: ((b*NP + pg)*H + hk).
__device__ inline void load_page(const CSrc& c, int64_t row, int64_t page, int g, PageBytes& pb) {
    const uint8_t* s = c.sm + row * 128 + 16 * g;
    pb.sm_lo = ld16(s);
    pb.sm_hi = ld16(s + 64);
    pb.code = ld16(c.code + row * 64 + 16 * g);
    const uint8_t* bp = c.base + page * 128 + 16 * g;
    pb.b_lo = ld16(bp);
    pb.b_hi = ld16(bp + 64);
    pb.rmask = c.rowmask[page];
    pb.roff = c.rowoff[page];
}

template <bool Z>
__device__ inline void rebuild_page_impl(const PageBytes& pb, uint32_t out[16]) {
    const uint32_t S[4] = {pb.sm_lo.x, pb.sm_lo.y, pb.sm_lo.z, pb.sm_lo.w};
    const uint32_t SH[4] = {pb.sm_hi.x, pb.sm_hi.y, pb.sm_hi.z, pb.sm_hi.w};
    const uint32_t C[4] = {pb.code.x, pb.code.y, pb.code.z, pb.code.w};
    const uint32_t BL[4] = {pb.b_lo.x, pb.b_lo.y, pb.b_lo.z, pb.b_lo.w};
    const uint32_t BH[4] = {pb.b_hi.x, pb.b_hi.y, pb.b_hi.z, pb.b_hi.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t cl = C[i] & 0x0F0F0F0Fu;
        const uint32_t ch = (C[i] >> 4) & 0x0F0F0F0Fu;
        if (Z) {
            rebuild4<true>(S[i], cl, BL[i] & 0x7F7F7F7Fu, BL[i] & 0x80808080u, out[2 * i], out[2 * i + 1]);
            rebuild4<true>(SH[i], ch, BH[i] & 0x7F7F7F7Fu, BH[i] & 0x80808080u, out[8 + 2 * i], out[8 + 2 * i + 1]);
        } else {                               // no zero flag in the page: base bytes are < 128
            rebuild4<false>(S[i], cl, BL[i], 0u, out[2 * i], out[2 * i + 1]);
            rebuild4<false>(SH[i], ch, BH[i], 0u, out[8 + 2 * i], out[8 + 2 * i + 1]);
        }
    }
}

// Rebuild the lane's 32 values (the zero-group fix-up only when a group of this page
// carries the zero flag, decided for the whole wavefront).
__device__ inline void rebuild_values(const PageBytes& pb, uint32_t out[16]) {
    const uint32_t fl = (pb.b_lo.x | pb.b_lo.y | pb.b_lo.z | pb.b_lo.w | pb.b_hi.x | pb.b_hi.y |
                         pb.b_hi.z | pb.b_hi.w) & 0x80808080u;
    if (__ballot(fl != 0) != 0) {             // any zero-flagged group in this page
        rebuild_page_impl<true>(pb, out);
    } else {
        rebuild_page_impl<false>(pb, out);
    }
}

// Slot of token r's raw row: rowoff + popcount(rowmask & ((1 << r) - 1)) (reference
// kernels.py:119-123), clamped to the pool so that a page whose raw rows did not fit
// (the pool counter passed its capacity, which the host repairs by growing and
// re-encoding) cannot read out of bounds.
__device__ inline int64_t raw_slot(uint32_t rmask, int32_t roff, int r, int64_t raw_rows) {
    int64_t slot = (int64_t)roff + popc32(rmask & ((1u << r) - 1u));
    return slot < 0 ? 0 : (slot >= raw_rows ? raw_rows - 1 : slot);
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

// Rebuild, then splice raw rows straight from the pool (reference kernels.py:106-128).
__device__ inline void rebuild_page(const CSrc& c, const PageBytes& pb, int r, int g, uint32_t out[16]) {
    rebuild_values(pb, out);
    if (pb.rmask != 0) {
        const uint32_t m = (uint32_t)pb.rmask;
        if ((m >> r) & 1u) load_raw_values(c.raw, raw_slot(m, pb.roff, r, c.raw_rows), g, out);
    }
}

// Uncompressed twin: the same 32 values straight from a bf16 [B, TS, H, 128] buffer.
__device__ inline void load_bf16_row(const uint16_t* buf, int64_t row, int g, uint32_t out[16]) {
    const uint8_t* p = reinterpret_cast<const uint8_t*>(buf + row * 128) + 32 * g;
    const uint4 a0 = ld16(p), a1 = ld16(p + 16), h0 = ld16(p + 128), h1 = ld16(p + 144);
    out[0] = a0.x; out[1] = a0.y; out[2] = a0.z; out[3] = a0.w;
    out[4] = a1.x; out[5] = a1.y; out[6] = a1.z; out[7] = a1.w;
    out[8] = h0.x; out[9] = h0.y; out[10] = h0.z; out[11] = h0.w;
    out[12] = h1.x; out[13] = h1.y; out[14] = h1.z; out[15] = h1.w;
}

}  // namespace exkv
