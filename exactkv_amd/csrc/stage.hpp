// The compressed page stage of the head-dim-128 split kernels (and of the head-dim-64 pair
// kernels, whose virtual heads have the same byte layout): where the loader wavefronts'
// direct-to-LDS loads place a page's bytes, the per-lane offsets and arithmetic that
// rebuild V straight into the P.V operand layout from transposing byte reads, and those
// that rebuild K rows (and the V rows of pages with raw V rows) from row reads. Plain
// arithmetic, compiled for the host as well, so that a CPU program can build a stage the
// way the loads do and check the layout against the format rule.
//
// V^T from transposing byte reads: ds_read_b64_tr_b8 (gfx950): in each 16-lane group,
// lane L reads 8 bytes; lanes 2k and 2k + 1 form row k (16 bytes) of an 8 x 16 byte matrix,
// and lane i receives byte i of rows 0..7. The P.V MFMA's A operand for channel block nb is
// V^T: lane (i = lane & 15, kb = lane >> 4) holds V[4kb + j][16nb + i], j = 0..3. With rows
// 0-3 = tokens 4kb .. 4kb + 3 of one 16-byte segment and rows 4-7 = the same tokens of
// another, one read gives a lane the sign|mantissa bytes of its 4 tokens in blocks nb and
// nb + 4 (segments nb and nb + 4 of the sm rows), one the code bytes of two blocks (code
// byte j holds channel j in its low nibble and j + 64 in its high one, so they serve
// blocks + 4 too), and one read of the base row (row k = bytes 16k .. 16k + 15) the lane's
// base byte of all 8 blocks. The rebuild then yields the A operand itself: V makes no bf16
// round trip through LDS.
#pragma once

#include "common.hpp"

namespace exkv {

typedef short s16x4 __attribute__((ext_vector_type(4)));

// compressed page stage (bytes): K sm 16x128 | K code 16x64 | V sm | V code | K base,
// V base (128 each); rowmask/rowoff of the wavefront's pages are loaded once, up front
constexpr int CS_KSM = 0, CS_KCODE = 2048, CS_VSM = 3072, CS_VCODE = 5120, CS_BASE = 6144, CS_BYTES = 6400;
// bf16 page stage: K rows 16x256 | V rows 16x256
constexpr int BS_K = 0, BS_V = 4096, BS_BYTES = 8192;

// Per-lane parts of a page's DMA addresses (fixed for the kernel): byte offsets from the
// page's first row in each array, with the XOR swizzle of the destination applied.
struct DmaLane {
    uint32_t sm0, sm1, code, base, bf_k[4], bf_v[4];
};

template <bool COMP>
__host__ __device__ inline DmaLane dma_lane_offsets(int lane, int64_t rs) {
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

struct VtLane {
    uint32_t sm[4], code[2], base;     // stage offsets of the lane's 8-byte reads
};
__host__ __device__ inline VtLane vt_lane_offsets(int lane) {
    const int L = lane & 15, kb = lane >> 4, k = L >> 1, h = L & 1;
    const int t = 4 * kb + (k & 3);                    // token of the lane's row
    VtLane o;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {                   // sm: segments nb (rows 0-3), nb + 4 (rows 4-7)
        const int s = nb + 4 * (k >> 2);
        o.sm[nb] = (uint32_t)(CS_VSM + t * 128 + 16 * (s ^ (t & 7)) + 8 * h);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {                      // code: segments 2c (rows 0-3), 2c + 1 (rows 4-7)
        const int s = 2 * c + (k >> 2);
        o.code[c] = (uint32_t)(CS_VCODE + t * 64 + 16 * (s ^ ((t >> 1) & 3)) + 8 * h);
    }
    o.base = (uint32_t)(CS_BASE + 128 + 16 * k + 8 * h);
    return o;
}
struct VtBytes {
    uint32_t sm[8], code[4], base[2];  // sm[nb], code[nb & 3], base[nb >> 2] byte nb & 3
};

// PAIR: a pair of head-dim-64 heads as one 128-channel virtual head (attn_pair_kernel). Its
// code row is the two heads' 32-byte rows, byte j holding channels j (low nibble) and j + 32
// (high) of its head, so block nb's codes are in segment (nb & 1) | ((nb >> 1) & 2), high
// nibbles when nb & 2; with one head of 128 channels, segment nb & 3, high when nb >= 4.
template <bool Z, int NB, bool PAIR>
__host__ __device__ __forceinline__ void rebuild_vt_block(const VtBytes& vb, s16x4& out) {
    constexpr int SEG = PAIR ? ((NB & 1) | ((NB >> 1) & 2)) : (NB & 3);
    constexpr bool HIGH = PAIR ? ((NB & 2) != 0) : (NB >= 4);
    const uint32_t cd = vb.code[SEG];
    const uint32_t cn = (HIGH ? cd >> 4 : cd) & 0x0F0F0F0Fu;
    const uint32_t b4 = perm_b32(vb.base[NB >> 2], vb.base[NB >> 2], (NB & 3) * 0x01010101u);
    uint32_t o01, o23;
    bf16_pairs(vb.sm[NB], Z ? exponents(cn, b4) : cn + b4, o01, o23);
    out = __builtin_bit_cast(s16x4, make_uint2(o01, o23));
}
template <bool Z, int NB0, bool PAIR>
__host__ __device__ __forceinline__ void rebuild_vt_run(const VtBytes& vb, s16x4 (&vt)[8]) {
    rebuild_vt_block<Z, NB0 + 0, PAIR>(vb, vt[NB0 + 0]);
    rebuild_vt_block<Z, NB0 + 1, PAIR>(vb, vt[NB0 + 1]);
    rebuild_vt_block<Z, NB0 + 2, PAIR>(vb, vt[NB0 + 2]);
    rebuild_vt_block<Z, NB0 + 3, PAIR>(vb, vt[NB0 + 3]);
}

// ---- per-lane LDS offsets within a stage (fixed for the kernel). With the stage base in
// an SGPR every LDS access is one v_add plus an immediate offset; accesses whose offsets
// differ by a constant share one register.
struct LdsLane {
    uint32_t sml, smh, code;          // compressed: sm units g and 4+g of row r, code
    uint32_t bw;                      // compressed: the base dword this lane reads for its row (row_bcast)
    uint32_t tw;                      // V tile row r: units 2g (+16: 2g+1, +128: 8+2g, +144: 9+2g)
    uint32_t tr[4];                   // transpose reads of channel blocks nb (+128: nb + 4)
    uint32_t bk[4];                   // bf16 K row r: units 2g, 2g+1, 8+2g, 9+2g
};

__host__ __device__ inline LdsLane lds_lane_offsets(int r, int g) {
    LdsLane o;
    o.sml = (uint32_t)(r * 128 + 16 * (g ^ (r & 7)));
    o.smh = (uint32_t)(r * 128 + 16 * ((4 + g) ^ (r & 7)));
    o.code = (uint32_t)(r * 64 + 16 * (g ^ ((r >> 1) & 3)));
    // r = 0-3: K base dword 4g + r (channels 16g + 4r ..), 4-7: K dword 16 + 4g + r - 4
    // (channels 64 + 16g + 4(r - 4) ..), 8-15: the same dwords of V (row_bcast)
    o.bw = (uint32_t)(CS_BASE + 128 * (r >> 3) + 64 * ((r >> 2) & 1) + 16 * g + 4 * (r & 3));
    // V tile / staged bf16 V: row r's logical unit u sits at physical unit u ^ ((r & 3) << 1);
    // the XOR only touches bits 1-2 of u, so units 2g+1, 8+2g, 9+2g follow at +16, +128, +144
    o.tw = (uint32_t)(r * 256 + 16 * ((2 * g) ^ ((r & 3) << 1)));
    // transpose read: lane supplies row trow = 4g + r/4, 8-byte half r & 1 of unit
    // u = 2nb + ((r & 3) >> 1), i.e. physical 2(nb ^ (trow & 3)) + ((r & 3) >> 1) for nb < 4
    const int trow = 4 * g + (r >> 2), xq = trow & 3, b1 = (r & 3) >> 1;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) o.tr[nb] = (uint32_t)(trow * 256 + 8 * (r & 1) + 16 * (2 * (nb ^ xq) + b1));
    // bf16 K rows: unit u at u ^ (r & 7)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = (j < 2 ? 2 * g : 8 + 2 * g) + (j & 1);
        o.bk[j] = (uint32_t)(r * 256 + 16 * (u ^ (r & 7)));
    }
    return o;
}

// The 16-byte sm and code reads of a lane's row (K or V) from a stage
struct StageSC {
    uint4 sm_lo, sm_hi, code;
};

// K rows (and V rows on pages with raw V rows) rebuilt from a lane's staged bytes. The 16
// lanes of one row of a wavefront (one channel group g) need the same 32 base dwords of K
// and of V: lane r of the row reads one (LdsLane::bw; r = 0-3 and 4-7: dwords 0-3 of its
// group's low and high K runs, 8-11 and 12-15: the same of V), and the rebuild takes dword
// i of a run from lane i of its own row. Bc::get<L>() returns lane L's dword: a DPP row
// broadcast on the GPU (folded by the compiler into the exponent add), an array on the host.
template <bool Z, int L, class Bc>
__host__ __device__ __forceinline__ void rebuild4_from(uint32_t s, uint32_t cn, const Bc& bc, uint32_t& o01,
                                                       uint32_t& o23) {
    const uint32_t b = bc.template get<L>();
    bf16_pairs(s, Z ? exponents(cn, b) : cn + b, o01, o23);
}
template <bool Z, bool HIGH, int L0, class Bc>
__host__ __device__ __forceinline__ void rebuild_run_from(const uint4& sm, const uint4& code, const Bc& bc,
                                                          uint32_t out[8]) {
    constexpr uint32_t m = 0x0F0F0F0Fu;
    rebuild4_from<Z, L0 + 0>(sm.x, (HIGH ? code.x >> 4 : code.x) & m, bc, out[0], out[1]);
    rebuild4_from<Z, L0 + 1>(sm.y, (HIGH ? code.y >> 4 : code.y) & m, bc, out[2], out[3]);
    rebuild4_from<Z, L0 + 2>(sm.z, (HIGH ? code.z >> 4 : code.z) & m, bc, out[4], out[5]);
    rebuild4_from<Z, L0 + 3>(sm.w, (HIGH ? code.w >> 4 : code.w) & m, bc, out[6], out[7]);
}
// K (V = false) or V values of the lane (out[0..7]: channels 16g.., out[8..15]: 64 + 16g..);
// zf = the wavefront's ballot of (bw & 0x80808080) != 0, whose bits 16g + 4q .. 16g + 4q + 3
// cover run q (K low, K high, V low, V high): the zero-group fix-up runs for a run when some
// row flags it.
template <bool V, class Bc>
__host__ __device__ __forceinline__ void rebuild_values_from(const StageSC& sc, const Bc& bc, uint64_t zf,
                                                             uint32_t out[16]) {
    constexpr int L_LO = V ? 8 : 0, L_HI = L_LO + 4;
    constexpr uint64_t rows = 0x000F000F000F000Full;
    if ((zf & (rows << L_LO)) != 0)
        rebuild_run_from<true, false, L_LO>(sc.sm_lo, sc.code, bc, out);
    else
        rebuild_run_from<false, false, L_LO>(sc.sm_lo, sc.code, bc, out);
    if ((zf & (rows << L_HI)) != 0)
        rebuild_run_from<true, true, L_HI>(sc.sm_hi, sc.code, bc, out + 8);
    else
        rebuild_run_from<false, true, L_HI>(sc.sm_hi, sc.code, bc, out + 8);
}

// Per-lane LDS offsets of the pair layout within a stage (the loader's swizzles: sm rows
// of 128 bytes with 16-byte unit u at u ^ (r & 7), code rows of 64 bytes with unit u at
// u ^ ((r >> 1) & 3), base unswizzled, V tile and staged bf16 V rows with unit u at
// u ^ ((r & 3) << 1), bf16 K rows with unit u at u ^ (r & 7)).
struct PairLane {
    uint32_t sm[4];       // 8-byte pieces: head 2v channels 8g.., 2v+1's, 2v's 32+8g.., 2v+1's
    uint32_t code[2];     // code bytes 8g..8g+7 of head 2v, of 2v+1
    uint32_t base[4];     // base bytes, in the order of sm
    uint32_t bw;          // the base dword this lane reads for its row (row_bcast)
    uint32_t tw[2];       // V tile row r: units g, 4+g (+128: 8+g, 12+g)
    uint32_t bk[4];       // bf16 K row r: units g, 8+g, 4+g, 12+g
};

__host__ __device__ inline PairLane pair_lane_offsets(int r, int g) {
    PairLane o;
    const int x7 = r & 7, xc = (r >> 1) & 3, xt = (r & 3) << 1, half = 8 * (g & 1), gu = g >> 1;
    const int smu[4] = {gu, 4 + gu, 2 + gu, 6 + gu};
#pragma unroll
    for (int i = 0; i < 4; ++i) o.sm[i] = (uint32_t)(r * 128 + 16 * (smu[i] ^ x7) + half);
    o.code[0] = (uint32_t)(r * 64 + 16 * (gu ^ xc) + half);
    o.code[1] = (uint32_t)(r * 64 + 16 * ((2 + gu) ^ xc) + half);
    o.base[0] = (uint32_t)(8 * g);
    o.base[1] = (uint32_t)(64 + 8 * g);
    o.base[2] = (uint32_t)(32 + 8 * g);
    o.base[3] = (uint32_t)(96 + 8 * g);
    // row g's base dwords in the order the rebuild takes them (b_lo = pieces 0, 1; b_hi =
    // pieces 2, 3): lane r = 0-7 K dword r, 8-15 V dword r - 8 (piece (r & 7) >> 1, half r & 1)
    const int pc = (r & 7) >> 1;                       // piece pc: bytes 8g + 64 (pc & 1) + 32 (pc >> 1)
    o.bw = (uint32_t)(CS_BASE + 128 * (r >> 3) + 8 * g + 64 * (pc & 1) + 32 * (pc >> 1) + 4 * (r & 1));
    o.tw[0] = (uint32_t)(r * 256 + 16 * (g ^ xt));
    o.tw[1] = (uint32_t)(r * 256 + 16 * ((4 + g) ^ xt));
    const int bku[4] = {g, 8 + g, 4 + g, 12 + g};
#pragma unroll
    for (int j = 0; j < 4; ++j) o.bk[j] = (uint32_t)(r * 256 + 16 * (bku[j] ^ x7));
    return o;
}

// A pair lane's row pieces into the row rebuild's registers: rd(lane offset, array offset)
// returns the 8 stage bytes at their sum (an LDS read on the GPU, the array offset an
// immediate); sm pieces in the order head 2v channels 8g.., 2v+1's, 2v's 32 + 8g.., 2v+1's,
// code pieces head 2v's then 2v+1's.
template <class R8>
__host__ __device__ __forceinline__ void stage_sm_code_pair_from(const R8& rd, const PairLane& o, int sm_off,
                                                                 int code_off, StageSC& sc) {
    const uint2 s0 = rd(o.sm[0], sm_off), s1 = rd(o.sm[1], sm_off);
    const uint2 s2 = rd(o.sm[2], sm_off), s3 = rd(o.sm[3], sm_off);
    const uint2 c0 = rd(o.code[0], code_off), c1 = rd(o.code[1], code_off);
    sc.sm_lo = make_uint4(s0.x, s0.y, s1.x, s1.y);
    sc.sm_hi = make_uint4(s2.x, s2.y, s3.x, s3.y);
    sc.code = make_uint4(c0.x, c0.y, c1.x, c1.y);
}

}  // namespace exkv
