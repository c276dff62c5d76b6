// Shared definitions for the exactkv HIP kernels (gfx950 / CDNA4).
//
// Byte format (reference exactkv/codec.py:1-25): per (sequence, 16-token page, KV head,
// channel) one base byte; per element a sign|mantissa byte and a 4-bit exponent code,
// where code byte j of a row holds channel j (low nibble) and channel j + D/2 (high
// nibble). base < 128: exponent = base + code. base >= 128 (a group with zeros):
// code 0 means exponent 0, otherwise exponent = base - 128 + code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exkv {

constexpr int kPage = 16;     // tokens per page
constexpr int kD = 128;       // head dimension of the tuned attention kernels

// Head dimensions the kernels are built for: 128 (Qwen2/2.5/3, Llama-3), 64 (the small
// Qwen2.5 and Llama-3.2 models) and 256.
__host__ __device__ constexpr bool head_dim_ok(int D) { return D == 64 || D == 128 || D == 256; }

// ---------------------------------------------------------------- bit helpers

// v_perm_b32: byte i of the result = byte sel.byte[i] of the 8-byte value {hi, lo}
// (bytes 0-3 from lo, 4-7 from hi; selector 12 gives 0x00).
__host__ __device__ inline uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_perm(hi, lo, sel);
#else
    uint64_t v = ((uint64_t)hi << 32) | lo;
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        uint32_t s = (sel >> (8 * i)) & 0xFF;
        uint32_t b = s < 8 ? (uint32_t)((v >> (8 * s)) & 0xFF) : (s == 12 ? 0u : 0xFFu);
        r |= b << (8 * i);
    }
    return r;
#endif
}

// (m & a) | (~m & b): one v_bfi_b32.
__host__ __device__ inline uint32_t bfi_b32(uint32_t m, uint32_t a, uint32_t b) {
    return (m & a) | (~m & b);
}

// ---------------------------------------------------------------- value rebuild
//
// Four consecutive channels at once. s: their sign|mantissa bytes; cn: their 4-bit codes,
// one per byte (0..15); base: their base bytes. Without zero groups (HAS_ZERO_GROUPS false)
// every base byte must be < 128. Result: two dwords of bf16 pairs (channel c in the low
// half, c + 1 in the high half), bit-identical to the reference decoder (codec.py:65-68,
// kernels.py:96-103).
//
// exponent e = (base & 127) + code (<= 142, so the bytewise add never carries), or 0 in a
// flagged group (base >= 128) where code == 0. The bf16 is
// hi byte = (s & 0x80) | (e >> 1), lo byte = (e & 1) << 7 | (s & 0x7F).
__host__ __device__ inline uint32_t exponents(uint32_t cn, uint32_t base) {
    // z80: bit 7 of a byte set iff its group is flagged and its code is 0 (code <= 15, so
    // 0x80 - code keeps bit 7 exactly when code == 0); fm: 0x7F in those bytes, which
    // clears the base there (the exponent is then the code, 0)
    const uint32_t z80 = base & (0x80808080u - cn) & 0x80808080u;
    const uint32_t fm = z80 - (z80 >> 7);
    return (base & 0x7F7F7F7Fu & ~fm) + cn;
}

// The two bf16 pairs of four channels from their sign|mantissa bytes s and exponents e.
__host__ __device__ inline void bf16_pairs(uint32_t s, uint32_t e, uint32_t& out01, uint32_t& out23) {
    const uint32_t lo = bfi_b32(0x7F7F7F7Fu, s, e << 7);
    const uint32_t hi = bfi_b32(0x80808080u, s, e >> 1);
    out01 = perm_b32(hi, lo, 0x05010400u);
    out23 = perm_b32(hi, lo, 0x07030602u);
}

template <bool HAS_ZERO_GROUPS>
__host__ __device__ inline void rebuild4(uint32_t s, uint32_t cn, uint32_t base, uint32_t& out01, uint32_t& out23) {
    bf16_pairs(s, HAS_ZERO_GROUPS ? exponents(cn, base) : cn + base, out01, out23);
}

// ---------------------------------------------------------------- small device utils

__device__ inline int popc32(uint32_t x) { return __builtin_popcount(x); }

// Inclusive prefix sum across the 64 lanes of a wavefront (DPP row shifts within each row
// of 16 lanes, then the row-15 and row-31 broadcasts into the rows above them).
__device__ inline int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15 -> rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31 -> rows 2, 3
    return x;
}

// Block-wide exclusive scan of one int per thread (1024 threads, all of them calling).
// Synchronises on entry to the cross-wavefront step and before returning.
__device__ inline int block_excl_scan(int v, int& total) {
    __shared__ int wsum[16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int inc = wave_incl_scan(v);
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    int wpre = 0;
    total = 0;
    for (int i = 0; i < 16; ++i) {
        const int s = wsum[i];
        if (i < w) wpre += s;
        total += s;
    }
    __syncthreads();
    return wpre + inc - v;
}

}  // namespace exkv

// ---------------------------------------------------------------- C-ABI error plumbing
namespace exkv {
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* where);
// Launch the fetch of one source file's sticky error word (errors.hpp) on `stream`.
hipError_t fetch_errors_attention(uint32_t* out, int first, int clear, hipStream_t stream);
hipError_t fetch_errors_encode(uint32_t* out, int first, int clear, hipStream_t stream);
hipError_t fetch_errors_wire(uint32_t* out, int first, int clear, hipStream_t stream);
}  // namespace exkv

#define EXKV_OK 0
#define EXKV_E_ARG 1
#define EXKV_E_HIP 2

#define EXKV_REQUIRE(cond, ...)                  \
    do {                                         \
        if (!(cond)) {                           \
            exkv::set_error(__VA_ARGS__);        \
            return EXKV_E_ARG;                   \
        }                                        \
    } while (0)
