// Exhaustive CPU check of the 4-channel value rebuild used by the HIP decoder
// (exactkv_amd/csrc/common.hpp rebuild4, exponents) against the scalar format rule
// (reference exactkv/codec.py:65-68): for every sign|mantissa byte, every base byte and
// every 4-bit code, in every byte lane, with random neighbours in the other lanes.
#include "../../exactkv_amd/csrc/common.hpp"
#include <cstdio>
#include <cstdlib>

static uint16_t scalar_decode(uint32_t sm, uint32_t code, uint32_t base) {
    uint32_t e = (base & 127) + code;
    if (base >= 128 && code == 0) e = 0;
    return (uint16_t)(((sm & 0x80) << 8) | ((e & 0xFF) << 7) | (sm & 0x7F));
}

int main() {
    uint64_t rng = 0x9E3779B97F4A7C15ull;
    auto next = [&]() { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return (uint32_t)rng; };
    long bad = 0, n = 0;
    for (int lane = 0; lane < 4; ++lane)
        for (uint32_t sm = 0; sm < 256; ++sm)
            for (uint32_t base = 0; base < 256; ++base)
                for (uint32_t code = 0; code < 16; ++code) {
                    uint32_t s[4], c[4], b[4];
                    for (int i = 0; i < 4; ++i) { s[i] = next() & 255; c[i] = next() & 15; b[i] = next() & 255; }
                    s[lane] = sm; c[lane] = code; b[lane] = base;
                    uint32_t S = 0, CN = 0, BB = 0, ZF = 0;
                    for (int i = 0; i < 4; ++i) {
                        S |= s[i] << (8 * i); CN |= c[i] << (8 * i);
                        BB |= b[i] << (8 * i); ZF |= (b[i] & 128) << (8 * i);
                    }
                    uint32_t o01, o23, p01, p23;
                    exkv::rebuild4<true>(S, CN, BB, o01, o23);
                    uint16_t got[4] = {(uint16_t)o01, (uint16_t)(o01 >> 16), (uint16_t)o23, (uint16_t)(o23 >> 16)};
                    for (int i = 0; i < 4; ++i) {
                        ++n;
                        if (got[i] != scalar_decode(s[i], c[i], b[i])) { if (bad < 5) printf("bad lane %d sm %u base %u code %u\n", i, s[i], b[i], c[i]); ++bad; }
                    }
                    // without zero groups the fast variant must agree whenever no flag is set
                    if (ZF == 0) {
                        exkv::rebuild4<false>(S, CN, BB, p01, p23);
                        if (p01 != o01 || p23 != o23) { ++bad; }
                    }
                }
    printf("checked %ld values, %ld mismatches\n", n, bad);
    return bad ? 1 : 0;
}
