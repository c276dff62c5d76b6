// CPU check of the compressed split kernel's row rebuild (exactkv_amd/csrc/stage.hpp: K rows,
// and the V rows of pages with raw V rows) against the scalar format rule (reference
// exactkv/codec.py:65-68). A page's bytes are placed in a stage image the way the loader
// wavefronts' direct-to-LDS loads place them (dma_lane_offsets); lane (r = lane & 15,
// g = lane >> 4) reads its sm and code row pieces and its base dword at lds_lane_offsets(r, g);
// the zero-group decision is the wavefront's ballot of flagged base dwords; and
// rebuild_values_from runs with the dwords of the lane's own 16-lane row as the broadcast
// source (the DPP row broadcast of the GPU build). Lane (r, g) must hold token r's channels
// 16g + 2k, 16g + 2k + 1 in out[k] (k < 8) and 64 + 16g + 2(k - 8), + 1 in out[k] (k >= 8).
// Also with the fix-up forced on every run, and with it off on pages without flagged groups.
// Then the head-dim-64 pair kernel's K rows (two heads 2v, 2v + 1 of 64 channels as one
// 128-byte virtual row, each head's code row of 32 bytes holding channels j and j + 32):
// lane (r, g) reads its pieces at pair_lane_offsets(r, g) through stage_sm_code_pair_from and
// must hold head 2v channels 8g.. in out[0..3], head 2v + 1's in out[4..7], head 2v channels
// 32 + 8g.. in out[8..11] and head 2v + 1's in out[12..15].
#include "../../exactkv_amd/csrc/stage.hpp"
#include <cstdio>
#include <cstring>
#include <vector>

using namespace exkv;

static uint16_t scalar_decode(uint32_t sm, uint32_t code, uint32_t base) {
    uint32_t e = (base & 127) + code;
    if (base >= 128 && code == 0) e = 0;
    return (uint16_t)(((sm & 0x80) << 8) | ((e & 0xFF) << 7) | (sm & 0x7F));
}

struct Rng {
    uint64_t s;
    uint32_t next() { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return (uint32_t)s; }
};

// One page of K and V in HBM order: sm [16][rs][128], code [16][rs][64], base [rs][128].
struct Arr {
    std::vector<uint8_t> sm, code, base;
};
struct Page {
    int rs, hk;
    Arr k, v;
};

static uint16_t expect(const Page& p, const Arr& a, int t, int c) {
    const size_t row = (size_t)t * p.rs + p.hk;
    const uint32_t code = (a.code[row * 64 + (c & 63)] >> (c >= 64 ? 4 : 0)) & 15;
    return scalar_decode(a.sm[row * 128 + c], code, a.base[(size_t)p.hk * 128 + c]);
}

static void place(const Page& p, uint8_t* st) {
    for (int lane = 0; lane < 64; ++lane) {
        const DmaLane o = dma_lane_offsets<true>(lane, p.rs);
        const size_t r0 = (size_t)p.hk;
        memcpy(st + CS_KSM + 16 * lane, &p.k.sm[r0 * 128 + o.sm0], 16);
        memcpy(st + CS_VSM + 16 * lane, &p.v.sm[r0 * 128 + o.sm0], 16);
        memcpy(st + CS_KSM + 1024 + 16 * lane, &p.k.sm[r0 * 128 + o.sm1], 16);
        memcpy(st + CS_VSM + 1024 + 16 * lane, &p.v.sm[r0 * 128 + o.sm1], 16);
        memcpy(st + CS_KCODE + 16 * lane, &p.k.code[r0 * 64 + o.code], 16);
        memcpy(st + CS_VCODE + 16 * lane, &p.v.code[r0 * 64 + o.code], 16);
        if (lane < 16)                                  // lanes 0-7: K's base row, 8-15: V's
            memcpy(st + CS_BASE + 16 * lane, &(lane < 8 ? p.k : p.v).base[(size_t)p.hk * 128 + o.base], 16);
    }
}

struct HostRow {                                        // lane L of the row
    const uint32_t* bw;
    template <int L>
    uint32_t get() const { return bw[L]; }
};

static uint4 rd16(const uint8_t* st, uint32_t off) {
    uint4 v;
    memcpy(&v, st + off, 16);
    return v;
}

// force: -1 the wavefront's ballot, 0 no fix-up, 1 fix-up on every run
template <bool V>
static long check(const Page& p, const uint8_t* st, int force, bool* flagged) {
    uint32_t bw[64];
    uint64_t zf = 0;
    for (int lane = 0; lane < 64; ++lane) {
        const LdsLane o = lds_lane_offsets(lane & 15, lane >> 4);
        memcpy(&bw[lane], st + o.bw, 4);
        if ((bw[lane] & 0x80808080u) != 0u) zf |= 1ull << lane;
    }
    if (flagged) *flagged = zf != 0;
    const uint64_t z = force < 0 ? zf : (force ? ~0ull : 0ull);
    long bad = 0;
    for (int lane = 0; lane < 64; ++lane) {
        const int r = lane & 15, g = lane >> 4;
        const LdsLane o = lds_lane_offsets(r, g);
        StageSC sc;
        sc.sm_lo = rd16(st, (V ? CS_VSM : CS_KSM) + o.sml);
        sc.sm_hi = rd16(st, (V ? CS_VSM : CS_KSM) + o.smh);
        sc.code = rd16(st, (V ? CS_VCODE : CS_KCODE) + o.code);
        uint32_t out[16];
        rebuild_values_from<V>(sc, HostRow{bw + 16 * g}, z, out);
        for (int k = 0; k < 16; ++k)
            for (int h = 0; h < 2; ++h) {
                const int c = (k < 8 ? 16 * g + 2 * k : 64 + 16 * g + 2 * (k - 8)) + h;
                const uint16_t got = (uint16_t)(out[k] >> (16 * h));
                const uint16_t want = expect(p, V ? p.v : p.k, r, c);
                if (got != want) {
                    if (bad < 4)
                        printf("  %s lane %d token %d channel %d: got %04x want %04x\n", V ? "V" : "K", lane, r, c,
                               got, want);
                    ++bad;
                }
            }
    }
    return bad;
}

static void fill(Arr& a, Rng& rng, int rs, int mode) {
    a.sm.resize((size_t)16 * rs * 128);
    a.code.resize((size_t)16 * rs * 64);
    a.base.resize((size_t)rs * 128);
    for (auto& b : a.sm) b = rng.next() & 255;
    for (auto& b : a.code) b = (rng.next() % 5 == 0) ? 0 : rng.next() & 255;
    for (auto& b : a.base) {
        uint32_t x = rng.next() & 127;
        const uint32_t u = rng.next() % 64;
        if ((mode == 1 && u == 0) || (mode == 2 && u < 16) || (mode == 3 && u < 60)) x |= 128;
        b = (uint8_t)x;
    }
}

// Pair layout: virtual channel 64h + c is head 2v + h's channel c (c < 64)
static uint16_t expect_pair(const Page& p, int t, int h, int c) {
    const size_t row = (size_t)t * p.rs + p.hk;
    const uint32_t code = (p.k.code[row * 64 + 32 * h + (c & 31)] >> (c >= 32 ? 4 : 0)) & 15;
    return scalar_decode(p.k.sm[row * 128 + 64 * h + c], code, p.k.base[(size_t)p.hk * 128 + 64 * h + c]);
}

static long check_pair(const Page& p, const uint8_t* st, int force, bool* flagged) {
    uint32_t bw[64];
    uint64_t zf = 0;
    for (int lane = 0; lane < 64; ++lane) {
        const PairLane o = pair_lane_offsets(lane & 15, lane >> 4);
        memcpy(&bw[lane], st + o.bw, 4);
        if ((bw[lane] & 0x80808080u) != 0u) zf |= 1ull << lane;
    }
    if (flagged) *flagged = zf != 0;
    const uint64_t z = force < 0 ? zf : (force ? ~0ull : 0ull);
    auto rd = [&](uint32_t off, int arr) {
        uint2 v;
        memcpy(&v, st + off + arr, 8);
        return v;
    };
    long bad = 0;
    for (int lane = 0; lane < 64; ++lane) {
        const int r = lane & 15, g = lane >> 4;
        const PairLane o = pair_lane_offsets(r, g);
        StageSC sc;
        stage_sm_code_pair_from(rd, o, CS_KSM, CS_KCODE, sc);
        uint32_t out[16];
        rebuild_values_from<false>(sc, HostRow{bw + 16 * g}, z, out);
        for (int k = 0; k < 16; ++k)
            for (int x = 0; x < 2; ++x) {
                const int h = (k >> 2) & 1, c = (k >= 8 ? 32 : 0) + 8 * g + 2 * (k & 3) + x;
                const uint16_t got = (uint16_t)(out[k] >> (16 * x)), want = expect_pair(p, r, h, c);
                if (got != want) {
                    if (bad < 4)
                        printf("  pair lane %d token %d head %d channel %d: got %04x want %04x\n", lane, r, h, c, got,
                               want);
                    ++bad;
                }
            }
    }
    return bad;
}

int main() {
    Rng rng{0x9E3779B97F4A7C15ull};
    long bad = 0, pages = 0, flagged = 0, plain = 0;
    const int shapes[][2] = {{1, 0}, {4, 3}, {8, 5}, {3, 1}};   // (row stride in heads, head)
    for (int trial = 0; trial < 400; ++trial) {
        Page p;
        p.rs = shapes[trial & 3][0];
        p.hk = shapes[trial & 3][1];
        fill(p.k, rng, p.rs, (trial >> 2) % 4);
        fill(p.v, rng, p.rs, (trial >> 4) % 4);
        static uint8_t st[CS_BYTES];
        memset(st, 0x5A, sizeof st);
        place(p, st);
        for (int v = 0; v < 2; ++v) {
            bool any = false;
            long b0 = v ? check<true>(p, st, -1, &any) : check<false>(p, st, -1, &any);
            long b1 = v ? check<true>(p, st, 1, nullptr) : check<false>(p, st, 1, nullptr);
            long b2 = 0;
            if (!any) {
                b2 = v ? check<true>(p, st, 0, nullptr) : check<false>(p, st, 0, nullptr);
                ++plain;
            } else {
                ++flagged;
            }
            if (b0 || b1 || b2) printf("trial %d (rs %d head %d, %s): %ld %ld %ld\n", trial, p.rs, p.hk, v ? "V" : "K", b0, b1, b2);
            bad += b0 + b1 + b2;
            ++pages;
        }
    }
    // head-dim-64 pairs: the same stage placement (a virtual head's rows are the pair's)
    for (int trial = 0; trial < 200; ++trial) {
        Page p;
        p.rs = shapes[trial & 3][0];
        p.hk = shapes[trial & 3][1];
        fill(p.k, rng, p.rs, (trial >> 2) % 4);
        fill(p.v, rng, p.rs, 0);
        static uint8_t st[CS_BYTES];
        memset(st, 0xC3, sizeof st);
        place(p, st);
        bool any = false;
        const long b0 = check_pair(p, st, -1, &any), b1 = check_pair(p, st, 1, nullptr);
        const long b2 = any ? 0 : check_pair(p, st, 0, nullptr);
        (any ? flagged : plain) += 1;
        if (b0 || b1 || b2) printf("pair trial %d (rs %d pair %d): %ld %ld %ld\n", trial, p.rs, p.hk, b0, b1, b2);
        bad += b0 + b1 + b2;
        ++pages;
    }
    printf("checked %ld page rebuilds (%ld with flagged base bytes, %ld without), %ld mismatches\n", pages, flagged,
           plain, bad);
    return bad || !flagged || !plain ? 1 : 0;
}
