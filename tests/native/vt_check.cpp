// CPU check of the compressed split kernels' V^T path (exactkv_amd/csrc/stage.hpp) against
// the scalar format rule (reference exactkv/codec.py:65-68): a page's bytes are placed in a
// stage image the way the loader wavefronts' direct-to-LDS loads place them
// (dma_lane_offsets, each lane's 16 bytes at the load's LDS base + 16 * lane), each lane's
// ds_read_b64_tr_b8 reads at vt_lane_offsets are emulated (in each 16-lane group, lanes 2k
// and 2k + 1 form row k of an 8 x 16 byte matrix and lane i receives byte i of rows 0..7:
// rows 0-3 in the low dword, rows 4-7 in the high one), and rebuild_vt_run must then give
// lane (i = lane & 15, kb = lane >> 4) the values V[4kb + j][16nb + i], j = 0..3, of every
// channel block nb. Both layouts: one head of 128 channels, and a pair of head-dim-64
// heads as one virtual head (attn_pair_kernel). Each run of four blocks takes the
// zero-group fix-up when any lane of the wavefront has a flagged base byte (the kernel's
// ballot); the fix-up is also checked on every page, and the plain form on pages with no
// flagged base byte.
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

// One page of one head's V in HBM order: sm [16][rs][128], code [16][rs][64] (row stride rs
// heads, or head pairs), base [rs][128]; the checked head is hk.
struct Page {
    int rs, hk;
    std::vector<uint8_t> sm, code, base;
};

// The value of token t, virtual channel c of head hk under the format rule. PAIR: channels
// 0-63 are head 2hk's, 64-127 head 2hk + 1's, each with 32-byte code rows whose byte j holds
// its channels j (low nibble) and j + 32 (high); otherwise code byte j holds channels j and
// j + 64.
static uint16_t expect(const Page& p, int t, int c, bool pair) {
    const size_t row = (size_t)t * p.rs + p.hk;
    const uint32_t sm = p.sm[row * 128 + c];
    int cb, hi;
    if (pair) {
        const int h = c >> 6, cc = c & 63;
        cb = 32 * h + (cc & 31);
        hi = cc >= 32;
    } else {
        cb = c & 63;
        hi = c >= 64;
    }
    const uint32_t code = (p.code[row * 64 + cb] >> (hi ? 4 : 0)) & 15;
    const uint32_t base = p.base[(size_t)p.hk * 128 + c];
    return scalar_decode(sm, code, base);
}

// The stage as the loads leave it (only the V parts and the base rows matter here; the K
// parts get the same treatment with K's arrays).
static void place(const Page& p, uint8_t* stage) {
    for (int lane = 0; lane < 64; ++lane) {
        const DmaLane o = dma_lane_offsets<true>(lane, p.rs);
        const size_t row0 = (size_t)p.hk;              // token 0 of the page, head hk
        memcpy(stage + CS_VSM + 16 * lane, &p.sm[row0 * 128 + o.sm0], 16);
        memcpy(stage + CS_VSM + 1024 + 16 * lane, &p.sm[row0 * 128 + o.sm1], 16);
        memcpy(stage + CS_VCODE + 16 * lane, &p.code[row0 * 64 + o.code], 16);
        if (lane >= 8 && lane < 16)                    // lanes 8-15: V's base row
            memcpy(stage + CS_BASE + 16 * lane, &p.base[(size_t)p.hk * 128 + o.base], 16);
    }
}

// ds_read_b64_tr_b8 over the wavefront: addr[lane] -> out[lane]
static void tr_b8(const uint8_t* stage, const uint32_t* addr, uint32_t (*out)[2]) {
    for (int g = 0; g < 4; ++g) {
        uint8_t rows[8][16];
        for (int k = 0; k < 8; ++k) {
            memcpy(rows[k], stage + addr[16 * g + 2 * k], 8);
            memcpy(rows[k] + 8, stage + addr[16 * g + 2 * k + 1], 8);
        }
        for (int i = 0; i < 16; ++i) {
            uint32_t x = 0, y = 0;
            for (int j = 0; j < 4; ++j) {
                x |= (uint32_t)rows[j][i] << (8 * j);
                y |= (uint32_t)rows[4 + j][i] << (8 * j);
            }
            out[16 * g + i][0] = x;
            out[16 * g + i][1] = y;
        }
    }
}

static void read_vt_bytes(const uint8_t* stage, VtBytes* vb) {
    VtLane o[64];
    for (int lane = 0; lane < 64; ++lane) o[lane] = vt_lane_offsets(lane);
    uint32_t addr[64], out[64][2];
    for (int nb = 0; nb < 4; ++nb) {
        for (int l = 0; l < 64; ++l) addr[l] = o[l].sm[nb];
        tr_b8(stage, addr, out);
        for (int l = 0; l < 64; ++l) { vb[l].sm[nb] = out[l][0]; vb[l].sm[nb + 4] = out[l][1]; }
    }
    for (int c = 0; c < 2; ++c) {
        for (int l = 0; l < 64; ++l) addr[l] = o[l].code[c];
        tr_b8(stage, addr, out);
        for (int l = 0; l < 64; ++l) { vb[l].code[2 * c] = out[l][0]; vb[l].code[2 * c + 1] = out[l][1]; }
    }
    for (int l = 0; l < 64; ++l) addr[l] = o[l].base;
    tr_b8(stage, addr, out);
    for (int l = 0; l < 64; ++l) { vb[l].base[0] = out[l][0]; vb[l].base[1] = out[l][1]; }
}

template <bool PAIR, int NB0>
static void run(const VtBytes& vb, bool z, s16x4 (&vt)[8]) {
    if (z)
        rebuild_vt_run<true, NB0, PAIR>(vb, vt);
    else
        rebuild_vt_run<false, NB0, PAIR>(vb, vt);
}

// Rebuild every lane's operand with the given fix-up choice per run (-1: the wavefront's
// ballot) and count the values that differ from the rule.
template <bool PAIR>
static long check(const Page& p, const VtBytes* vb, int force, bool* any_flag) {
    bool z[2] = {false, false};
    for (int l = 0; l < 64; ++l)
        for (int r = 0; r < 2; ++r) z[r] = z[r] || (vb[l].base[r] & 0x80808080u) != 0u;
    if (any_flag) *any_flag = z[0] || z[1];
    if (force >= 0) z[0] = z[1] = force != 0;
    long bad = 0;
    for (int lane = 0; lane < 64; ++lane) {
        s16x4 vt[8];
        run<PAIR, 0>(vb[lane], z[0], vt);
        run<PAIR, 4>(vb[lane], z[1], vt);
        const int i = lane & 15, kb = lane >> 4;
        for (int nb = 0; nb < 8; ++nb)
            for (int j = 0; j < 4; ++j) {
                const uint16_t got = (uint16_t)vt[nb][j], want = expect(p, 4 * kb + j, 16 * nb + i, PAIR);
                if (got != want) {
                    if (bad < 4)
                        printf("  %s lane %d block %d token %d channel %d: got %04x want %04x\n", PAIR ? "pair" : "d128",
                               lane, nb, 4 * kb + j, 16 * nb + i, got, want);
                    ++bad;
                }
            }
    }
    return bad;
}

int main() {
    Rng rng{0x2545F4914F6CDD1Dull};
    long bad = 0, pages = 0, flagged = 0, plain = 0;
    const int shapes[][2] = {{1, 0}, {4, 3}, {8, 5}, {3, 1}};   // (row stride, head)
    for (int trial = 0; trial < 400; ++trial) {
        Page p;
        p.rs = shapes[trial & 3][0];
        p.hk = shapes[trial & 3][1];
        p.sm.resize((size_t)16 * p.rs * 128);
        p.code.resize((size_t)16 * p.rs * 64);
        p.base.resize((size_t)p.rs * 128);
        for (auto& b : p.sm) b = rng.next() & 255;
        // codes: mostly random, some all-zero rows so that flagged groups hold zeros
        for (auto& b : p.code) b = (rng.next() % 5 == 0) ? 0 : rng.next() & 255;
        // base bytes: none flagged, a few, or many (mode per trial); every value reachable
        const int mode = (trial >> 2) % 4;
        for (auto& b : p.base) {
            uint32_t v = rng.next() & 127;
            const uint32_t u = rng.next() % 64;
            if ((mode == 1 && u == 0) || (mode == 2 && u < 16) || (mode == 3 && u < 60)) v |= 128;
            b = (uint8_t)v;
        }
        static uint8_t stage[CS_BYTES];
        memset(stage, 0xA5, sizeof stage);
        place(p, stage);
        VtBytes vb[64];
        read_vt_bytes(stage, vb);
        bool any = false;
        const bool pair = trial & 1;
        const long b0 = pair ? check<true>(p, vb, -1, &any) : check<false>(p, vb, -1, &any);
        const long b1 = pair ? check<true>(p, vb, 1, nullptr) : check<false>(p, vb, 1, nullptr);
        long b2 = 0;
        if (!any) {
            b2 = pair ? check<true>(p, vb, 0, nullptr) : check<false>(p, vb, 0, nullptr);
            ++plain;
        } else {
            ++flagged;
        }
        if (b0 || b1 || b2) printf("trial %d (rs %d head %d, %s): %ld %ld %ld\n", trial, p.rs, p.hk, pair ? "pair" : "d128", b0, b1, b2);
        bad += b0 + b1 + b2;
        ++pages;
    }
    printf("checked %ld pages (%ld with flagged base bytes, %ld without), %ld mismatches\n", pages, flagged, plain, bad);
    return bad || !flagged || !plain ? 1 : 0;
}
