// CPU check of the clamp detection behind the kernels' sticky error bit EXKV_ERR_RAW_SLOT
// (exactkv_amd/csrc/tile.hpp raw_slot_checked, errors.hpp clamp_slot): the slot of token
// r's raw row is rowoff + popcount(rowmask below r) (reference kernels.py:119-123); a slot
// outside [0, raw_rows) is clamped into the pool and flagged, but only for a token that
// has a raw row (other lanes compute a slot they never use).
#include "../../exactkv_amd/csrc/tile.hpp"
#include <cstdio>

int main() {
    long bad_cases = 0, n = 0;
    auto check = [&](bool cond, const char* what, uint32_t m, int32_t roff, int r, int64_t rows) {
        ++n;
        if (!cond) {
            if (bad_cases < 10) printf("FAIL %s: mask %#x roff %d r %d rows %lld\n", what, m, roff, r, (long long)rows);
            ++bad_cases;
        }
    };
    uint64_t rng = 0x2545F4914F6CDD1Dull;
    auto next = [&]() { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return rng; };
    for (int it = 0; it < 200000; ++it) {
        const uint32_t m = (uint32_t)next() & 0xFFFFu;
        const int64_t rows = 1 + (int64_t)(next() % 4096);
        // rowoff anywhere from well below 0 to well past the pool
        const int32_t roff = (int32_t)((int64_t)(next() % (3 * 4096 + 64)) - 4096 - 32);
        for (int r = 0; r < 16; ++r) {
            bool bad = false;
            const int64_t s = exkv::raw_slot_checked(m, roff, r, rows, bad);
            const int64_t want = (int64_t)roff + __builtin_popcount(m & ((1u << r) - 1u));
            const bool used = (m >> r) & 1u;
            const bool inside = want >= 0 && want < rows;
            check(s >= 0 && s < rows, "slot inside the pool", m, roff, r, rows);
            check(!inside || s == want, "in-pool slot unchanged", m, roff, r, rows);
            check(bad == (used && !inside), "flag exactly for a used, clamped slot", m, roff, r, rows);
        }
    }
    // edges: the last slot of the pool, one past it, -1
    bool b = true;
    check(exkv::raw_slot_checked(1u, 99, 0, 100, b) == 99 && !b, "last slot", 1u, 99, 0, 100);
    check(exkv::raw_slot_checked(1u, 100, 0, 100, b) == 99 && b, "one past", 1u, 100, 0, 100);
    check(exkv::raw_slot_checked(1u, -1, 0, 100, b) == 0 && b, "below zero", 1u, -1, 0, 100);
    check(exkv::raw_slot_checked(2u, 100, 0, 100, b) == 99 && !b, "unused lane", 2u, 100, 0, 100);
    bool cb = false;
    check(exkv::clamp_slot(5, 5, cb) == 4 && cb, "clamp_slot past", 0, 5, 0, 5);
    check(exkv::clamp_slot(4, 5, cb) == 4 && !cb, "clamp_slot inside", 0, 4, 0, 5);
    printf("%ld checks, %ld failures\n", n, bad_cases);
    return bad_cases == 0 ? 0 : 1;
}
