// C-ABI plumbing: version, error messages, the split planner.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"
#include "../../include/exactkv.h"

namespace exkv {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int hip_status(hipError_t e, const char* where) {
    if (e == hipSuccess) return EXKV_OK;
    set_error("%s: HIP error %d (%s)", where, (int)e, hipGetErrorString(e));
    return EXKV_E_HIP;
}

}  // namespace exkv

extern "C" int exkv_abi_version(void) { return 4; }

extern "C" int exkv_error_bits(uint32_t* out, int32_t clear, hipStream_t stream) {
    EXKV_REQUIRE(out, "error_bits: null output");
    hipError_t e = exkv::fetch_errors_attention(out, 1, clear, stream);
    if (e == hipSuccess) e = exkv::fetch_errors_encode(out, 0, clear, stream);
    if (e == hipSuccess) e = exkv::fetch_errors_wire(out, 0, clear, stream);
    return exkv::hip_status(e, "error_bits");
}

extern "C" const char* exkv_last_error(void) { return exkv::g_err; }

// Split plan for MI355X: about target_blocks workgroups in total over B * (Hkv / HW) * head
// groups, where a workgroup covers HW = min(gcd(Hkv, 8), 4) KV heads -- 256 by default, one per
// CU, since a workgroup holds ~150 KB of LDS -- with
// at least min_split tokens per split (16 by default, one page: a wavefront's pages follow
// one another at about one memory round trip each, so a few units are served best by many
// short splits; measured with one round of workgroups, 64- / 32- / 16-token splits: a
// 1024-token window of one B1 x 128K sequence 14.2 / 11.1 / 9.6 us, B8 x 1024 15.8 / 14.7
// us, B1 x 8192 16.1 / 14.3 us) and a split length that is a multiple of 32, or 16. Plays
// the role of the reference's choose_split
// (kernels.py:273-277), which targets 512 programs for a 128-SM-class GPU.
// The split count for `units` workgroup units: up to target_blocks units, one round of
// about target_blocks workgroups; more units than that: the fewest splits that give at
// least two rounds (the second round's workgroups start as the first ones end, which
// staggers the tail) with the last round at least 95% full (else the fullest within 16
// splits). Every workgroup pays a first-page latency of a few us, so long splits win once
// the GPU is full: measured at B256 x 4352, 1/2/4/8 splits: 610/601/614/636 us; B620: 2
// splits 1454 us, 4 splits 1490 us.
static void plan_core(int64_t units, int32_t T, int64_t target_blocks, int32_t min_split, int32_t* nsplit,
                      int32_t* split_len) {
    int64_t ns = 1;
    if (units < target_blocks) {
        ns = (target_blocks + units - 1) / units;
    } else {
        double best = -1.0;
        for (int64_t n = 1; n <= 16; ++n) {
            const double rounds = (double)(units * n) / target_blocks;
            if (rounds < 2.0) continue;
            const double full = rounds / (double)(int64_t)(rounds + 0.999999);
            if (full > best) {
                best = full;
                ns = n;
            }
            if (full >= 0.95) break;
        }
    }
    const int64_t cap = ((int64_t)T + min_split - 1) / min_split;
    if (ns > cap) ns = cap;
    if (ns < 1) ns = 1;
    int64_t sl = ((int64_t)T + ns - 1) / ns;
    sl = sl <= exkv::kPage ? exkv::kPage : (sl + 31) / 32 * 32;
    *split_len = (int32_t)sl;
    *nsplit = (int32_t)(((int64_t)T + sl - 1) / sl);
}

extern "C" int exkv_plan_splits(int32_t B, int32_t Hkv, int32_t Hq, int32_t T, int32_t target_blocks,
                                int32_t min_split, int32_t* nsplit, int32_t* split_len) {
    EXKV_REQUIRE(B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && T > 0, "plan_splits: bad arguments");
    EXKV_REQUIRE(nsplit && split_len, "plan_splits: null output");
    if (target_blocks <= 0) target_blocks = 256;
    if (min_split <= 0) min_split = exkv::kPage;
    const int64_t hg = (Hq / Hkv + 15) / 16;
    int hw = Hkv, m = 8;                               // KV heads per workgroup: gcd(Hkv, 8), at most 4
    while (m) {
        const int t = hw % m;
        hw = m;
        m = t;
    }
    if (hw > 4) hw = 4;
    plan_core((int64_t)B * (Hkv / hw) * hg, T, target_blocks, min_split, nsplit, split_len);
    return EXKV_OK;
}

// Split plan per head dim. 128: the plan of exkv_plan_splits with its defaults. 64 with an
// even number of KV heads runs the head-dim-128 kernel structure over pairs of heads
// (virtual heads of 128 bytes per row): the same plan over Hkv / 2 virtual heads, a
// workgroup covering min(gcd(Hkv / 2, 8), 4) of them. Otherwise (256, or 64 with an odd
// count) the generic kernel, whose workgroups cover one KV head and one group of 16 query
// heads: rounds are counted in 512 workgroups, two per CU (the GPU holds three at head dim
// 64, two at 256, by their LDS rings); with fewer units than that, head dim 64 fills all
// three slots of every CU (768 workgroups). Measured at the c2a shape (B8 x 8192, 32q/8kv,
// split kernel): at 256, 8 splits 88.3 us against 153.1 / 95.0 for 4 / 16.
extern "C" int exkv_plan_splits_hd(int32_t B, int32_t Hkv, int32_t Hq, int32_t T, int32_t D, int32_t* nsplit,
                                   int32_t* split_len) {
    EXKV_REQUIRE(exkv::head_dim_ok(D), "plan_splits_hd: head dim must be 64, 128 or 256 (got %d)", D);
    if (D == 128) return exkv_plan_splits(B, Hkv, Hq, T, 0, 0, nsplit, split_len);
    EXKV_REQUIRE(B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && T > 0, "plan_splits_hd: bad arguments");
    EXKV_REQUIRE(nsplit && split_len, "plan_splits_hd: null output");
    if (D == 64 && Hkv % 2 == 0) {
        int hw = Hkv / 2, m = 8;                       // virtual heads per workgroup: gcd(Hkv / 2, 8), at most 4
        while (m) {
            const int t = hw % m;
            hw = m;
            m = t;
        }
        if (hw > 4) hw = 4;
        plan_core((int64_t)B * (Hkv / 2 / hw) * ((Hq / Hkv + 15) / 16), T, 256, exkv::kPage, nsplit, split_len);
        return EXKV_OK;
    }
    const int64_t units = (int64_t)B * Hkv * ((Hq / Hkv + 15) / 16);
    plan_core(units, T, D == 64 && units < 512 ? 768 : 512, 64, nsplit, split_len);
    return EXKV_OK;
}
