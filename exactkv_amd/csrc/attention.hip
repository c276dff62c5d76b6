// Split-K GQA decode attention for gfx950, over the compressed cache or over plain bf16.
//
// Reference: exactkv/kernels.py _split_c_kernel :142-165, _split_ref_kernel :168-194,
// _attn_block :46-59, _reduce_kernel :33-43.
//
// Grid: x = token split, y = (sequence, KV head, group of 16 query heads). A workgroup is
// 4 wavefronts; they take the split's 32-token chunks round robin, each with its own
// online-softmax state, and are merged through LDS at the end (one partial per split).
//
// Per chunk, per wavefront (two 16-token pages):
//   * K and V pages are loaded as 16-byte vectors and rebuilt bit-exactly in VGPRs
//     (tile.hpp); the bf16 twin loads the same 32 values per lane from a bf16 cache.
//     Everything after the loader is shared, so the two kernels give identical bits.
//   * S^T = K Q^T with v_mfma_f32_16x16x32_bf16: tokens are the MFMA rows (the rebuilt
//     registers are already the A operand), the G query heads of the KV head are the
//     columns (padded to 16).
//   * Online softmax in base 2 on the MFMA output (lane = one head, 8 tokens), scores
//     scaled by D^-1/2 log2(e), p rounded to bf16 for P.V, l summed from fp32 p.
//   * O^T += V^T P^T with the same MFMA: the C layout of S^T is exactly the B-operand
//     layout of P^T, and V^T comes from a per-wavefront LDS tile written transposed by
//     the rebuilding lanes. The accumulator stays in the (lane = head) layout, so the
//     softmax rescale needs no cross-lane traffic.
#include "tile.hpp"
#include "../../include/exactkv.h"

namespace exkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kChunk = 32;
constexpr int kVtStride = 40;   // halfwords per row of the transposed V tile (32 slots + pad)

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
    float qk_scale;
};

__device__ inline bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 u = {a, b, c, d};
    return __builtin_bit_cast(bf16x8, u);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <bool COMP>
__global__ void __launch_bounds__(256) attn_split_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[kWaves * kD * kVtStride];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
    const int split = blockIdx.x;
    int y = blockIdx.y;
    const int hg = y % a.HG;
    y /= a.HG;
    const int hk = y % a.Hkv;
    const int b = y / a.Hkv;
    int len = a.lens ? a.lens[b * a.lens_stride] : a.T;
    len = min(max(len, 0), a.TS);
    const int start = split * a.split_len;
    const int end = min(start + a.split_len, len);
    const int NP = a.TS / kPage;

    // Q^T as the B operand: column = head hg*16 + r of this KV head's group, k-block kc
    // holds channels 16g + 8kc.. (kc < 2) or 64 + 16g + 8(kc-2).. (kc >= 2).
    const int hl = hg * 16 + r;
    bf16x8 qop[4];
    {
        const uint16_t* qp = a.q + ((int64_t)b * a.Hq + (int64_t)hk * a.G + min(hl, a.G - 1)) * kD;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
            const int d0 = kc < 2 ? 16 * g + 8 * kc : 64 + 16 * g + 8 * (kc - 2);
            u32x4 v = {0u, 0u, 0u, 0u};
            if (hl < a.G) v = *reinterpret_cast<const u32x4*>(qp + d0);
            qop[kc] = __builtin_bit_cast(bf16x8, v);
        }
    }

    float m_i = -INFINITY, l_i = 0.f;
    f32x4 acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint16_t* vt = lds + wave * kD * kVtStride;
    const int nchunks = end > start ? (end - start + kChunk - 1) / kChunk : 0;
    const int slot0 = 8 * (r >> 2) + (r & 3);

    for (int c = wave; c < nchunks; c += kWaves) {
        const int t0 = start + c * kChunk;
        uint32_t kd[2][16], vd[2][16];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int pg = (t0 >> 4) + s;
            if (pg * kPage < end) {
                const int64_t row = ((int64_t)b * a.TS + pg * kPage + r) * a.Hkv + hk;
                if constexpr (COMP) {
                    const int64_t page = ((int64_t)b * NP + pg) * a.Hkv + hk;
                    PageBytes pk, pv;
                    load_page(a.k, row, page, g, pk);
                    load_page(a.v, row, page, g, pv);
                    rebuild_page(a.k, pk, r, g, kd[s]);
                    rebuild_page(a.v, pv, r, g, vd[s]);
                } else {
                    load_bf16_row(a.kb, row, g, kd[s]);
                    load_bf16_row(a.vb, row, g, vd[s]);
                }
                if (pg * kPage + r >= end) {          // rows past the end: zero (as masked loads)
#pragma unroll
                    for (int i = 0; i < 16; ++i) kd[s][i] = vd[s][i] = 0u;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) kd[s][i] = vd[s][i] = 0u;
            }
        }

        // scores: lane holds head r, tokens t0 + 16s + 4g + i
        float sc[8];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            f32x4 sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < 4; ++kc)
                sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(kd[s][4 * kc], kd[s][4 * kc + 1], kd[s][4 * kc + 2], kd[s][4 * kc + 3]), qop[kc], sa,
                    0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = t0 + 16 * s + 4 * g + i;
                sc[4 * s + i] = tok < end ? sa[i] * a.qk_scale : -INFINITY;
            }
        }
        float mloc = sc[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mloc = fmaxf(mloc, sc[i]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_i, mloc);
        const float alpha = fast_exp2(m_i - m_new);
        float psum = 0.f;
        bf16x8 pop;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p = fast_exp2(sc[i] - m_new);
            psum += p;
            pop[i] = (__bf16)p;
        }
        l_i = l_i * alpha + psum;
        m_i = m_new;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb] *= alpha;

        // V^T into LDS: row = channel, slot = 8(r/4) + 4s + r%4 (the P^T k order)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            uint16_t* col = vt + slot0 + 4 * s;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int d = (k < 8 ? 16 * g : 64 + 16 * g - 16) + 2 * k;
                col[d * kVtStride] = (uint16_t)vd[s][k];
                col[(d + 1) * kVtStride] = (uint16_t)(vd[s][k] >> 16);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const u32x4 av = *reinterpret_cast<const u32x4*>(vt + (16 * nb + r) * kVtStride + 8 * g);
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), pop, acc[nb], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // merge the 4 wavefronts' states (same algebra as the split merge)
    float l_t = l_i + __shfl_xor(l_i, 16);
    l_t = l_t + __shfl_xor(l_t, 32);
    __syncthreads();
    float* mo = reinterpret_cast<float*>(lds);            // [wave][16 heads][128]
    float* mm = mo + kWaves * 16 * kD;                     // [wave][16]
    float* ml = mm + kWaves * 16;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
        *reinterpret_cast<f32x4*>(mo + (wave * 16 + r) * kD + 16 * nb + 4 * g) = acc[nb];
    if (g == 0) {
        mm[wave * 16 + r] = m_i;
        ml[wave * 16 + r] = l_t;
    }
    __syncthreads();
    const int gh = min(16, a.G - hg * 16);
    for (int idx = threadIdx.x; idx < gh * kD; idx += 256) {
        const int h = idx >> 7, d = idx & (kD - 1);
        float M = mm[h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, mm[w * 16 + h]);
        float o = 0.f, l = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float wt = fast_exp2(mm[w * 16 + h] - M);
                o += wt * mo[(w * 16 + h) * kD + d];
                l += wt * ml[w * 16 + h];
            }
        }
        const int64_t prow = ((int64_t)b * a.Hq + (int64_t)hk * a.G + hg * 16 + h) * a.nsplit + split;
        a.part_o[prow * kD + d] = o;
        if (d == 0) {
            a.part_m[prow] = M;
            a.part_l[prow] = l;
        }
    }
}

// out[row] = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s  (kernels.py:33-43)
__global__ void __launch_bounds__(64) attn_reduce_kernel(const float* po, const float* pm, const float* pl,
                                                         uint16_t* out, int ns) {
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    const float* m = pm + row * ns;
    const float* l = pl + row * ns;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, m[s]);
    float n0 = 0.f, n1 = 0.f, den = 0.f;
    for (int s = 0; s < ns; ++s) {
        const float w = fast_exp2(m[s] - M);
        const float2 o = reinterpret_cast<const float2*>(po + (row * ns + s) * kD)[lane];
        n0 += o.x * w;
        n1 += o.y * w;
        den += l[s] * w;
    }
    __bf16 r0 = (__bf16)(n0 / den), r1 = (__bf16)(n1 / den);
    const uint32_t packed = (uint32_t)__builtin_bit_cast(uint16_t, r0) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
    reinterpret_cast<uint32_t*>(out + row * kD)[lane] = packed;
}

}  // namespace exkv

using namespace exkv;

static int check_attn(int B, int Hq, int Hkv, int D, int T, int TS, const int32_t* lens, int nsplit,
                      int split_len) {
    EXKV_REQUIRE(D == kD, "attention: head dim must be 128 (got %d)", D);
    EXKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "attention: bad heads Hq=%d Hkv=%d (B=%d)", Hq,
                 Hkv, B);
    EXKV_REQUIRE(TS > 0 && TS % kPage == 0, "attention: TS=%d must be a positive multiple of 16", TS);
    EXKV_REQUIRE(nsplit > 0 && split_len > 0 && split_len % kChunk == 0,
                 "attention: split_len=%d must be a positive multiple of 32 (nsplit=%d)", split_len, nsplit);
    if (lens == nullptr) {
        EXKV_REQUIRE(T >= 1 && T <= TS, "attention: T=%d outside [1, TS=%d]", T, TS);
        EXKV_REQUIRE((int64_t)nsplit * split_len >= T, "attention: %d splits of %d do not cover T=%d", nsplit,
                     split_len, T);
    } else {
        EXKV_REQUIRE((int64_t)nsplit * split_len >= TS,
                     "attention: with per-sequence lengths the splits must cover TS=%d", TS);
    }
    EXKV_REQUIRE((int64_t)B * Hkv * ((Hq / Hkv + 15) / 16) < 65536, "attention: too many (sequence, head) units");
    return EXKV_OK;
}

static int launch_split(bool comp, const AttnArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)a.nsplit, (unsigned)(a.B * a.Hkv * a.HG));
    if (comp)
        hipLaunchKernelGGL(attn_split_kernel<true>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(attn_split_kernel<false>, grid, dim3(256), 0, stream, a);
    return hip_status(hipGetLastError(), comp ? "attn_split_compressed" : "attn_split_bf16");
}

static int launch_reduce(const float* o, const float* m, const float* l, void* out, int64_t rows, int ns,
                         hipStream_t stream) {
    hipLaunchKernelGGL(attn_reduce_kernel, dim3((unsigned)rows), dim3(64), 0, stream, o, m, l, (uint16_t*)out, ns);
    return hip_status(hipGetLastError(), "attn_reduce");
}

static int fill_compressed(AttnArgs& a, const void* q, const void* k_sm, const void* k_code, const void* k_base,
                           const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw, int64_t k_raw_rows,
                           const void* v_sm, const void* v_code, const void* v_base, const int32_t* v_rowmask,
                           const int32_t* v_rowoff, const void* v_raw, int64_t v_raw_rows, float* ws_o,
                           float* ws_m, float* ws_l, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T,
                           int32_t TS, const int32_t* lens, int64_t lens_stride, int32_t nsplit,
                           int32_t split_len, float qk_scale) {
    const int rc = check_attn(B, Hq, Hkv, D, T, TS, lens, nsplit, split_len);
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
    a.nsplit = nsplit; a.split_len = split_len; a.qk_scale = qk_scale;
    return EXKV_OK;
}

static int fill_bf16(AttnArgs& a, const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                     float* ws_l, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                     const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len, float qk_scale) {
    const int rc = check_attn(B, Hq, Hkv, D, T, TS, lens, nsplit, split_len);
    if (rc) return rc;
    EXKV_REQUIRE(q && k && v && ws_o && ws_m && ws_l, "attn_bf16: null pointer");
    a = AttnArgs{};
    a.q = (const uint16_t*)q;
    a.kb = (const uint16_t*)k; a.vb = (const uint16_t*)v;
    a.part_o = ws_o; a.part_m = ws_m; a.part_l = ws_l;
    a.lens = lens; a.lens_stride = lens_stride;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.HG = (a.G + 15) / 16; a.TS = TS; a.T = T;
    a.nsplit = nsplit; a.split_len = split_len; a.qk_scale = qk_scale;
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
        int32_t nsplit, int32_t split_len, float qk_scale
#define EXKV_SHAPE_ARGS B, Hq, Hkv, D, T, TS, lens, lens_stride, nsplit, split_len, qk_scale

extern "C" int exkv_attn_compressed(EXKV_C_PARAMS, void* out, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_compressed: null output");
    rc = launch_split(true, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, stream);
}

extern "C" int exkv_attn_split_compressed(EXKV_C_PARAMS, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    const int rc = fill_compressed(a, EXKV_C_ARGS, EXKV_SHAPE_ARGS);
    return rc ? rc : launch_split(true, a, stream);
}

extern "C" int exkv_attn_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m, float* ws_l,
                              void* out, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    int rc = fill_bf16(a, q, k, v, ws_o, ws_m, ws_l, EXKV_SHAPE_ARGS);
    if (rc) return rc;
    EXKV_REQUIRE(out, "attn_bf16: null output");
    rc = launch_split(false, a, stream);
    return rc ? rc : launch_reduce(ws_o, ws_m, ws_l, out, (int64_t)B * Hq, nsplit, stream);
}

extern "C" int exkv_attn_split_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m,
                                    float* ws_l, EXKV_SHAPE_PARAMS, hipStream_t stream) {
    AttnArgs a;
    const int rc = fill_bf16(a, q, k, v, ws_o, ws_m, ws_l, EXKV_SHAPE_ARGS);
    return rc ? rc : launch_split(false, a, stream);
}

extern "C" int exkv_attn_reduce(const float* ws_o, const float* ws_m, const float* ws_l, void* out, int64_t rows,
                                int32_t nsplit, int32_t D, hipStream_t stream) {
    EXKV_REQUIRE(D == kD, "attn_reduce: head dim must be 128 (got %d)", D);
    EXKV_REQUIRE(rows > 0 && nsplit > 0, "attn_reduce: bad rows=%lld nsplit=%d", (long long)rows, nsplit);
    EXKV_REQUIRE(ws_o && ws_m && ws_l && out, "attn_reduce: null pointer");
    return launch_reduce(ws_o, ws_m, ws_l, out, rows, nsplit, stream);
}
