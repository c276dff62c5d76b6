/* exactkv on MI355X -- C ABI of libexactkv_hip.so (gfx950).
 *
 * The drop-in boundary of the compressed-KV decode path. Each entry point replaces one
 * launch site of the reference (zyfyz666/exactkv, Python + Triton); the reference file:line
 * it stands in for is given above each declaration.
 *
 * Conventions
 *   - All pointers are device pointers (HIP), except the outputs of the split planners.
 *   - Work is enqueued on `stream` only; nothing synchronizes, nothing allocates, so
 *     calls can be captured in a HIP graph. The library's one piece of device state is
 *     exkv_attn_compressed_noalloc's fixed scratch array on each GPU it runs on.
 *   - bf16 tensors are passed as raw 16-bit patterns. Tensors are row-major with the
 *     shapes given; "elements" strides count bf16 elements.
 *   - Return value: 0 ok, 1 invalid argument, 2 HIP launch error; exkv_last_error()
 *     returns the message of the last failure on the calling thread.
 *   - Pages hold 16 tokens. Head dim D is 64, 128 or 256 in every entry point that takes
 *     one (the wire form: 128); the reference builds 128 only (cache.py:21), its codec
 *     any D (code byte j holds channels j and j + D/2).
 *   - Compressed cache of one layer's keys or values (reference cache.py:24-32):
 *       sm [B, TS, H, D] u8, code [B, TS, H, D/2] u8, base [B, TS/16, H, D] u8,
 *       rowmask, rowoff [B, TS/16, H] i32, raw [raw_rows, D] bf16 with
 *       raw_rows = cap + B*H*16 (rows that do not fit | open-page tail area),
 *       cnt / before: i32 pool counter and its value before the last encode.
 */
#ifndef EXACTKV_H
#define EXACTKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* ABI version of the library (2: the encoders take a scan workspace; 3: head dims 64 and
 * 256 and exkv_plan_splits_hd; 4: exkv_error_bits and exkv_set_wait_limit). */
int exkv_abi_version(void);

/* Sticky error bits of the kernels. A kernel that gives up a bounded wait (a correct call
 * never reaches the bound) or clamps an index that a broken invariant put out of bounds
 * (say, attention over a page whose raw rows overflowed the pool before check_overflow
 * repaired it) carries on -- no access leaves its buffers -- but its results are then not
 * the format's bits although the call returned 0; it records that by OR-ing a bit into
 * an error word that the library keeps on the GPU (one per kernel source file, zero when
 * the library loads). */
#define EXKV_ERR_WAIT 0x1u      /* attention: a wait on another wavefront's LDS flag gave up */
#define EXKV_ERR_RAW_SLOT 0x2u  /* attention, decode: a raw row's pool slot lay outside the pool */
#define EXKV_ERR_LOOKBACK 0x4u  /* encoder: the slot scan's look-back gave up on a predecessor */
#define EXKV_ERR_SCAN_WS 0x8u   /* encoder: an inconsistent scan workspace (more blocks than tickets) */
#define EXKV_ERR_WIRE 0x10u     /* wire pack: a raw row's pool slot lay outside the pool */

/* out (a device uint32 on the GPU of `stream`) = the OR of the error words of that GPU, in
 * stream order (three small kernels; nothing synchronizes, nothing is allocated); clear != 0
 * resets the words. Bits set by kernels on other streams of the GPU are included once they
 * have completed.
 * No counterpart in the reference, whose one such condition, raw-pool overflow, is a
 * counter the host reads (cache.py:149-158); that protocol is unchanged here. */
int exkv_error_bits(uint32_t* out, int32_t clear, hipStream_t stream);

/* Test hook: the bound, in polls, of every wait of the split kernels on another wavefront's
 * LDS flag, for the attention calls the calling thread makes afterwards (<= 0: the default,
 * 2^22 polls, which a correct call never reaches). A tiny bound makes those waits give up
 * (the call then returns garbage and sets EXKV_ERR_WAIT; every access stays in bounds and
 * the kernel ends normally), so a test can check that a give-up is reported.
 * No counterpart in the reference. */
int exkv_set_wait_limit(int32_t polls);

/* Message of the last failed call on this thread. */
const char* exkv_last_error(void);

/* Page encoder: encode nb sequences x npg pages x H heads of `src` (bf16, element strides
 * s_b, s_pg, s_p, s_h for sequence, page, token-in-page, head; channels contiguous) into
 * pages [pg0, pg0+npg) of sequences [b0, b0+nb) of the cache. Raw rows get pool slots
 * *cnt + running count in (sequence, page, head, token) order; rows whose slot is >= cap
 * are not written, and *cnt advances by the call's total (overflow = *cnt > cap).
 * *before (may be NULL) receives the counter's value before the call.
 * scan_ws (8-byte aligned, may be NULL): a workspace of scan_ws_words 64-bit words, all zero
 * when first used and reserved for this library's encodes on one stream; with at least
 * 2 + ceil(nb*npg*H / 1024) words the encode is two launches (the page kernel, then one
 * chained slot scan), else four (the page kernel, then a three-launch scan). Same bytes
 * either way.
 * Replaces: kernels.py:340-346 encode_pages (launch of _encode_pages_kernel :233-268),
 * byte-identical to codec.py:31-55 encode_reference. */
int exkv_encode_pages(const void* src, int64_t s_b, int64_t s_pg, int64_t s_p, int64_t s_h,
                      void* sm, void* code, void* base, int32_t* rowmask, int32_t* rowoff, void* raw,
                      int32_t* cnt, int32_t* before, int64_t cap, int64_t raw_rows, int32_t B,
                      int32_t b0, int32_t pg0, int32_t nb, int32_t npg, int32_t H, int32_t TS,
                      int32_t D, void* scan_ws, int64_t scan_ws_words, hipStream_t stream);

/* The page encoder into a paged cache: page pg of source sequence bi goes to page
 * dst_pages[bi*dst_stride + pg] of the B x TS arrays read as a list of B*TS/16 pages (entries
 * clamped to it). Same bytes and raw-slot order as exkv_encode_pages, and the same scan
 * workspace.
 * No counterpart in the reference (contiguous caches only); paged KV is in its future
 * work (README.md:121-123). */
int exkv_encode_pages_paged(const void* src, int64_t s_b, int64_t s_pg, int64_t s_p, int64_t s_h,
                            void* sm, void* code, void* base, int32_t* rowmask, int32_t* rowoff, void* raw,
                            int32_t* cnt, int32_t* before, int64_t cap, int64_t raw_rows, int32_t B,
                            const int32_t* dst_pages, int64_t dst_stride, int32_t nb, int32_t npg, int32_t H,
                            int32_t TS, int32_t D, void* scan_ws, int64_t scan_ws_words, hipStream_t stream);

/* Append one token per sequence (x: [B, H, D] bf16, row strides sx_b, sx_h) to the cache
 * whose token count is state[0] (device): write it into the tail area; when it completes
 * page T/16, encode that page (slots as above, *before = counter before) and open the next
 * page (rowmask 0xFFFF, rowoff into the tail area); then state[0] += 1. Nothing is written
 * once state[0] == TS. One launch: state[1] is its arrival counter (zero before the first
 * call; each call leaves it zero), so state points to at least two words.
 * Replaces: cache.py:100-112 CompressedKV.append (tail write + _encode + _open_tail). */
int exkv_cache_append(const void* x, int64_t sx_b, int64_t sx_h, void* sm, void* code, void* base,
                      int32_t* rowmask, int32_t* rowoff, void* raw, int32_t* cnt, int32_t* before,
                      int32_t* state, int64_t cap, int64_t raw_rows, int32_t B, int32_t H, int32_t TS,
                      int32_t D, hipStream_t stream);

/* Append to a plain bf16 cache buf [B, TS, H, D] at position state[0]; state[0] += 1.
 * Replaces: cache.py:141-143 BF16KV.append. */
int exkv_bf16_append(const void* x, int64_t sx_b, int64_t sx_h, void* buf, int32_t* state, int32_t B,
                     int32_t H, int32_t TS, int32_t D, hipStream_t stream);

/* Append one token for each of n sequences of a paged cache: a pool of pool_pages pages
 * (arrays as a [1, 16 * pool_pages, H, D] cache) shared by max_seqs sequence slots.
 * Batch row i is slot slots[i] (slots == NULL: slot i; the slots must differ); slot s owns
 * pool pages block_table[s * bt_stride + pg] (pg < max_pages, entries clamped to the
 * pool) and holds lens[s] tokens, the new one included (the caller raises lens first; the
 * call never writes it). Slot s's open page is held in the tail area at raw rows
 * cap + (s * H + h) * 16 (raw_rows >= cap + max_seqs * H * 16). When the new token
 * fills page pg, that page is encoded into its pool page (raw slots in (row, head, token)
 * order from *cnt, *before = counter before) and table entry pg + 1, which the caller
 * has filled, is opened (rowmask 0xFFFF, rowoff into the tail area).
 * No counterpart in the reference (contiguous caches only); paged KV is in its future
 * work (README.md:121-123). The per-sequence steps are those of cache.py:100-112. */
int exkv_cache_append_paged(const void* x, int64_t sx_b, int64_t sx_h, void* sm, void* code, void* base,
                            int32_t* rowmask, int32_t* rowoff, void* raw, int32_t* cnt, int32_t* before,
                            int64_t cap, int64_t raw_rows, const int32_t* slots, const int32_t* lens,
                            const int32_t* block_table, int64_t bt_stride, int32_t n, int32_t H,
                            int32_t max_seqs, int32_t max_pages, int32_t pool_pages, int32_t D,
                            hipStream_t stream);

/* bf16 twin of exkv_cache_append_paged over a pool buf [16 * pool_pages, H, D]: token
 * lens[s] - 1 of slot s goes to row (block_table[s, t / 16] * 16 + t % 16).
 * No counterpart in the reference (see exkv_cache_append_paged). */
int exkv_bf16_append_paged(const void* x, int64_t sx_b, int64_t sx_h, void* buf, const int32_t* slots,
                           const int32_t* lens, const int32_t* block_table, int64_t bt_stride, int32_t n,
                           int32_t H, int32_t max_seqs, int32_t max_pages, int32_t pool_pages, int32_t D,
                           hipStream_t stream);

/* Open the page holding token state[0] (device) of every (sequence, head) of a contiguous
 * compressed cache: rowmask = 0xFFFF, rowoff = cap + (b * H + h) * 16 (its rows in the
 * tail area after the cap escaped-row slots). Nothing when state[0] >= TS. Called when a
 * cache is filled and after its raw pool moves (growth), so the page index and offsets are
 * worked out on the device.
 * Replaces: cache.py:54-56 _open_tail and the open-page fix-up of cache.py:70-71 (host-side
 * indexing of rowmask / rowoff by the host token count). */
int exkv_cache_open_page(int32_t* rowmask, int32_t* rowoff, const int32_t* state, int64_t cap, int64_t raw_rows,
                         int32_t B, int32_t H, int32_t TS, hipStream_t stream);

/* The same for a paged cache: for each sequence slot s = slots[i] (i < n), table entry
 * lens[s] / 16 (if < max_pages) of block_table is opened with its rows at
 * cap + (s * H + h) * 16. No counterpart in the reference (contiguous caches only; see
 * exkv_cache_append_paged). */
int exkv_cache_open_pages_paged(int32_t* rowmask, int32_t* rowoff, const int32_t* slots, int32_t n,
                                const int32_t* lens, const int32_t* block_table, int64_t bt_stride, int32_t max_seqs,
                                int32_t max_pages, int32_t pool_pages, int64_t cap, int64_t raw_rows, int32_t H,
                                hipStream_t stream);

/* Number of int32 arrival counters ws_cnt must hold for the merge in the split kernel's tail
 * (units x (groups + 1)), or -1 for arguments with no fused merge (nsplit > 1024).
 * Replaces: the workspace sizing of kernels.py:280-290 (_WS), for the counters. */
int64_t exkv_merge_counters(int32_t B, int32_t Hq, int32_t Hkv, int32_t nsplit);

/* Timing hook: the next split-kernel launch on the calling thread (any exkv_attn_* entry
 * point) records `start` and `stop` (hipEvent_t, created by the caller; either may be NULL)
 * at its own start and end, so a benchmark reads that kernel's duration from HIP events on
 * the launch stream. One launch consumes the pair. No counterpart in the reference (its
 * benchmark times whole calls with triton.testing.do_bench, bench/attention.py:72-78). */
typedef struct ihipEvent_t* hipEvent_t;
int exkv_time_next_split(hipEvent_t start, hipEvent_t stop);

/* Wire form of a sequence's compressed cache: one contiguous little-endian blob
 *   header  256 B: u32 magic 0x564B5845 ("EXKV"), version 1, heads H, head_dim 128,
 *           tokens T, full_pages T/16, tail_rows T%16, raw_rows N; u64 off_tail,
 *           off_rowmask, off_base, off_sm, off_code, off_raw, total; zeros
 *   tail bf16 [T%16, H, 128] | rowmask i32 [T/16, H] | base u8 [T/16, H, 128] |
 *   sm u8 [16*(T/16), H, 128] | code u8 [16*(T/16), H, 64] | raw bf16 [N, 128]
 * each section at a multiple of 256 B (gaps zero); raw rows in (page, head, token) order,
 * rowoff implicit (running count of raw rows in (page, head) order).
 * No counterpart in the reference (its buffers(), cache.py:121-123, hands out the six
 * tensors); a wire form for offload/transfer is in its future work. */

/* Blob size for H heads, T tokens and N raw rows (-1 for bad arguments). */
int64_t exkv_wire_bytes(int32_t H, int32_t T, int64_t raw_rows);

/* Pack nseq sequences of one compressed cache (arrays as above, pool_pages pages of
 * 16 tokens) into one blob each. Sequence s has tokens[s] (<= max_tokens) tokens; its page
 * p is pool page pages[s * page_stride + p] (entries clamped to the pool); its open page's
 * row r of head h is raw row tail_rows[s] + h*16 + r. blobs[s] (device address, 256-byte
 * aligned) has blob_bytes[s] >= exkv_wire_bytes(H, tokens[s], N_s) bytes for the sequence's
 * N_s raw rows (rows past blob_bytes[s] are not written). ws: int32 scratch
 * [nseq, ws_stride], ws_stride >= (max_tokens/16)*H + 3. Two launches; a sequence whose
 * tokens or blob size do not fit is skipped. */
int exkv_wire_pack(const void* sm, const void* code, const void* base, const int32_t* rowmask,
                   const int32_t* rowoff, const void* raw, int64_t raw_rows, int64_t pool_pages, int32_t nseq,
                   const int32_t* pages, int64_t page_stride, const int32_t* tokens, const int64_t* tail_rows,
                   const uint64_t* blobs, const int64_t* blob_bytes, int32_t max_tokens, int32_t H, int32_t D,
                   int32_t* ws, int64_t ws_stride, hipStream_t stream);

/* Unpack nseq blobs into sequences of a compressed cache (arguments as for exkv_wire_pack;
 * the blob's header must give heads H, head_dim 128 and tokens[s], else it is skipped).
 * Raw rows take pool slots from *cnt on, blob after blob, each blob's rows in its
 * (page, head, token) order; *before = the counter before, *cnt += the rows the headers
 * declare; slots >= cap are dropped (overflow shows in the counter, as for
 * exkv_encode_pages). The open page's rows go to raw rows tail_rows[s] + h*16 + r (which
 * must lie in the tail area, at or past cap), and if open[s], page
 * pages[s * page_stride + tokens[s]/16] is opened (rowmask 0xFFFF, rowoff into the tail
 * area). */
int exkv_wire_unpack(void* sm, void* code, void* base, int32_t* rowmask, int32_t* rowoff, void* raw,
                     int64_t raw_rows, int64_t cap, int32_t* cnt, int32_t* before, int64_t pool_pages, int32_t nseq,
                     const int32_t* pages, int64_t page_stride, const int32_t* tokens, const int32_t* open,
                     const int64_t* tail_rows, const uint64_t* blobs, const int64_t* blob_bytes,
                     int32_t max_tokens, int32_t H, int32_t D, int32_t* ws, int64_t ws_stride, hipStream_t stream);

/* Compressed cache -> bf16 out [B, T, H, D] through the attention kernels' page decoder.
 * Replaces: kernels.py:331-337 decode_to_bf16 (_dec_only_kernel :197-211). */
int exkv_decode_to_bf16(const void* sm, const void* code, const void* base, const int32_t* rowmask,
                        const int32_t* rowoff, const void* raw, int64_t raw_rows, void* out, int32_t B,
                        int32_t T, int32_t TS, int32_t H, int32_t D, hipStream_t stream);

/* decode_to_bf16 over a paged cache (arrays of pool_pages pages): out [B, T, H, D] holds
 * tokens [0, T) of each sequence b, page p read from pool page block_table[b*bt_stride + p]
 * (entries clamped to the pool; T <= 16*bt_stride). No counterpart in the reference
 * (contiguous caches only; paged KV is in its future work, README.md:121-123). */
int exkv_decode_to_bf16_paged(const void* sm, const void* code, const void* base, const int32_t* rowmask,
                              const int32_t* rowoff, const void* raw, int64_t raw_rows, int64_t pool_pages,
                              const int32_t* block_table, int64_t bt_stride, void* out, int32_t B, int32_t T,
                              int32_t H, int32_t D, hipStream_t stream);

/* Split-K GQA decode attention over compressed K and V caches, then the split merge.
 * q [B, Hq, D] bf16; out [B, Hq, D] bf16; workspace ws_o [B*Hq, nsplit, D],
 * ws_m, ws_l [B*Hq, nsplit] f32, and ws_cnt: exkv_merge_counters(B, Hq, Hkv, nsplit) i32
 * arrival counters, all zero before the first call (each call leaves them zero). With
 * ws_cnt (and nsplit <= 1024) the merge runs inside the split kernel: the last workgroup of
 * each unit merges its splits (one level, with the separate merge's bits, up to 32 splits;
 * beyond, groups of about sqrt(nsplit) splits, then the groups); without it, as a second
 * kernel. Calls that share a workspace must not overlap.
 * Tokens [0, T) of every sequence, or [0, lens[b*lens_stride])
 * when lens != NULL (then nsplit*split_len must cover TS). split_len: a positive multiple
 * of 16.
 * window > 0 (sliding-window attention): only the last `window` of those tokens,
 * [len - window, len); the splits then start at that range's first page, so they need
 * to cover only min(T or TS, window + 15) tokens. window = 0: all tokens. (Additive: the
 * reference has no window, engine.py:26-28.)
 * qk_scale = 128^-1/2 * log2(e). Bit-identical to exkv_attn_bf16 on the decoded contents.
 * Replaces: kernels.py:310-318 attention_compressed (_split_c_kernel :142-165 and
 * _reduce_kernel :33-43). */
int exkv_attn_compressed(const void* q, const void* k_sm, const void* k_code, const void* k_base,
                         const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw,
                         int64_t k_raw_rows, const void* v_sm, const void* v_code, const void* v_base,
                         const int32_t* v_rowmask, const int32_t* v_rowoff, const void* v_raw,
                         int64_t v_raw_rows, float* ws_o, float* ws_m, float* ws_l, int32_t* ws_cnt, void* out,
                         int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                         const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len,
                         int32_t window, float qk_scale, hipStream_t stream);

/* exkv_attn_compressed with no workspace argument and no allocation, for callers that cannot
 * allocate (code under HIP-graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The split partials go to a fixed scratch
 * array in device memory that the library holds on every GPU it runs on, for the life of
 * the process: B * Hq * nsplit partials of (D + 2) floats must fit its
 * exkv_noalloc_scratch_bytes() (32 MiB), i.e. B * Hq * nsplit <= floor(32 MiB / ((D + 2) * 4)):
 * 127,100 at D = 64, 64,527 at D = 128, 32,513 at D = 256; larger calls return 1 with a
 * message. The merge runs as the second kernel. The array used is that of the GPU `stream`
 * belongs to (all tensors must live there); the first call on a GPU looks its address up
 * (not under stream capture: make one call before capturing). Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams or threads) race. Same
 * arguments otherwise, and the same bits as exkv_attn_compressed. */
int exkv_attn_compressed_noalloc(const void* q, const void* k_sm, const void* k_code, const void* k_base,
                                 const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw,
                                 int64_t k_raw_rows, const void* v_sm, const void* v_code, const void* v_base,
                                 const int32_t* v_rowmask, const int32_t* v_rowoff, const void* v_raw,
                                 int64_t v_raw_rows, void* out, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                                 int32_t T, int32_t TS, const int32_t* lens, int64_t lens_stride, int32_t nsplit,
                                 int32_t split_len, int32_t window, float qk_scale, hipStream_t stream);

/* Size in bytes of exkv_attn_compressed_noalloc's per-GPU scratch array. */
int64_t exkv_noalloc_scratch_bytes(void);

/* The same attention over plain bf16 caches k, v [B, TS, Hkv, D].
 * Replaces: kernels.py:321-328 attention_reference (_split_ref_kernel :168-194). */
int exkv_attn_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m, float* ws_l,
                   int32_t* ws_cnt, void* out, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                   const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len,
                   int32_t window, float qk_scale, hipStream_t stream);

/* The two phases of exkv_attn_compressed / exkv_attn_bf16 separately: the split kernel
 * (partials into ws_o, ws_m, ws_l) and the merge of `nsplit` partials per row into
 * out [rows, D] bf16 (rows = B*Hq).
 * Replaces: the _split_c_kernel / _split_ref_kernel launches (kernels.py:316-317, :325-327)
 * and kernels.py:295-299 _reduce (_reduce_kernel :33-43). */
int exkv_attn_split_compressed(const void* q, const void* k_sm, const void* k_code, const void* k_base,
                               const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw,
                               int64_t k_raw_rows, const void* v_sm, const void* v_code, const void* v_base,
                               const int32_t* v_rowmask, const int32_t* v_rowoff, const void* v_raw,
                               int64_t v_raw_rows, float* ws_o, float* ws_m, float* ws_l, int32_t B,
                               int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS, const int32_t* lens,
                               int64_t lens_stride, int32_t nsplit, int32_t split_len, int32_t window, float qk_scale,
                               hipStream_t stream);
int exkv_attn_split_bf16(const void* q, const void* k, const void* v, float* ws_o, float* ws_m, float* ws_l,
                         int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                         const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len,
                         int32_t window, float qk_scale, hipStream_t stream);
int exkv_attn_reduce(const float* ws_o, const float* ws_m, const float* ws_l, void* out, int64_t rows,
                     int32_t nsplit, int32_t D, hipStream_t stream);

/* Paged caches (block tables): the arrays hold a pool of pool_pages 16-token pages, laid out
 * as one sequence ([1, 16*pool_pages, Hkv, ...] and [1, pool_pages, Hkv, ...]), and page p of
 * sequence b is pool page block_table[b*bt_stride + p] (int32; entries are clamped to the
 * pool). T / lens / TS count the sequences' tokens (TS <= 16*bt_stride). Same kernels and
 * bits as the contiguous calls on the same page contents.
 * No counterpart in the reference, which stores [B, TS, ...] only: this is the first item of
 * the paged serving layout its README lists as future work (README.md:121-123). */
int exkv_attn_compressed_paged(const void* q, const void* k_sm, const void* k_code, const void* k_base,
                               const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw,
                               int64_t k_raw_rows, const void* v_sm, const void* v_code, const void* v_base,
                               const int32_t* v_rowmask, const int32_t* v_rowoff, const void* v_raw,
                               int64_t v_raw_rows, float* ws_o, float* ws_m, float* ws_l, int32_t* ws_cnt,
                               void* out, const int32_t* block_table, int64_t bt_stride, int32_t pool_pages,
                               int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                               const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len,
                               int32_t window, float qk_scale, hipStream_t stream);
int exkv_attn_split_compressed_paged(const void* q, const void* k_sm, const void* k_code, const void* k_base,
                                     const int32_t* k_rowmask, const int32_t* k_rowoff, const void* k_raw,
                                     int64_t k_raw_rows, const void* v_sm, const void* v_code, const void* v_base,
                                     const int32_t* v_rowmask, const int32_t* v_rowoff, const void* v_raw,
                                     int64_t v_raw_rows, float* ws_o, float* ws_m, float* ws_l,
                                     const int32_t* block_table, int64_t bt_stride, int32_t pool_pages, int32_t B,
                                     int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                                     const int32_t* lens, int64_t lens_stride, int32_t nsplit,
                                     int32_t split_len, int32_t window, float qk_scale, hipStream_t stream);
int exkv_attn_bf16_paged(const void* q, const void* k, const void* v, float* ws_o, float* ws_m, float* ws_l,
                         int32_t* ws_cnt, void* out, const int32_t* block_table, int64_t bt_stride,
                         int32_t pool_pages, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t T, int32_t TS,
                         const int32_t* lens, int64_t lens_stride, int32_t nsplit, int32_t split_len,
                         int32_t window, float qk_scale, hipStream_t stream);

/* Host-side split plan for MI355X (host pointers out): about target_blocks workgroups
 * (<= 0: 256, one per CU), at least min_split tokens per split (<= 0: 16, one page), split_len
 * a multiple of 32, or 16.
 * Replaces: kernels.py:273-277 choose_split. */
int exkv_plan_splits(int32_t B, int32_t Hkv, int32_t Hq, int32_t T, int32_t target_blocks,
                     int32_t min_split, int32_t* nsplit, int32_t* split_len);

/* The split plan for head dim D (host pointers out): at 128 exkv_plan_splits with its
 * defaults; at 64 with an even Hkv the same plan over Hkv / 2 pairs of KV heads (the
 * attention calls run head dim 64 as pairs of heads with the head-dim-128 kernel
 * structure); at 256, and 64 with an odd Hkv, rounds of 512 of the generic-head-dim
 * kernel's workgroups (one per KV head and group of 16 query heads).
 * No counterpart in the reference (head dim 128 only, cache.py:21). */
int exkv_plan_splits_hd(int32_t B, int32_t Hkv, int32_t Hq, int32_t T, int32_t D, int32_t* nsplit,
                        int32_t* split_len);

#ifdef __cplusplus
}
#endif

#endif /* EXACTKV_H */
