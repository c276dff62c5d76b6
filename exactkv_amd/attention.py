"""decode_attention: one decode step's attention over whichever cache holds the keys and
values (the reference's entry point, exactkv/attention.py:6-15, same name and arguments)."""
from .cache import CompressedKV, BF16KV
from .paged import PagedCompressedKV, PagedBF16KV
from .kernels import attention_compressed, attention_reference


def decode_attention(q, k_cache, v_cache, **kw):
    """Attention of one new query token per sequence over its cached keys and values.

    q: bf16 [B, Hq, D], contiguous, RoPE already applied (D = 64, 128 or 256). k_cache / v_cache: a matching
    pair -- CompressedKV, BF16KV, or PagedCompressedKV / PagedBF16KV of one PageTable (then
    row i of q belongs to the current step's slot i) -- whose appends for this step have
    already run, so the current token is attended to. Extra keywords go to the kernel call
    (window=, nsplit=, split_len=, out=, ...). Returns bf16 [B, Hq, D].

    A compressed pair and a bf16 pair holding the same tokens return the same bits for the
    same split plan. Any other cache type raises TypeError."""
    if isinstance(k_cache, (PagedCompressedKV, PagedBF16KV)):
        _, bt, lens = k_cache.table.step_rows()
        if isinstance(k_cache, PagedCompressedKV):
            return attention_compressed(q, k_cache.buffers(), v_cache.buffers(), 0, lens=lens, block_table=bt, **kw)
        return attention_reference(q, k_cache.buf, v_cache.buf, 0, lens=lens, block_table=bt, **kw)
    if isinstance(k_cache, CompressedKV):
        return attention_compressed(q, k_cache, v_cache, k_cache.T, **kw)
    if isinstance(k_cache, BF16KV):
        return attention_reference(q, k_cache.buf, v_cache.buf, k_cache.T, **kw)
    raise TypeError(type(k_cache))
