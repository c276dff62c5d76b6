"""Decode attention over either cache type, for one query token per sequence
(drop-in for the reference's exactkv/attention.py:6-15)."""
from .cache import CompressedKV, BF16KV
from .paged import PagedCompressedKV, PagedBF16KV
from .kernels import attention_compressed, attention_reference


def decode_attention(q, k_cache, v_cache, **kw):
    """q: [B, Hq, D] bf16 contiguous (after RoPE). k_cache / v_cache: both CompressedKV or both BF16KV
    (or both PagedCompressedKV / PagedBF16KV of one PageTable, q row i being the current
    step's slot i), already holding the current token. Returns [B, Hq, D] bf16.

    The two cache types give bit-identical results for the same contents and split plan."""
    if isinstance(k_cache, (PagedCompressedKV, PagedBF16KV)):
        _, bt, lens = k_cache.table.step_rows()          # row i of q is the step's slot i
        if isinstance(k_cache, PagedCompressedKV):
            return attention_compressed(q, k_cache.buffers(), v_cache.buffers(), 0, lens=lens, block_table=bt, **kw)
        return attention_reference(q, k_cache.buf, v_cache.buf, 0, lens=lens, block_table=bt, **kw)
    if isinstance(k_cache, CompressedKV):
        return attention_compressed(q, k_cache, v_cache, k_cache.T, **kw)
    if isinstance(k_cache, BF16KV):
        return attention_reference(q, k_cache.buf, v_cache.buf, k_cache.T, **kw)
    raise TypeError(type(k_cache))
