"""exactkv_amd: keys and values of a decoding LLM held in exactkv's compressed page format
(every bf16 bit kept), with a gfx950 decode-attention kernel that rebuilds pages on the fly
from that format. All kernels are hand-written HIP behind the reference's Python names, so
code written against zyfyz666/exactkv runs unchanged.

    import exactkv_amd as exactkv
"""
from .cache import CompressedKV, BF16KV, check_overflow
from .attention import decode_attention
from .paged import PageTable, PagedCompressedKV, PagedBF16KV
from .codec import encode_reference, decode_reference, bits_per_value
from .kernels import attention_compressed, attention_reference, decode_to_bf16, encode_pages


def __getattr__(name):
    if name in ("Engine", "PagedEngine"):   # imports transformers-side helpers lazily
        from . import engine
        return getattr(engine, name)
    raise AttributeError(name)


__version__ = "0.1.0"
__all__ = ["CompressedKV", "BF16KV", "check_overflow", "decode_attention", "Engine",
           "encode_reference", "decode_reference", "bits_per_value",
           "attention_compressed", "attention_reference", "decode_to_bf16", "encode_pages",
           "PageTable", "PagedCompressedKV", "PagedBF16KV", "PagedEngine"]
