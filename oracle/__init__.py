"""CPU oracle for the compressed-KV decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU in numpy, the algorithms of the reference
implementation (zyfyz666/exactkv) that the HIP path must reproduce:

  oracle.codec      the byte format: encode / decode / bits_per_value
                    (reference exactkv/codec.py:31-78)
  oracle.attention  GQA decode attention in fp32 / fp64 and the split-K plan and
                    merge algebra (reference exactkv/kernels.py:33-59, 273-277)
  oracle.cache      the CompressedKV bookkeeping protocol: tail area, open page,
                    deterministic raw slots, pool growth
                    (reference exactkv/cache.py:17-158)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or as the timed CPU baseline. The product
path (exactkv_amd) never imports it and has no CPU fallback.

How each function is pinned (beyond restating the reference):
  codec.encode / decode   golden vectors written by the reference codec itself
                          (tests/golden/), round trip of all 65,536 bf16 patterns,
                          closed-form pages (zeros, constants, inf/nan, lone zero),
                          and a brute-force per-group check that an element is
                          escaped exactly when no 4-bit code decodes to it.
  attention.attention     torch.nn.functional.scaled_dot_product_attention in
                          float64 on the CPU, uniform-key and one-hot closed forms.
  attention.choose_split  closed-form integer cases of the reference planner.
  attention.merge_splits  invariance: any split of the tokens merges to the
                          unsplit result.
  cache.CacheModel        decoded contents equal the plain bf16 cache after every
                          append and growth; full-page prefill equals codec.encode.
"""
