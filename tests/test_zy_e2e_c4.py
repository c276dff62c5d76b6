"""Config 4 at its own workload: batched greedy decoding with the engine on a random-init
Llama-3.1-8B (32 layers, hidden 4096, 32q / 8kv, head dim 128, FFN 14336, vocab 128,256,
RoPE theta 5e5, bf16 weights N(0, 0.02)), 4,096-token prompts of uniform random token ids
and 256 greedy tokens per sequence, at the batch the KV budget of the GPU gives the bf16
cache (the reference's rule, bench/e2e.py:54-63: free memory after the weights minus
1.6 GiB, KV per sequence = kv_bytes(B=2) - kv_bytes(B=1); 6 GiB of it kept for the
prefill's activations, the step's logits and the fingerprints). Both caches run that
batch one after the other, and must give the same tokens and bit-identical logits at
every step (the reference's end-to-end check, tests/test_exactkv.py:107-122, at the
benchmark's protocol, bench/e2e.py:66-91).

The logits of a step ([B, 128256] bf16) are compared through per-row fingerprints of
their 16-bit patterns (two weighted sums in wrapping int64 arithmetic), so no step's
logits need to be kept: storing them all would take about 32 GB. On a mismatch the test
names the first decode step and rows where the two runs part.

The file is named to run late in the GPU suite (just before the no-alloc entry point's
tests): it holds the GPU for minutes, and under -x a failure here stops no other test."""
import gc

import pytest
import torch

import exactkv_amd as exactkv

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

LLAMA31_8B = dict(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                  num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072, rope_theta=5e5,
                  rms_norm_eps=1e-5, initializer_range=0.02, tie_word_embeddings=False)
PROMPT, NEW = 4096, 256
HEADROOM_GIB, WORK_GIB = 1.6, 6.0
CHUNK = 64                                  # sequences per prefill call


def _say(capsys, *a):
    with capsys.disabled():                 # progress on the terminal while the test runs
        print("[c4]", *a, flush=True)


def _fingerprint(logits, w):
    """[B, 2] int64: sum over the vocabulary of bits * w[j] for the two weight rows of w
    (products and sums wrap modulo 2**64, the same on every run)."""
    x = logits.contiguous().view(torch.int16).to(torch.int64)
    return torch.stack([(x * w[0]).sum(-1), (x * w[1]).sum(-1)], dim=1)


def _run(model, backend, B, ids, w, capsys):
    eng = exactkv.Engine(model, B, PROMPT + NEW, backend=backend)
    first = []
    for b0 in range(0, B, CHUNK):
        first.append(eng.prefill(ids[b0:min(B, b0 + CHUNK)], b0=b0))
        _say(capsys, backend, f"B={B}: prefilled {min(B, b0 + CHUNK)}")
    t = torch.cat(first)
    toks, fps = [t], []
    for s in range(NEW - 1):
        logits = eng.step(t)
        fps.append(_fingerprint(logits, w))
        t = logits.argmax(-1)
        toks.append(t)
        if s % 64 == 63:
            _say(capsys, backend, f"B={B}: step {s + 1}")
    torch.cuda.synchronize()
    assert eng.use_graph and eng.captures >= 1
    grows, T = eng.grows, eng.kv[0][0].T
    del eng, logits
    gc.collect()
    torch.cuda.empty_cache()
    return torch.stack(toks, 1).cpu(), torch.stack(fps).cpu(), grows, T


def _where_they_part(tok_b, tok_c, fp_b, fp_c):
    """The first decode step whose logits differ (fp: [steps, B, 2]), the rows there, and the
    first token position where the greedy tokens differ (tok: [B, NEW])."""
    rows = (fp_b != fp_c).any(-1)                      # [steps, B]
    steps = rows.any(-1).nonzero().flatten().tolist()
    toks = (tok_b != tok_c).any(0).nonzero().flatten().tolist()
    if not steps:
        return f"logits equal at every step; tokens first differ at position {toks[:1]}"
    s = steps[0]
    r = rows[s].nonzero().flatten().tolist()
    return (f"logits first differ at decode step {s} (token position {s + 1}) in {len(r)} rows {r[:8]}; "
            f"{len(steps)} steps differ; tokens first differ at position {toks[:1]}")


def test_c4_llama31_8b_full_workload_tokens_and_logits(capsys):
    from transformers import LlamaConfig, LlamaForCausalLM
    gc.collect()
    torch.cuda.empty_cache()
    torch.manual_seed(0)
    with torch.device(DEV):
        model = LlamaForCausalLM(LlamaConfig(**LLAMA31_8B)).to(torch.bfloat16).eval()
    torch.cuda.empty_cache()
    budget = torch.cuda.mem_get_info(DEV)[0] - HEADROOM_GIB * 2**30

    def per_seq(be):
        e1 = exactkv.Engine(model, 1, PROMPT + NEW, backend=be)
        e2 = exactkv.Engine(model, 2, PROMPT + NEW, backend=be)
        d = e2.kv_bytes() - e1.kv_bytes()
        del e1, e2
        torch.cuda.empty_cache()
        return d
    ps = {be: per_seq(be) for be in ("bf16", "exactkv")}
    fit = {be: int(budget // n) for be, n in ps.items()}
    B = min(fit["bf16"], int((budget - WORK_GIB * 2**30) // ps["bf16"]))
    _say(capsys, f"budget {budget / 2**30:.1f} GiB, fit {fit}, batch {B}")
    assert fit["exactkv"] > fit["bf16"] and B > 0

    ids = torch.randint(0, LLAMA31_8B["vocab_size"], (B, PROMPT), generator=torch.Generator().manual_seed(1)).to(DEV)
    w = torch.randint(1, 2**31, (2, LLAMA31_8B["vocab_size"]), generator=torch.Generator().manual_seed(2),
                      dtype=torch.int64).to(DEV)
    tok_b, fp_b, _, T_b = _run(model, "bf16", B, ids, w, capsys)
    tok_c, fp_c, grows_c, T_c = _run(model, "exactkv", B, ids, w, capsys)
    assert T_b == T_c == PROMPT + NEW - 1
    assert tok_b.shape == (B, NEW)
    if not (torch.equal(tok_b, tok_c) and torch.equal(fp_b, fp_c)):
        _say(capsys, _where_they_part(tok_b, tok_c, fp_b, fp_c))
    assert torch.equal(tok_b, tok_c), "greedy tokens differ between the bf16 and the compressed cache"
    assert torch.equal(fp_b, fp_c), "logits differ between the bf16 and the compressed cache"
    # the greedy tokens are not degenerate (random weights still give varied argmaxes)
    assert len(torch.unique(tok_b[:, -1])) > 1
    _say(capsys, f"tokens and logits identical over {NEW} tokens x {B} sequences; pool grows {grows_c}")
