"""Engine (reference exactkv/engine.py:18-95, tests/test_exactkv.py:107-122): greedy decoding
of small random-init Llama-3 / Qwen3 / Qwen2 models over the compressed and the bf16 cache.

  * the two backends give the same tokens and bit-identical logits (the cache is lossless
    and the two attention kernels are bit-identical);
  * HIP-graph replay of the step equals eager steps bit for bit;
  * a raw-pool growth between steps makes the engine capture the step again, and the
    results stay exact;
  * an attention plug-in (reference engine.py:30-33) runs the step eagerly.

Prompts are 37 tokens (a partly filled page) and 40 tokens are generated, so the run
crosses two page boundaries (page encodes inside the step, check_overflow after it)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

B, PROMPT, NEW = 3, 37, 40


def _model(kind, layers=2, seed=0):
    from transformers import (LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM, Qwen3Config,
                              Qwen3ForCausalLM)
    common = dict(vocab_size=1024, hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096)
    if kind == "llama":
        cfg, cls = LlamaConfig(rope_theta=5e5, **common), LlamaForCausalLM
    elif kind == "qwen3":
        cfg, cls = Qwen3Config(head_dim=128, rope_theta=1e6, **common), Qwen3ForCausalLM
    else:
        cfg, cls = Qwen2Config(rope_theta=1e6, **common), Qwen2ForCausalLM
    torch.manual_seed(seed)
    with torch.device("cuda"):
        m = cls(cfg)
    return m.to(torch.bfloat16).eval()


def _ids(vocab=1024, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (B, PROMPT), generator=g).cuda()


def _run(model, backend, graph=True, **kw):
    import exactkv_amd as exactkv
    eng = exactkv.Engine(model, B, PROMPT + NEW, backend=backend, graph=graph, **kw)
    toks, logits = eng.generate(_ids(), NEW)
    torch.cuda.synchronize()
    return eng, toks, logits


@pytest.mark.parametrize("kind", ["llama", "qwen3", "qwen2"])
def test_backends_give_identical_tokens_and_logits(kind):
    m = _model(kind)
    print(f"[engine] {kind}: bf16 backend", flush=True)
    _, tb, lb = _run(m, "bf16")
    print(f"[engine] {kind}: exactkv backend", flush=True)
    e, tc, lc = _run(m, "exactkv")
    assert torch.equal(tb, tc)
    assert torch.equal(lb.view(torch.int16), lc.view(torch.int16))
    assert torch.isfinite(lc.float()).all()
    assert e.kv[0][0].T == PROMPT + NEW - 1


def test_graph_replay_equals_eager_steps():
    m = _model("llama")
    print("[engine] eager", flush=True)
    ee, te, le = _run(m, "exactkv", graph=False)
    print("[engine] graph", flush=True)
    eg, tg, lg = _run(m, "exactkv", graph=True)
    assert eg.use_graph and eg._graph is not None and not ee.use_graph
    assert torch.equal(te, tg)
    assert torch.equal(le.view(torch.int16), lg.view(torch.int16))


def test_pool_growth_between_steps_recaptures_and_stays_exact():
    import exactkv_amd as exactkv
    m = _model("llama")
    ids = _ids()
    ref = exactkv.Engine(m, B, PROMPT + NEW, backend="bf16")
    eng = exactkv.Engine(m, B, PROMPT + NEW, backend="exactkv")
    t_r, t_e = ref.prefill(ids), eng.prefill(ids)
    assert torch.equal(t_r, t_e)
    for s in range(NEW - 1):
        if s in (3, 17):                      # grow two pools between steps
            c = eng.kv[s % 2][1]
            cap = c.cap
            c._grow(c.cap + 1)
            assert c.cap > cap
        lr, le = ref.step(t_r), eng.step(t_e)
        assert torch.equal(lr.view(torch.int16), le.view(torch.int16)), s
        t_r, t_e = lr.argmax(-1), le.argmax(-1)
    assert eng.captures >= 3                  # captured, then captured again after each growth
    # (buffer addresses are not a count: the allocator may hand a freed block back)


def test_attention_plugin_runs_eagerly():
    import exactkv_amd as exactkv
    m = _model("llama")
    calls = []

    def attn(q, kc, vc):
        calls.append(kc.T)
        return exactkv.decode_attention(q, kc, vc)

    _, tb, lb = _run(m, "bf16", attn=attn)
    calls.clear()
    e, tp, lp = _run(m, "exactkv", attn=attn)
    assert not e.use_graph
    assert len(calls) == 2 * (NEW - 1)       # layers x steps
    assert calls[0] == PROMPT + 1 and calls[-1] == PROMPT + NEW - 1
    assert torch.equal(tb, tp)
    assert torch.equal(lb.view(torch.int16), lp.view(torch.int16))


@pytest.mark.parametrize("kind", ["llama", "qwen3"])
def test_fused_prefill_writes_the_same_cache(kind):
    """Prefill with the write-through cache (each layer's K/V encoded straight from the
    attention module, no DynamicCache copy) leaves the same bytes in every cache as the
    two-pass prefill, and the same next tokens; the model's own DynamicCache output then
    holds nothing."""
    import exactkv_amd as exactkv
    m = _model(kind)
    ids = _ids(seed=5)
    a = exactkv.Engine(m, B, PROMPT + NEW, backend="exactkv")
    f = exactkv.Engine(m, B, PROMPT + NEW, backend="exactkv")
    print(f"[engine] {kind}: two-pass prefill", flush=True)
    ta = a.prefill(ids, fused=False)
    print(f"[engine] {kind}: fused prefill", flush=True)
    tf = f.prefill(ids, fused=True)
    torch.cuda.synchronize()
    assert torch.equal(ta, tf)
    for (ka, va), (kf, vf) in zip(a.kv, f.kv):
        for ca, cf in ((ka, kf), (va, vf)):
            assert ca.T == cf.T == PROMPT and ca.cap == cf.cap
            for name in ("sm", "code", "base", "rowmask", "rowoff", "cnt"):
                assert torch.equal(getattr(ca, name), getattr(cf, name)), name
            assert torch.equal(ca.raw.view(torch.int16), cf.raw.view(torch.int16))
    ba = exactkv.Engine(m, B, PROMPT + NEW, backend="bf16")
    bf = exactkv.Engine(m, B, PROMPT + NEW, backend="bf16")
    assert torch.equal(ba.prefill(ids, fused=False), bf.prefill(ids))
    for (ka, va), (kf, vf) in zip(ba.kv, bf.kv):
        assert torch.equal(ka.buf.view(torch.int16), kf.buf.view(torch.int16))
        assert torch.equal(va.buf.view(torch.int16), vf.buf.view(torch.int16))


@pytest.mark.parametrize("kind", ["llama", "qwen3"])
def test_write_through_prefill_equals_the_oracle_codec(kind):
    """The write-through prefill's bytes against the oracle: the reference prefills with a
    DynamicCache and copies each layer's K/V into its cache (engine.py:42-49,
    cache.py:87-98), i.e. codec.encode of those tensors for the full pages and bf16 rows in
    the tail area for the open page. Encode the model's own DynamicCache K/V with the CPU
    oracle and compare every byte of every layer's caches."""
    import numpy as np
    import exactkv_amd as exactkv
    from exactkv_amd.engine import _fused_sdpa
    from oracle import codec as ocodec
    from tests.conftest import u16
    m = _model(kind)
    ids = _ids(seed=21)
    eng = exactkv.Engine(m, B, PROMPT + NEW, backend="exactkv")
    print(f"[engine] {kind}: write-through prefill vs oracle", flush=True)
    eng.prefill(ids, fused=True)
    ref = [[[], []] for _ in range(eng.L)]             # per layer: K, V of each sequence [T, H, D]
    with torch.no_grad(), _fused_sdpa():
        for b in range(B):
            pkv = m.model(ids[b:b + 1], use_cache=True).past_key_values
            for i in range(eng.L):
                ref[i][0].append(pkv.layers[i].keys[0].transpose(0, 1).cpu())
                ref[i][1].append(pkv.layers[i].values[0].transpose(0, 1).cpu())
    torch.cuda.synchronize()
    Tf = PROMPT // 16 * 16
    for i in range(eng.L):
        for c, xs in zip(eng.kv[i], ref[i]):
            x = torch.stack(xs)                        # [B, T, H, D]
            want = ocodec.encode(u16(x[:, :Tf]))
            npg = Tf // 16
            for name, t in (("sm", c.sm[:, :Tf]), ("code", c.code[:, :Tf]), ("base", c.base[:, :npg]),
                            ("rowmask", c.rowmask[:, :npg]), ("rowoff", c.rowoff[:, :npg])):
                assert np.array_equal(t.cpu().numpy(), want[name]), (kind, i, name)
            n = want["raw"].shape[0]
            assert int(c.cnt.item()) == n, (kind, i)
            assert np.array_equal(u16(c.raw[:n]), want["raw"]), (kind, i, "raw")
            H = c.H
            assert (c.rowmask[:, npg] == 0xFFFF).all()
            slots = c.cap + torch.arange(B * H, device=c.raw.device, dtype=torch.int32).view(B, H) * 16
            assert torch.equal(c.rowoff[:, npg], slots)
            for b in range(B):
                for h in range(H):
                    s0 = c.cap + (b * H + h) * 16
                    assert np.array_equal(u16(c.raw[s0: s0 + PROMPT - Tf]), u16(x[b, Tf:, h])), (kind, i, b, h)


def test_sliding_window_model():
    """Qwen2 with sliding-window layers (use_sliding_window, window 24 < the 37-token
    prompt): both backends give bit-identical logits, and with teacher forcing they follow
    the model's own full forward pass (its sliding-window mask) within bf16 noise, much
    closer than the same engine with the window switched off."""
    import exactkv_amd as exactkv
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=1024, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096, rope_theta=1e6,
                      use_sliding_window=True, sliding_window=24, max_window_layers=0)
    torch.manual_seed(0)
    with torch.device("cuda"):
        m = Qwen2ForCausalLM(cfg)
    m = m.to(torch.bfloat16).eval()
    N = 24
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 1024, (B, PROMPT + N + 1), generator=g).cuda()
    with torch.no_grad():
        ref = m(ids).logits.float()                    # the model's own masks, all positions
    out = {}
    for name, backend, windows in (("c", "exactkv", None), ("b", "bf16", None), ("off", "exactkv", [0, 0])):
        eng = exactkv.Engine(m, B, PROMPT + N, backend=backend)
        assert eng.windows == [24, 24]
        if windows is not None:
            eng.windows = windows
        print(f"[engine] window {name}", flush=True)
        eng.prefill(ids[:, :PROMPT])
        ls = [eng.step(ids[:, PROMPT + t]).float() for t in range(N)]
        out[name] = torch.stack(ls, 1)                 # logits at positions PROMPT + t
    torch.cuda.synchronize()
    assert torch.equal(out["c"], out["b"])
    want = ref[:, PROMPT:PROMPT + N]
    scale = want.abs().max().item()
    err_on = (out["c"] - want).abs().max().item()
    err_off = (out["off"] - want).abs().max().item()
    print(f"[engine] window: err {err_on:.4g}, without the window {err_off:.4g}, scale {scale:.4g}", flush=True)
    assert err_on <= 0.03 * scale
    assert err_off > 4 * err_on


def test_paged_engine_matches_the_contiguous_engine():
    """Equal-length prompts: the paged engine (block tables over a shared pool) gives the
    contiguous engine's logits bit for bit (same pages, same split plan)."""
    import exactkv_amd as exactkv
    m = _model("llama")
    ids = _ids(seed=11)
    ref = exactkv.Engine(m, B, PROMPT + NEW, backend="exactkv", graph=False)
    pe = exactkv.PagedEngine(m, B, PROMPT + NEW, backend="exactkv")
    t_r = ref.prefill(ids)
    t_p = torch.stack([pe.add(ids[b])[1] for b in range(B)])
    assert torch.equal(t_r, t_p)
    print("[engine] paged vs contiguous", flush=True)
    for s in range(NEW - 1):
        lr, lp = ref.step(t_r), pe.step(t_p)
        assert torch.equal(lr.view(torch.int16), lp.view(torch.int16)), s
        t_r, t_p = lr.argmax(-1), lp.argmax(-1)


def test_paged_engine_ragged_sequences_join_and_leave():
    """Prompts of different lengths decode side by side; a sequence leaves and a new one
    joins in its slot. The compressed and bf16 paged engines agree bit for bit, and with
    teacher forcing each sequence follows the model's own forward pass over its tokens."""
    import exactkv_amd as exactkv
    m = _model("qwen3")
    g = torch.Generator().manual_seed(13)
    lens = [37, 20, 50, 9]
    total = 90
    toks = torch.randint(0, 1024, (len(lens), total), generator=g).cuda()
    ec = exactkv.PagedEngine(m, 4, total, backend="exactkv")
    eb = exactkv.PagedEngine(m, 4, total, backend="bf16")
    for b, L in enumerate(lens[:3]):
        assert ec.add(toks[b, :L])[0] == eb.add(toks[b, :L])[0] == b
    pos = {0: lens[0], 1: lens[1], 2: lens[2]}                   # next position of each live slot
    got = {b: [] for b in range(4)}
    print("[engine] paged ragged", flush=True)
    for s in range(30):
        if s == 10:                                              # slot 1 leaves, a new prompt joins it
            ec.release(1)
            eb.release(1)
            assert ec.add(toks[3, :lens[3]])[0] == eb.add(toks[3, :lens[3]])[0] == 1
            pos[1] = lens[3]
            got[1] = []
        live = sorted(pos)
        row = {0: 0, 1: 3, 2: 2}                                 # prompt row of each slot after the swap
        seq = lambda sl: row[sl] if s >= 10 or sl != 1 else 1    # noqa: E731
        tok = torch.stack([toks[seq(sl), pos[sl]] for sl in live])
        lc, lb = ec.step(tok, live), eb.step(tok, live)
        assert torch.equal(lc.view(torch.int16), lb.view(torch.int16)), s
        for i, sl in enumerate(live):
            got[sl].append((seq(sl), pos[sl], lc[i].float()))
            pos[sl] += 1
    with torch.no_grad():
        for sl, rows in got.items():
            if not rows:
                continue
            r, p_last = rows[0][0], rows[-1][1]
            ref = m(toks[r:r + 1, :p_last + 1]).logits[0].float()
            want = torch.stack([ref[p] for _, p, _ in rows])
            have = torch.stack([lg for _, _, lg in rows])
            err = (have - want).abs().max().item()
            assert err <= 0.03 * want.abs().max().item(), (sl, err)
    assert ec.table.free_pages() < ec.table.num_pages


def test_paged_engine_graph_replay_and_growth():
    """The paged engine's HIP-graph steps equal its eager steps bit for bit, also across a
    raw-pool growth between steps (which makes it capture the step again)."""
    import exactkv_amd as exactkv
    m = _model("llama")
    ids = _ids(seed=17)
    eg = exactkv.PagedEngine(m, B, PROMPT + NEW, backend="exactkv", graph=True)
    ee = exactkv.PagedEngine(m, B, PROMPT + NEW, backend="exactkv", graph=False)
    tg = torch.stack([eg.add(ids[b])[1] for b in range(B)])
    te = torch.stack([ee.add(ids[b])[1] for b in range(B)])
    assert torch.equal(tg, te)
    print("[engine] paged graph vs eager", flush=True)
    for s in range(NEW - 1):
        if s == 9:
            c = eg.kv[1][0]
            cap = c.cap
            c._grow(c.cap + 1)
            assert c.cap > cap
        lg, le = eg.step(tg), ee.step(te)
        assert torch.equal(lg.view(torch.int16), le.view(torch.int16)), s
        tg, te = lg.argmax(-1), le.argmax(-1)
    assert eg.captures >= 2 and ee.captures == 0
