"""Host-side check of the engine's write-through prefill cache (no GPU): the model's
forward pass hands every layer's RoPE'd keys and values to it exactly as they would land
in a DynamicCache (reference engine.py:42-49), and its outputs do not change."""
import torch

from exactkv_amd.engine import _write_through


class _Recorder:
    def __init__(self):
        self.seen = []

    def prefill_slot(self, b, x):
        self.seen.append((b, x.clone()))


class _FakeEngine:
    def __init__(self, layers):
        self.kv = [(_Recorder(), _Recorder()) for _ in range(layers)]


def _tiny(kind):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM
    common = dict(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    torch.manual_seed(0)
    if kind == "llama":
        return LlamaForCausalLM(LlamaConfig(rope_theta=5e5, **common)).eval()
    return Qwen3ForCausalLM(Qwen3Config(head_dim=128, rope_theta=1e6, **common)).eval()


def test_write_through_sees_the_dynamic_cache_contents():
    for kind in ("llama", "qwen3"):
        m = _tiny(kind)
        ids = torch.randint(0, 256, (1, 37), generator=torch.Generator().manual_seed(1))
        with torch.no_grad():
            ref = m.model(ids, use_cache=True)
            eng = _FakeEngine(2)
            out = m.model(ids, use_cache=True, past_key_values=_write_through(eng, 3))
        assert torch.equal(out.last_hidden_state, ref.last_hidden_state), kind
        pkv = ref.past_key_values
        for i, (kr, vr) in enumerate(eng.kv):
            assert len(kr.seen) == len(vr.seen) == 1
            (bk, k), (bv, v) = kr.seen[0], vr.seen[0]
            assert bk == bv == 3 and k.shape == (1, 37, 2, m.config.head_dim if kind == "qwen3" else 64)
            assert torch.equal(k, pkv.layers[i].keys.transpose(1, 2))
            assert torch.equal(v, pkv.layers[i].values.transpose(1, 2))
        assert out.past_key_values.get_seq_length() == 0        # nothing kept
