"""Host-side checks of the transformers connection (no GPU): the patch is a
pass-through without the packed cache and is fully undone by restore(); the
decode preconditions refuse what the reference refuses
(experiments/ac08/source/loop_kv_ac08_attention.py:26-33,46-96)."""
from types import SimpleNamespace

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM  # noqa: E402

from nsn_amd import adapter  # noqa: E402
from nsn_amd.errors import IntegrityError  # noqa: E402


def tiny_model(family="llama", seed=0):
    torch.manual_seed(seed)
    kw = dict(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
              num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=512)
    if family == "qwen3":
        return Qwen3ForCausalLM(Qwen3Config(**kw)).eval()
    return LlamaForCausalLM(LlamaConfig(**kw)).eval()


@pytest.mark.parametrize("family", ["llama", "qwen3"])
def test_install_is_passthrough_without_packed_cache_and_restore_undoes_it(family):
    m = tiny_model(family)
    ids = torch.randint(0, 64, (2, 9), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ref = m(input_ids=ids).logits
        originals = [l.self_attn.forward for l in m.model.layers]
        restore = adapter.install(m)
        assert all(l.self_attn.forward != o for l, o in zip(m.model.layers, originals))
        got = m(input_ids=ids).logits                      # DynamicCache: the original forward
        fused = [hasattr(l.self_attn, "_nsn_qkv") for l in m.model.layers]
        assert fused == [family == "llama"] * 2            # one QKV weight per Llama-family attention
        if family == "llama":
            a = m.model.layers[0].self_attn
            w, bias, nq, nk = a._nsn_qkv
            assert bias is None and (nq, nk) == (256, 128)
            assert torch.equal(w, torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]))
        restore()
        assert not any(hasattr(l.self_attn, "_nsn_qkv") for l in m.model.layers)
        assert [l.self_attn.forward for l in m.model.layers] == originals
        again = m(input_ids=ids).logits
    assert torch.equal(ref, got) and torch.equal(ref, again)


def _stub_cache(length=10, strict=True, batch=1, heads_q=2, arm="PACKED_KV_FUSED"):
    return SimpleNamespace(store=SimpleNamespace(length=[length]), batch=batch, heads_q=heads_q, strict=strict,
                           arm=arm)


def _module(training=False, window=None):
    return SimpleNamespace(training=training, sliding_window=window)


def test_check_decode_accepts_the_decode_step():
    q = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16)
    assert adapter.check_decode(_module(), q, _stub_cache(), 0, torch.tensor([[9]]), None) == 10
    assert adapter.check_decode(_module(), q, _stub_cache(), 0, torch.tensor([[9]]), torch.zeros(1, 1, 1, 10)) == 10
    assert adapter.check_decode(_module(), q, _stub_cache(), 0, None, torch.ones(1, 1, 1, 10, dtype=torch.bool)) == 10


@pytest.mark.parametrize("case", ["training", "window", "shape", "dtype", "position", "mask_len", "mask_blocked"])
def test_check_decode_refusals(case):
    q = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16)
    mod, pos, mask = _module(), torch.tensor([[9]]), None
    if case == "training":
        mod = _module(training=True)
    elif case == "window":
        mod = _module(window=128)
    elif case == "shape":
        q = torch.zeros(1, 2, 2, 128, dtype=torch.bfloat16)
    elif case == "dtype":
        q = q.float()
    elif case == "position":
        pos = torch.tensor([[8]])
    elif case == "mask_len":
        mask = torch.zeros(1, 1, 1, 9)
    elif case == "mask_blocked":
        mask = torch.zeros(1, 1, 1, 10)
        mask[..., 3] = float("-inf")
    with pytest.raises(IntegrityError):
        adapter.check_decode(mod, q, _stub_cache(), 0, pos, mask)


def test_check_decode_non_strict_skips_the_synchronising_checks():
    q = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16)
    mask = torch.zeros(1, 1, 1, 10)
    mask[..., 3] = float("-inf")
    assert adapter.check_decode(_module(), q, _stub_cache(strict=False), 0, torch.tensor([[3]]), mask) == 10


def test_unknown_arm_and_head_dim_refused():
    cfg = SimpleNamespace(num_attention_heads=2, num_key_value_heads=1, head_dim=128, hidden_size=256,
                          num_hidden_layers=2)
    with pytest.raises(IntegrityError):
        adapter.PackedKVCache(cfg, 1, 256, arm="TILE_MATERIALIZE")
    cfg.head_dim = 64
    with pytest.raises(IntegrityError):
        adapter.PackedKVCache(cfg, 1, 256)


def test_slot_of_looped_layers():
    """Slots of a looped model: current_ut * num_hidden_layers + layer_idx
    (loop_kv_ac08_attention.py:67); out-of-range layers or loops refused."""
    fake = SimpleNamespace(n_layers=24, store=SimpleNamespace(slots=96))
    assert adapter.PackedKVCache.slot(fake, 0) == 0
    assert adapter.PackedKVCache.slot(fake, 3, 2) == 51
    assert adapter.PackedKVCache.slot(fake, 23, 3) == 95
    for layer, ut in ((24, 0), (0, 4), (-1, 0)):
        with pytest.raises(IntegrityError):
            adapter.PackedKVCache.slot(fake, layer, ut)


def test_check_decode_takes_fp32_queries_on_the_native_arm_only():
    q = torch.zeros(1, 2, 1, 128, dtype=torch.float32)
    assert adapter.check_decode(_module(), q, _stub_cache(arm="NATIVE"), 0, None, None) == 10
    with pytest.raises(IntegrityError):
        adapter.check_decode(_module(), q, _stub_cache(), 0, None, None)


def test_sliding_window_configs_are_refused_before_any_append():
    """The window lives in the config (Mistral keeps no attribute on the
    module): a window shorter than the cache capacity is refused at cache
    construction and in check_decode; Qwen2's unused window is not."""
    from transformers import MistralConfig, Qwen2Config
    kw = dict(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=2, num_attention_heads=2,
              num_key_value_heads=1, head_dim=128, max_position_embeddings=8192)
    mistral = MistralConfig(sliding_window=4096, **kw)
    assert adapter.sliding_window(mistral, 0) == 4096
    with pytest.raises(IntegrityError, match="sliding-window"):
        adapter.PackedKVCache(mistral, 1, 8192, device=torch.device("cpu"))
    # a window at least the capacity never cuts the attention
    adapter._refuse_window(mistral, 0, 4096)
    qwen2 = Qwen2Config(**kw)
    assert adapter.sliding_window(qwen2, 0) is None
    layered = SimpleNamespace(sliding_window=512, layer_types=["full_attention", "sliding_attention"])
    assert adapter.sliding_window(layered, 0) is None and adapter.sliding_window(layered, 1) == 512
    mod = SimpleNamespace(training=False, sliding_window=None, config=mistral, layer_idx=0)
    with pytest.raises(IntegrityError, match="sliding-window"):
        adapter.check_decode(mod, torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16),
                             SimpleNamespace(store=SimpleNamespace(length=[10]), batch=1, heads_q=2, strict=False,
                                             arm="PACKED_KV_FUSED", max_tokens=8192), 0, None, None)


def test_fused_qkv_is_rebuilt_when_the_weights_change():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    torch.manual_seed(0)
    m = Qwen2ForCausalLM(Qwen2Config(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=1,
                                     num_attention_heads=2, num_key_value_heads=1, head_dim=128)).eval()
    restore = adapter.install(m)
    a = m.model.layers[0].self_attn
    w, bias, nq, nk = adapter._fused_qkv(a)
    assert bias is not None and torch.equal(bias, torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias]))
    assert adapter._fused_qkv(a)[0] is w                          # unchanged weights: the same copy
    with torch.no_grad():
        a.k_proj.weight.add_(1.0)                                 # an in-place update
    w2 = adapter._fused_qkv(a)[0]
    assert w2 is not w and torch.equal(w2[nq:nq + nk], a.k_proj.weight)
    m.to(torch.float64)                                           # a cast replaces the parameters
    assert adapter._fused_qkv(a)[0].dtype == torch.float64
    restore()
    assert not hasattr(a, "_nsn_qkv") and not hasattr(a, "_nsn_qkv_key")
