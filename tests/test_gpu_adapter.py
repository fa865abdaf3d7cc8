"""GPU parity of the transformers connection (the reference's AC08 decode
route, experiments/ac08/source/loop_kv_ac08_attention.py:46-96) on a
random-init GQA Llama (2 layers, 8 q-heads / 2 kv-heads, d=128, bf16).

- every decode step of every layer, through the fused arm, is checked
  against the oracle: the slot's packed blocks are restored by the C
  restatement of nsn_decode (fp32, as the fused kernel keeps them), the fp16
  tail appended, then float64 attention with the model's scale; tolerance
  |out - ref| <= 2e-3 + 1e-2 |ref| (the bf16 output);
- the run crosses a post_decode compression (prompt 150 -> 64 packed + 86
  tail; at 192 tokens the policy packs a second block);
- the other arms read the same cache: their teacher-forced logits agree
  with the NATIVE arm's (dense restore + sdpa).
"""
import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM  # noqa: E402

from nsn_amd import adapter  # noqa: E402
from oracle import oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
B, P, STEPS = 2, 150, 60
F16, BF16 = torch.float16, torch.bfloat16


def model(family="llama"):
    """Random-init 2-layer GQA decoder (8 q-heads / 2 kv-heads, d=128, bf16).
    qwen3 adds per-head RMS norms on q and k before the rotary embedding;
    qwen2 has q, k and v biases (concatenated into the fused QKV GEMM)."""
    torch.manual_seed(0)
    kw = dict(vocab_size=256, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
              num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=1024)
    if family == "qwen3":
        cfg = Qwen3Config(**kw)
        m = Qwen3ForCausalLM(cfg).to(DEV, torch.bfloat16).eval()
    elif family == "qwen2":
        from transformers import Qwen2Config, Qwen2ForCausalLM
        cfg = Qwen2Config(**kw)
        m = Qwen2ForCausalLM(cfg).to(DEV, torch.bfloat16).eval()
        with torch.no_grad():   # non-zero biases, so that a dropped or misplaced bias shows
            for layer in m.model.layers:
                for proj in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj):
                    proj.bias.normal_(0.0, 0.5)
    else:
        cfg = LlamaConfig(**kw)
        m = LlamaForCausalLM(cfg).to(DEV, torch.bfloat16).eval()
    ids = torch.randint(0, 256, (B, P), generator=torch.Generator().manual_seed(1)).to(DEV)
    return m, cfg, ids


def bits16(t):
    """fp16 tensor -> its raw bits (the oracle's metadata format)."""
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def slot_kv_oracle(cache, slot):
    """fp32 [B, H, L, 128] K and V of a slot as the fused kernel reads them."""
    st = cache.store
    L, C = st.length[slot], st.compressed[slot]
    out = []
    for name in ("K", "V"):
        kv = st.side(slot, name)
        nb = C // 64
        parts = []
        if nb:
            y = O.restore_blocks_f32(kv.codes[:, :, :nb].cpu().numpy(), bits16(kv.norm[:, :, :nb]),
                                     bits16(kv.min[:, :, :nb]), bits16(kv.scale[:, :, :nb]), kv.bits)
            parts.append(y.reshape(B, cache.heads, C, 128))
        parts.append(kv.tail[:, :, :L - C].float().cpu().numpy())
        out.append(np.concatenate(parts, axis=2))
    return out


@pytest.mark.parametrize("family", ["llama", "qwen3", "qwen2"])
def test_fused_arm_every_layer_and_step_vs_oracle(family):
    m, cfg, ids = model(family)
    cache = adapter.PackedKVCache(cfg, B, 1024, arm="PACKED_KV_FUSED", max_prefill=P)
    scale = m.model.layers[0].self_attn.scaling
    worst = [0.0]
    seen = []

    def capture(slot, total, q, out):
        k, v = slot_kv_oracle(cache, slot)
        assert k.shape[2] == total
        ref, _ = O.decode_attention64(q.float().cpu().numpy(), k, v, scale=scale)
        err = np.abs(out.float().cpu().numpy() - ref)
        assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), (slot, total, float(err.max()))
        worst[0] = max(worst[0], float(err.max()))
        seen.append((slot, total, cache.store.compressed[slot]))

    cache.capture = capture
    restore = adapter.install(m)
    try:
        toks, _ = adapter.greedy(m, cache, ids, STEPS)
    finally:
        restore()
    assert toks.shape == (B, STEPS)
    assert len(seen) == 2 * STEPS and sorted({s for s, _, _ in seen}) == [0, 1]
    assert {c for _, _, c in seen} == {64, 128}            # the decode crossed a compression
    assert all(cache.connection_calls[s] == STEPS for s in (0, 1))
    assert cache.store.length == [P + STEPS] * 2
    cache.check_status()


def forced_logits(m, cache, ids, tokens):
    """Prefill, then feed the given tokens (teacher forcing); logits of every step."""
    outs = []
    with torch.no_grad():
        out = m(input_ids=ids, past_key_values=cache, use_cache=True)
        cache.post_prefill()
        for i in range(tokens.shape[1]):
            outs.append(out.logits[:, -1].float())
            out = m(input_ids=tokens[:, i:i + 1], past_key_values=cache, use_cache=True)
            cache.post_decode()
    return torch.stack(outs)


@pytest.mark.parametrize("family,arm,tail_dtype", [("llama", "PACKED_KV_FUSED", F16), ("llama", "PACKED_GROUPED", F16),
                                                   ("llama", "PACKED_KV_EXACT", F16), ("qwen3", "PACKED_KV_FUSED", F16),
                                                   ("qwen2", "PACKED_KV_FUSED", F16), ("llama", "PACKED_KV_FUSED", BF16),
                                                   ("llama", "PACKED_GROUPED", BF16), ("llama", "PACKED_KV_EXACT", BF16)])
def test_arms_agree_with_native(family, arm, tail_dtype):
    m, cfg, ids = model(family)
    tokens = torch.randint(0, 256, (B, 40), generator=torch.Generator().manual_seed(2)).to(DEV)
    restore = adapter.install(m)
    try:
        ref = forced_logits(m, adapter.PackedKVCache(cfg, B, 1024, arm="NATIVE", max_prefill=P, tail_dtype=tail_dtype),
                            ids, tokens)
        got = forced_logits(m, adapter.PackedKVCache(cfg, B, 1024, arm=arm, max_prefill=P, tail_dtype=tail_dtype),
                            ids, tokens)
    finally:
        restore()
    assert torch.equal(got[0], ref[0])                    # the prefill is the native route in every arm
    # decode steps: the arms differ only in attention rounding (bf16 outputs
    # of fp32 or bf16 arithmetic), carried through o_proj, the MLP and the head
    err = (got - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item() + 1e-3, err


@pytest.mark.parametrize("tail_dtype", [F16, BF16])
def test_native_arm_prefill_matches_unpatched_model(tail_dtype):
    m, cfg, ids = model()
    with torch.no_grad():
        ref = m(input_ids=ids).logits
        restore = adapter.install(m)
        try:
            cache = adapter.PackedKVCache(cfg, B, 1024, arm="NATIVE", max_prefill=P, tail_dtype=tail_dtype)
            got = m(input_ids=ids, past_key_values=cache, use_cache=True).logits
        finally:
            restore()
    if tail_dtype == BF16:   # the model's own K/V stored and read back unchanged
        assert torch.equal(got, ref)
        return
    # the prefill appends bf16 K/V to the fp16 tail and reads them back:
    # exact down to 2^-17 (fp16 subnormal spacing 2^-24 against bf16's 8-bit
    # significand), so only the rare K/V element below that moves, by < 2^-24
    err = (got.float() - ref.float()).abs().max().item()
    assert err <= 1e-3 * ref.float().abs().max().item(), err


@pytest.mark.parametrize("tail_dtype", [F16, BF16])
def test_decode_graph_replays_match_eager_steps(tail_dtype):
    """The fused step captured as a HIP graph: every replay (with eager work
    and a synchronisation between replays) equals the same device-position
    step run eagerly, bit for bit, across a compression; both agree with the
    host-position fused arm to the arms' tolerance.  fp16 and bf16 tails."""
    m, cfg, ids = model()
    n = 80
    tokens = torch.randint(0, 256, (B, n), generator=torch.Generator().manual_seed(3)).to(DEV)
    restore = adapter.install(m)
    outs = {}
    try:
        for use_graph in (False, True):
            cache = adapter.PackedKVCache(cfg, B, 1024, arm="PACKED_KV_FUSED", max_prefill=P, strict=False,
                                          tail_dtype=tail_dtype)
            with torch.no_grad():
                m(input_ids=ids, past_key_values=cache, use_cache=True)
            cache.post_prefill()
            dg = adapter.DecodeGraph(m, cache, use_graph=use_graph)
            steps = []
            for i in range(n):
                steps.append(dg.step(tokens[:, i:i + 1])[:, -1].float().clone())
                torch.cuda.synchronize()
            cache.check_status()
            assert cache.store.length == [P + n] * 2 and cache.store.compressed == [128, 128]
            assert all(cache.connection_calls[s] == n for s in (0, 1))
            assert dg.replays == (n if use_graph else 0)
            outs[use_graph] = torch.stack(steps)
        ref = forced_logits(m, adapter.PackedKVCache(cfg, B, 1024, arm="PACKED_KV_FUSED", max_prefill=P,
                                                     tail_dtype=tail_dtype), ids, tokens)
    finally:
        restore()
    assert torch.equal(outs[True], outs[False])
    err = (outs[True][:-1] - ref[1:]).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item() + 1e-3, err


def test_tail_append_to_places_like_tail_append_and_refuses_out_of_range():
    """nsn_tail_append_to through the C ABI: the tokens land at
    [end - n, end) of every row, bit for bit what nsn_tail_append writes at
    offset end - n; an end outside [n, tail_cap] writes nothing and raises
    NSN_ST_TAIL_RANGE (the kernel's own range check, set from the host)."""
    from nsn_amd import _dev, _lib
    lib = _lib.lib()
    rows, n, cap = 6, 3, 20
    g = torch.Generator(device=DEV).manual_seed(7)
    k = torch.randn((rows, n, 128), generator=g, device=DEV).to(torch.float16)
    v = torch.randn((rows, n, 128), generator=g, device=DEV).to(torch.float16)
    stream = _dev.stream()
    for end in (n, 11, cap):
        kt_a = torch.zeros((rows, cap, 128), dtype=torch.float16, device=DEV)
        vt_a, kt_b, vt_b = kt_a.clone(), kt_a.clone(), kt_a.clone()
        end_t = torch.tensor([end], dtype=torch.int32, device=DEV)
        st = _dev.new_status(DEV)
        assert lib.nsn_tail_append_to(k.data_ptr(), v.data_ptr(), rows, n, n, kt_a.data_ptr(), vt_a.data_ptr(), cap,
                                      end_t.data_ptr(), _lib.DTYPE_F16, st.data_ptr(), stream) == 0
        assert lib.nsn_tail_append(k.data_ptr(), v.data_ptr(), rows, n, n, kt_b.data_ptr(), vt_b.data_ptr(), cap,
                                   end - n, _lib.DTYPE_F16, stream) == 0
        assert _dev.read_status(st) == 0
        assert torch.equal(kt_a.view(torch.int16), kt_b.view(torch.int16))
        assert torch.equal(vt_a.view(torch.int16), vt_b.view(torch.int16))
        assert torch.equal(kt_a[:, end - n:end], k) and torch.equal(vt_a[:, end - n:end], v)
    for end in (n - 1, cap + 1):
        kt = torch.zeros((rows, cap, 128), dtype=torch.float16, device=DEV)
        vt = kt.clone()
        end_t = torch.tensor([end], dtype=torch.int32, device=DEV)
        st = _dev.new_status(DEV)
        assert lib.nsn_tail_append_to(k.data_ptr(), v.data_ptr(), rows, n, n, kt.data_ptr(), vt.data_ptr(), cap,
                                      end_t.data_ptr(), _lib.DTYPE_F16, st.data_ptr(), stream) == 0
        assert _dev.read_status(st) == _lib.ST_TAIL_RANGE
        assert not kt.any() and not vt.any()


def test_strict_decode_raises_on_nonfinite_tail():
    """A nonfinite K token in the tail reaches the fused kernel's input flag:
    the strict decode step raises NumericalFailure (the reference raises at
    its finite check, loop_kv_ac08_attention.py:70-72)."""
    from nsn_amd.errors import NumericalFailure
    m, cfg, ids = model()
    cache = adapter.PackedKVCache(cfg, B, 1024, arm="PACKED_KV_FUSED", max_prefill=P)
    restore = adapter.install(m)
    try:
        with torch.no_grad():
            out = m(input_ids=ids, past_key_values=cache, use_cache=True)
            cache.post_prefill()
            cache.store.side(1, "K").tail[1, 0, 5, 17] = float("inf")
            with pytest.raises(NumericalFailure):
                m(input_ids=out.logits[:, -1:].argmax(-1), past_key_values=cache, use_cache=True)
    finally:
        restore()


@pytest.mark.parametrize("tail_dtype", [F16, BF16])
def test_values_past_fp16_range_compute_on_bf16_tails(tail_dtype):
    """Layer 0's value projection scaled by 1e5 after the prefill puts the
    decode tokens' V past 65504, fp16's largest finite value.  On fp16 tails
    they become Inf and the strict decode step raises NumericalFailure; on
    bf16 tails they are kept as the model computed them, and every decode
    step of the fused arm (fused rotary append into the bf16 tail, bf16 MFMA
    over the tail, packed blocks from the prompt) meets the oracle, with the
    tolerance's absolute term scaled by the slot's largest |V|."""
    from nsn_amd.errors import NumericalFailure
    m, cfg, ids = model()
    cache = adapter.PackedKVCache(cfg, B, 1024, arm="PACKED_KV_FUSED", max_prefill=P, tail_dtype=tail_dtype)
    scale = m.model.layers[0].self_attn.scaling
    seen = []

    def capture(slot, total, q, out):
        k, v = slot_kv_oracle(cache, slot)
        ref, _ = O.decode_attention64(q.float().cpu().numpy(), k, v, scale=scale)
        vmax = float(np.abs(v).max())
        err = np.abs(out.float().cpu().numpy() - ref)
        assert np.all(err <= 2e-3 * max(1.0, vmax) + 1e-2 * np.abs(ref)), (slot, total, float(err.max()))
        seen.append((slot, vmax))

    restore = adapter.install(m)
    try:
        with torch.no_grad():
            out = m(input_ids=ids, past_key_values=cache, use_cache=True)
            cache.post_prefill()
            m.model.layers[0].self_attn.v_proj.weight.mul_(1e5)
            nxt = out.logits[:, -1:].argmax(-1)
            if tail_dtype == F16:
                with pytest.raises(NumericalFailure):
                    m(input_ids=nxt, past_key_values=cache, use_cache=True)
                return
            cache.capture = capture
            for _ in range(20):
                out = m(input_ids=nxt, past_key_values=cache, use_cache=True)
                cache.post_decode()
                nxt = out.logits[:, -1:].argmax(-1)
            assert torch.isfinite(out.logits).all()
        cache.check_status()
    finally:
        restore()
    assert len(seen) == 40 and cache.store.compressed == [64, 64]
    assert max(vm for s, vm in seen if s == 0) > 65504 > max(vm for s, vm in seen if s == 1)


def test_check_status_reports_a_tail_range_flag():
    """A device-position step whose tail end was pushed past the tail
    capacity (from the host) appends nothing; check_status raises
    IntegrityError for it."""
    from nsn_amd.errors import IntegrityError
    m, cfg, ids = model()
    cache = adapter.PackedKVCache(cfg, B, 1024, arm="PACKED_KV_FUSED", max_prefill=P, strict=False)
    restore = adapter.install(m)
    try:
        with torch.no_grad():
            m(input_ids=ids, past_key_values=cache, use_cache=True)
        cache.post_prefill()
        dg = adapter.DecodeGraph(m, cache, use_graph=False)
        dg.step(ids[:, :1])
        cache.check_status()
        dg._load_counters()
        cache.counters[B:].fill_(cache.store.tail_cap)   # the step's add makes it tail_cap + 1
        dg.step(ids[:, 1:2])
        torch.cuda.synchronize()
        with pytest.raises(IntegrityError):
            cache.check_status()
    finally:
        restore()


@pytest.mark.parametrize("family,tail_dtype", [("llama", F16), ("qwen3", F16), ("llama", BF16)])
def test_packed_prefill_is_as_accurate_as_the_native_route(family, tail_dtype):
    """A 600-token prompt in chunks of 200 (compressed after each), then 20
    forced decode steps.  The packed prefill route (chunk queries attend the
    packed context on the fp16 MFMA prefill kernel) and the reference's
    native route (dense bf16 restore + sdpa) both run the bf16 model; the
    truth is the same model in fp32 through the NATIVE arm (fp32 restore of
    the same packed storage, fp32 sdpa).  The packed route's logits must be
    no further from the truth than 1.5x the native route's, and layer 0's
    packed blocks (independent of any attention) are bitwise equal.  With
    bf16 tails the chunk's products run on bf16 MFMA tiles."""
    prompt = torch.randint(0, 256, (B, 600), generator=torch.Generator().manual_seed(4)).to(DEV)
    tokens = torch.randint(0, 256, (B, 20), generator=torch.Generator().manual_seed(5)).to(DEV)
    runs = {}
    for name, route, arm, fp32 in (("native", "native", "PACKED_KV_FUSED", False),
                                   ("packed", "packed", "PACKED_KV_FUSED", False),
                                   ("truth", "native", "NATIVE", True)):
        m, cfg, _ = model(family)
        if fp32:
            m = m.float()
        restore = adapter.install(m)
        try:
            cache = adapter.PackedKVCache(cfg, B, 1024, arm=arm, max_prefill=200, prefill=route,
                                          tail_dtype=tail_dtype)
            logits = []
            with torch.no_grad():
                for c in range(3):
                    out = m(input_ids=prompt[:, 200 * c:200 * (c + 1)], past_key_values=cache, use_cache=True)
                    cache.post_prefill()
                    logits.append(out.logits.float())
                for i in range(tokens.shape[1]):
                    out = m(input_ids=tokens[:, i:i + 1], past_key_values=cache, use_cache=True)
                    cache.post_decode()
                    logits.append(out.logits.float())
            cache.check_status()
        finally:
            restore()
        runs[name] = (torch.cat([x.reshape(-1, x.shape[-1]) for x in logits]), cache)
    truth = runs["truth"][0]
    e_native = (runs["native"][0] - truth).abs().max().item()
    e_packed = (runs["packed"][0] - truth).abs().max().item()
    print(f"{family}: max |logit - fp32 truth|: native route {e_native:.4f}, packed route {e_packed:.4f}")
    assert e_packed <= 1.5 * e_native + 1e-3, (e_packed, e_native)
    c_ref, c_got = runs["native"][1], runs["packed"][1]
    assert c_ref.store.compressed == c_got.store.compressed == [512, 512]
    for name in ("K", "V"):
        a, b = c_ref.store.side(0, name), c_got.store.side(0, name)
        assert torch.equal(a.codes[:, :, :8], b.codes[:, :, :8])
        assert torch.equal(a.norm[:, :, :8].view(torch.int16), b.norm[:, :, :8].view(torch.int16))


def looped(base, loops):
    """The decoder layers of a transformers Llama applied `loops` times with
    shared weights (an Ouro-like looped model); loop ut's attention gets
    current_ut = ut and so reads cache slot ut * layers + i."""
    import types

    class Looped(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.base = base

        def forward(self, input_ids, position_ids=None, past_key_values=None, use_cache=True, logits_to_keep=0):
            mdl = self.base.model
            h = mdl.embed_tokens(input_ids)
            if position_ids is None:
                past = past_key_values.get_seq_length()
                position_ids = torch.arange(past, past + input_ids.shape[1], device=h.device)[None]
            pe = mdl.rotary_emb(h, position_ids=position_ids)
            for ut in range(loops):
                for layer in mdl.layers:
                    h = layer(h, attention_mask=None, position_ids=position_ids, past_key_values=past_key_values,
                              use_cache=use_cache, position_embeddings=pe, current_ut=ut)
            h = mdl.norm(h)
            return types.SimpleNamespace(logits=self.base.lm_head(h[:, -logits_to_keep:]))

    return Looped().eval()


def test_looped_model_slots_vs_oracle_and_graph():
    """2 layers x 2 loops = 4 slots.  The fused arm at every slot and decode
    step against the oracle over that slot's packed bytes (the loops write
    different K/V, so a wrong slot mapping fails), then the same decode as a
    HIP graph equals its eager device-position steps bit for bit."""
    base, cfg, ids = model()
    m = looped(base, 2)
    scale = base.model.layers[0].self_attn.scaling
    restore = adapter.install(base)
    try:
        cache = adapter.PackedKVCache(cfg, B, 1024, loops=2, arm="PACKED_KV_FUSED", max_prefill=P)
        seen = []

        def capture(slot, total, q, out):
            k, v = slot_kv_oracle(cache, slot)
            ref, _ = O.decode_attention64(q.float().cpu().numpy(), k, v, scale=scale)
            err = np.abs(out.float().cpu().numpy() - ref)
            assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), (slot, total, float(err.max()))
            seen.append(slot)

        cache.capture = capture
        adapter.greedy(m, cache, ids, 10)
        assert sorted(set(seen)) == [0, 1, 2, 3] and len(seen) == 40
        # loop 1 re-applies the layers to different hidden states: its K differ from loop 0's
        assert not torch.equal(cache.store.side(0, "K").tail, cache.store.side(2, "K").tail)

        tokens = torch.randint(0, 256, (B, 70), generator=torch.Generator().manual_seed(6)).to(DEV)
        outs = {}
        for use_graph in (False, True):
            c = adapter.PackedKVCache(cfg, B, 1024, loops=2, arm="PACKED_KV_FUSED", max_prefill=P, strict=False)
            with torch.no_grad():
                m(input_ids=ids, past_key_values=c, use_cache=True)
            c.post_prefill()
            dg = adapter.DecodeGraph(m, c, use_graph=use_graph)
            outs[use_graph] = torch.stack([dg.step(tokens[:, i:i + 1])[:, -1].float().clone() for i in range(70)])
            c.check_status()
            assert c.store.length == [P + 70] * 4 and c.store.compressed == [128] * 4
        assert torch.equal(outs[True], outs[False])
    finally:
        restore()


@pytest.mark.parametrize("tail_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shared_rows,fused", [(True, False), (False, False), (False, True)])
def test_rope_append_matches_transformers_rotary_bitwise(dtype, shared_rows, fused, tail_dtype):
    """nsn_rope_append against transformers' own apply_rotary_pos_emb (Llama
    rotary, the model dtype's rounding) and a plain cast of k and v to the
    tail dtype (fp16 or bf16): the rotated q and the appended tail rows are
    bit-identical, at a host offset and at a device tail end; other tail rows
    stay untouched."""
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb
    from nsn_amd import _dev, _lib
    lib = _lib.lib()
    b_, hq, hkv, cap = 3, 8, 2, 10
    cfg = LlamaConfig(hidden_size=1024, num_attention_heads=hq, num_key_value_heads=hkv, head_dim=128,
                      max_position_embeddings=8192)
    rot = LlamaRotaryEmbedding(cfg).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(8)
    if fused:   # slices of one fused QKV projection row, as the adapter passes them
        qkv = (torch.randn((b_, 1, (hq + 2 * hkv) * 128), generator=g, device=DEV) * 3).to(dtype)
        q, k, v = qkv[..., :hq * 128], qkv[..., hq * 128:(hq + hkv) * 128], qkv[..., (hq + hkv) * 128:]
    else:
        q = (torch.randn((b_, 1, hq * 128), generator=g, device=DEV) * 3).to(dtype)
        k = (torch.randn((b_, 1, hkv * 128), generator=g, device=DEV) * 3).to(dtype)
        v = torch.randn((b_, 1, hkv * 128), generator=g, device=DEV).to(dtype)
    pos = torch.tensor([[517]], device=DEV) if shared_rows else torch.tensor([[17], [517], [4000]], device=DEV)
    cos, sin = rot(q, pos)
    cos, sin = cos.contiguous(), sin.contiguous()
    qr, kr = apply_rotary_pos_emb(q.reshape(b_, 1, hq, 128).transpose(1, 2),
                                  k.reshape(b_, 1, hkv, 128).transpose(1, 2), cos, sin)
    for device_end in (False, True):
        q_out = torch.empty((b_, hq, 128), dtype=dtype, device=DEV)
        kt = torch.zeros((b_ * hkv, cap, 128), dtype=tail_dtype, device=DEV)
        vt = torch.zeros_like(kt)
        st = _dev.new_status(DEV)
        end_t = torch.tensor([5], dtype=torch.int32, device=DEV)
        rc = lib.nsn_rope_append(q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0), cos.data_ptr(),
                                 sin.data_ptr(),
                                 0 if shared_rows else 128, b_, hq, hkv, q_out.data_ptr(), kt.data_ptr(), vt.data_ptr(),
                                 cap, end_t.data_ptr() if device_end else None, 4, _dev.dtype_code(dtype),
                                 _dev.dtype_code(tail_dtype), st.data_ptr(), _dev.stream())
        assert rc == 0 and _dev.read_status(st) == 0
        assert torch.equal(q_out.view(torch.int16), qr[:, :, 0].contiguous().view(torch.int16))
        want_k = kr[:, :, 0].to(tail_dtype).reshape(b_ * hkv, 128)
        want_v = v.reshape(b_ * hkv, 128).to(tail_dtype)
        assert torch.equal(kt[:, 4].view(torch.int16), want_k.view(torch.int16))
        assert torch.equal(vt[:, 4].view(torch.int16), want_v.view(torch.int16))
        rest = torch.ones(cap, dtype=torch.bool)
        rest[4] = False
        assert not kt[:, rest].any() and not vt[:, rest].any()


def test_generate_with_auto_policy_matches_the_manual_policy():
    """transformers' generate() never calls post_prefill / post_decode; with
    auto_policy each slot applies the pending policy right before its next
    append, which leaves the same cache state at every attention: the
    greedy tokens equal the manual loop's, across a compression."""
    m, cfg, ids = model()
    m.generation_config.eos_token_id = None
    m.generation_config.pad_token_id = 0
    restore = adapter.install(m)
    try:
        manual = adapter.PackedKVCache(cfg, B, 1024, max_prefill=P)
        want, _ = adapter.greedy(m, manual, ids, 90)
        auto = adapter.PackedKVCache(cfg, B, 1024, max_prefill=P, auto_policy=True)
        with torch.no_grad():
            out = m.generate(ids, past_key_values=auto, max_new_tokens=90, do_sample=False)
    finally:
        restore()
    assert torch.equal(out[:, P:], want)
    assert auto.store.compressed == [128, 128] == manual.store.compressed
