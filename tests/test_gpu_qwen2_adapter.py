"""The Qwen2 adapter end to end on a small random-weight Qwen2 (transformers 5.x): PhaseKV
decode steps and an input chunk against the model's own dense DynamicCache decode on the
same tokens, and a prefill with prompt selection."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(gpu, attn="sdpa", layers=2, dtype=torch.float16):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=2000, hidden_size=512, intermediate_size=1024,
                      num_hidden_layers=layers, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=8192, attn_implementation=attn)
    torch.manual_seed(0)
    with torch.device(gpu):
        model = Qwen2ForCausalLM(cfg)
    for p in model.parameters():           # wider weights than the default init, so the
        p.data.normal_(0.0, 0.06)          # logits spread and small errors would show
    return model.to(dtype).eval()


def _close(a, b):
    a, b = a.float().flatten(), b.float().flatten()
    cos = torch.nn.functional.cosine_similarity(a, b, dim=0).item()
    rel = ((a - b).abs().max() / b.abs().max()).item()
    return cos, rel


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@torch.no_grad()
def test_decode_and_chunk_match_the_dense_cache(gpu, dtype):
    """fp16 and bf16 models (both take the fused RoPE append in decode steps)."""
    from transformers import DynamicCache
    from phasekv_amd.qwen2_attention import (install_qwen2_phasekv_attention, phasekv_prefill,
                                             phasekv_step)
    print(f"case dtype={dtype}", flush=True)
    model = _model(gpu, dtype=dtype)
    install_qwen2_phasekv_attention(model)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, 2000, (1, 300), generator=g).to(gpu)
    first, cache = phasekv_prefill(model, prompt, prompt_bits=8, cold_bits=8, recent_window=32,
                                   lazy_g=16)
    dense = DynamicCache(config=model.config)
    ref = model(prompt, past_key_values=dense, use_cache=True).logits[:, -1]
    assert torch.equal(first, ref)                      # the prefill itself is the model's
    tok = ref.argmax(-1, keepdim=True)
    worst = 1.0
    for step in range(60):
        mine = phasekv_step(model, tok, cache)
        want = model(tok, past_key_values=dense, use_cache=True).logits[:, -1]
        cos, rel = _close(mine, want)
        worst = min(worst, cos)
        assert cos > 0.999 and rel < 0.05, (step, cos, rel)
        tok = want.argmax(-1, keepdim=True)
    tiers = cache.layer_tiers(0)
    assert len(tiers.cold) == 1 and cache.true_seq_length == 360
    # a new 12-token input chunk, attended in one pass per layer
    chunk = torch.randint(0, 2000, (1, 12), generator=g).to(gpu)
    mine = phasekv_step(model, chunk, cache)
    want = model(chunk, past_key_values=dense, use_cache=True).logits[:, -1]
    cos, rel = _close(mine, want)
    assert cos > 0.999 and rel < 0.05, (cos, rel)
    assert cache.true_seq_length == 372 and len(cache.layer_tiers(1).prompt_extensions) == 1
    print(f"worst decode cosine {worst:.6f}")


@torch.no_grad()
def test_prefill_with_prompt_selection(gpu):
    from phasekv_amd.qwen2_attention import (install_qwen2_phasekv_attention, phasekv_prefill,
                                             phasekv_step)
    model = _model(gpu, attn="eager")
    install_qwen2_phasekv_attention(model)
    prompt = torch.randint(0, 2000, (1, 256), generator=torch.Generator().manual_seed(2)).to(gpu)
    _, cache = phasekv_prefill(model, prompt, prefill_keep_ratio=0.5, sink_tokens=4,
                               obs_window=32, pool_kernel=7)
    assert cache.layer_tiers(0).prompt.length == 128 and cache.true_seq_length == 256
    logits = phasekv_step(model, prompt[:, -1:], cache)
    assert torch.isfinite(logits).all() and cache.true_seq_length == 257


@torch.no_grad()
def test_llama_adapter_matches_the_dense_cache(gpu):
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM
    from phasekv_amd.llama_attention import (install_llama_phasekv_attention, phasekv_prefill,
                                             phasekv_step)
    cfg = LlamaConfig(vocab_size=2000, hidden_size=512, intermediate_size=1024,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=8192, attn_implementation="sdpa")
    torch.manual_seed(0)
    with torch.device(gpu):
        model = LlamaForCausalLM(cfg)
    for p in model.parameters():
        p.data.normal_(0.0, 0.06)
    model = model.half().eval()
    install_llama_phasekv_attention(model)
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 2000, (1, 200), generator=g).to(gpu)
    _, cache = phasekv_prefill(model, prompt, prompt_bits=8, cold_bits=8)
    dense = DynamicCache(config=cfg)
    tok = model(prompt, past_key_values=dense, use_cache=True).logits[:, -1].argmax(-1, keepdim=True)
    for step in range(52):
        mine = phasekv_step(model, tok, cache)
        want = model(tok, past_key_values=dense, use_cache=True).logits[:, -1]
        cos, rel = _close(mine, want)
        assert cos > 0.999 and rel < 0.05, (step, cos, rel)
        tok = want.argmax(-1, keepdim=True)
    chunk = torch.randint(0, 2000, (1, 9), generator=g).to(gpu)
    cos, rel = _close(phasekv_step(model, chunk, cache),
                      model(chunk, past_key_values=dense, use_cache=True).logits[:, -1])
    assert cos > 0.999 and rel < 0.05 and len(cache.layer_tiers(0).cold) == 1


def _np_packed(pt):
    from oracle import packing_oracle as po
    return po.PackedArrays(pt.packed.cpu().numpy(), pt.scale.cpu().numpy(), pt.mins.cpu().numpy(),
                           pt.bits, pt.axis, pt.group_size, tuple(pt.orig_shape), pt.axis_len)


def _tier_arrays(tiers, hot_rows=None):
    """The layer's tiers as they stand, copied to the host (hot window cut at ``hot_rows``)."""
    from oracle import attention_oracle as ao
    seg = lambda s: ao.SegmentArrays(_np_packed(s.key), _np_packed(s.value))
    hk, hv = tiers.hot_views()
    if hot_rows is not None:
        hk, hv = tiers.hot_k[:, :, :hot_rows], tiers.hot_v[:, :, :hot_rows]
    return ao.LayerTiersArrays(seg(tiers.prompt), [seg(s) for s in tiers.prompt_extensions],
                               [seg(s) for s in tiers.cold], hk.cpu().numpy(), hv.cpu().numpy())


@torch.no_grad()
def test_adapter_attention_matches_the_oracle_on_its_own_tiers(gpu, monkeypatch):
    """Every attention call the adapter makes in a recorded step, against the float64 oracle
    over the same packed tiers and the same q, at the decode bar (max-abs 2e-3, relative
    1e-2): decode steps before and after a cooling, in both layers, and an input chunk
    (each chunk token against the tiers as they stand after its append)."""
    from oracle import attention_oracle as ao
    from phasekv_amd import qwen2_attention as qa
    model = _model(gpu)
    qa.install_qwen2_phasekv_attention(model)
    hq = model.config.num_attention_heads
    record = {"on": False, "decode": [], "chunk": []}
    decode, chunk = qa.fused_phasekv_decode, qa.fused_phasekv_prompt_chunk_attention

    def rec_decode(q, tiers, h, **kw):
        out = decode(q, tiers, h, **kw)
        if record["on"]:
            record["decode"].append((q.cpu().numpy(), _tier_arrays(tiers), out.float().cpu().numpy()))
        return out

    def rec_chunk(q, tiers, h, **kw):
        out = chunk(q, tiers, h, **kw)
        if record["on"]:
            T = q.shape[0]
            start = tiers.hot_len - T
            record["chunk"].append((q.cpu().numpy(), [_tier_arrays(tiers, start + t + 1)
                                                      for t in range(T)], out.float().cpu().numpy()))
        return out

    monkeypatch.setattr(qa, "fused_phasekv_decode", rec_decode)
    monkeypatch.setattr(qa, "fused_phasekv_prompt_chunk_attention", rec_chunk)
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, 2000, (1, 300), generator=g).to(gpu)
    first, cache = qa.phasekv_prefill(model, prompt, prompt_bits=2, cold_bits=4,
                                      recent_window=32, lazy_g=16)
    tok = first.argmax(-1, keepdim=True)
    recorded = (0, 1, 47, 48, 49, 59)
    for step in range(60):
        record["on"] = step in recorded
        tok = qa.phasekv_step(model, tok, cache).argmax(-1, keepdim=True)
    assert len(cache.layer_tiers(0).cold) == 1     # a cooling happened between the records
    record["on"] = True
    qa.phasekv_step(model, torch.randint(0, 2000, (1, 11), generator=g).to(gpu), cache)
    assert len(record["decode"]) == 2 * len(recorded) and len(record["chunk"]) == 2
    for i, (q, tiers, got) in enumerate(record["decode"]):
        want = ao.layer_tiers_attention(q, tiers, hq)
        np.testing.assert_allclose(got, want, atol=2e-3, rtol=1e-2, err_msg=f"decode call {i}")
    for i, (q, per_token, got) in enumerate(record["chunk"]):
        want = np.stack([ao.layer_tiers_attention(q[t], per_token[t], hq)
                         for t in range(q.shape[0])])
        np.testing.assert_allclose(got, want, atol=2e-3, rtol=1e-2, err_msg=f"chunk call {i}")
