"""The int4 path inside a transformers Qwen3 model (random init, no weights
needed): decode-time append into the int4 cache and the sparse attention
function behind transformers' attention interface.

* With every block kept, the decode logits equal dense SDPA's within bf16
  tolerance (the selection covers the whole cache, so only the attention
  arithmetic differs).
* With a sparse selection, the packed K, scales and slab that were appended
  token by token equal the oracle's on the final K (bit-exact); the channel
  subset is the one chosen when the int4 cache was built.
* ``generate`` runs end to end on the cache."""

import numpy as np
import pytest
import torch

from kv_cache_amd import hf
from oracle import qkv_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(layers=2):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      rope_theta=1.0e6)
    return Qwen3ForCausalLM(cfg).to(DEV, torch.bfloat16).eval()


def _decode(model, impl, cache, prompt, steps):
    model.config._attn_implementation = impl
    logits = []
    with torch.no_grad():
        out = model(prompt, past_key_values=cache, use_cache=True)
        nxt = out.logits[:, -1:].argmax(-1)
        for i in range(steps):
            out = model(nxt, past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
            # teacher-force a fixed token stream so both runs see the same inputs
            nxt = torch.full_like(nxt, (37 * i + 11) % 512)
    return logits


def test_all_blocks_kept_matches_dense():
    from transformers.cache_utils import DynamicCache

    hf.register()
    model = _model()
    prompt = torch.randint(0, 512, (2, 300), generator=torch.Generator().manual_seed(1)).to(DEV)
    cache = hf.Int4SparseCache(capacity=1024, group=32, selected=32, block=16, topk=64)   # 64 x 16 = all
    got = _decode(model, "int4_sparse", cache, prompt, 6)
    want = _decode(model, "sdpa", DynamicCache(config=model.config), prompt, 6)
    for g, w in zip(got, want):
        torch.testing.assert_close(g, w, rtol=3e-2, atol=3e-2)
    assert all(layer.int4 is not None for layer in cache.layers)
    assert cache.get_seq_length() == 306


def test_append_matches_rebuild():
    hf.register()
    model = _model()
    prompt = torch.randint(0, 512, (1, 200), generator=torch.Generator().manual_seed(2)).to(DEV)
    cache = hf.Int4SparseCache(capacity=512, group=32, selected=32, block=16, topk=4)
    logits = _decode(model, "int4_sparse", cache, prompt, 9)
    assert all(torch.isfinite(x).all() for x in logits)
    t = cache.get_seq_length()
    assert t == 209
    for layer in cache.layers:
        c = layer.int4
        assert c.tokens == t
        k = layer.keys.float().cpu().numpy().reshape(2, t, 128)          # 2 KV heads
        want_p, want_s = O.int4_pack_k(k, 32)
        assert np.array_equal(c.packed[0, :, :t].cpu().numpy(), want_p)
        assert np.array_equal(c.scales[0, :, :t].contiguous().cpu().view(torch.int16).numpy().view(np.uint16),
                              want_s)
        # channels chosen when the int4 cache was built: prefill + the first decode token
        pp, ps = O.int4_pack_k(k[:, :201], 32)
        chan = O.select_channels(O.channel_stats(pp, ps, 32), 32)
        assert np.array_equal(c.chan_idx[0].cpu().numpy(), chan)
        slab, sbits = O.build_slab(k, chan)
        stored = c.slab[0].cpu().numpy().reshape(2, -1)
        assert np.array_equal(O.unswizzle_slab(stored, 32, t), slab)
        assert np.array_equal(c.slab_scales[0, :, :t].contiguous().cpu().view(torch.int16).numpy().view(np.uint16),
                              sbits)


def test_generate_runs():
    hf.register()
    model = _model()
    model.config._attn_implementation = "int4_sparse"
    prompt = torch.randint(0, 512, (1, 150), generator=torch.Generator().manual_seed(3)).to(DEV)
    cache = hf.Int4SparseCache(capacity=256, group=32, selected=32, block=16, topk=4)
    with torch.no_grad():
        out = model.generate(prompt, past_key_values=cache, max_new_tokens=8, do_sample=False)
    assert out.shape == (1, 158)
    assert cache.get_seq_length() == 157


def test_keep_self_flag():
    # every history block kept: with keep_self (the reference's default) the
    # attention covers the whole cache and equals dense SDPA; without it the
    # current token is left out, as the reference's --always_keep_self false
    from transformers.cache_utils import DynamicCache

    hf.register()
    model = _model(layers=1)
    prompt = torch.randint(0, 512, (1, 120), generator=torch.Generator().manual_seed(4)).to(DEV)
    want = _decode(model, "sdpa", DynamicCache(config=model.config), prompt, 3)
    kept = _decode(model, "int4_sparse", hf.Int4SparseCache(capacity=512, topk=32, keep_self=True), prompt, 3)
    dropped = _decode(model, "int4_sparse", hf.Int4SparseCache(capacity=512, topk=32, keep_self=False), prompt, 3)
    for g, w in zip(kept, want):
        torch.testing.assert_close(g, w, rtol=3e-2, atol=3e-2)
    assert max(float((d - k).abs().max()) for d, k in zip(dropped, kept)) > 1e-3


def test_protected_tokens_flow_through():
    # a one-block selection plus sink / recent tokens: logits stay finite and
    # differ from the same cache without protection
    hf.register()
    model = _model(layers=1)
    prompt = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(5)).to(DEV)
    a = _decode(model, "int4_sparse", hf.Int4SparseCache(capacity=512, topk=1, protect_sink=8, protect_recent=32),
                prompt, 3)
    b = _decode(model, "int4_sparse", hf.Int4SparseCache(capacity=512, topk=1), prompt, 3)
    assert all(torch.isfinite(x).all() for x in a)
    assert max(float((x - y).abs().max()) for x, y in zip(a, b)) > 1e-3


def test_padded_batch_is_refused_at_decode():
    # the int4 kernels take no per-token mask: a left-padded batch must not
    # silently attend to its padding
    hf.register()
    model = _model(layers=1)
    model.config._attn_implementation = "int4_sparse"
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(6)).to(DEV)
    mask = torch.ones((2, 40), dtype=torch.long, device=DEV)
    mask[0, :7] = 0
    cache = hf.Int4SparseCache(capacity=128, topk=2)
    with torch.no_grad():
        model(ids, attention_mask=mask, past_key_values=cache, use_cache=True)     # prefill: SDPA with the mask
        with pytest.raises(RuntimeError, match="padded batches"):
            model(ids[:, :1], attention_mask=torch.cat([mask, mask[:, :1] * 0 + 1], dim=1), past_key_values=cache,
                  use_cache=True)


def test_decode_output_survives_the_next_step():
    # the attention output of one decode step is a tensor of its own: the
    # next step does not overwrite it
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    hf.register()
    model = _model(layers=1)
    kept = []
    fn = ALL_ATTENTION_FUNCTIONS["int4_sparse"]

    def rec(module, query, key, value, attention_mask, **kw):
        out, w = fn(module, query, key, value, attention_mask, **kw)
        if query.size(2) == 1:
            kept.append((out, out.clone()))
        return out, w

    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

    AttentionInterface.register("rec_int4_sparse", rec)
    AttentionMaskInterface.register("rec_int4_sparse", sdpa_mask)
    prompt = torch.randint(0, 512, (1, 200), generator=torch.Generator().manual_seed(6)).to(DEV)
    _decode(model, "rec_int4_sparse", hf.Int4SparseCache(capacity=512, topk=4), prompt, 4)
    assert len(kept) == 4
    for out, copy in kept:
        assert torch.equal(out, copy)


NATIVE_MODES = [
    ("qabs8cand5reuse", {"top_fraction": 0.05, "protect_sink": 4, "protect_recent": 8}),
    ("qabs8cand5reusefinal", {"top_fraction": 0.05}),
    ("qdriftheadqabs8cand5", {"top_fraction": 0.05}),
    ("lagrefresh3qabs8cand5", {"top_fraction": 0.05}),
    ("qabs8cand5attn", {"protect_sink": 4}),
    ("qabs8cand10r2attn", {}),
    ("qbb16q8s50cand10", {"top_fraction": 0.05}),
    ("brep16r2q8s50cand10", {"top_fraction": 0.05}),
    ("qboracle16q8s50cand10", {"top_fraction": 0.05}),
]


def _record(name):
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    fn = ALL_ATTENTION_FUNCTIONS[name]
    calls = []

    def rec(module, query, key, value, attention_mask, scaling=None, **kw):
        out, w = fn(module, query, key, value, attention_mask, scaling=scaling, **kw)
        if query.size(2) == 1:
            calls.append((module, query.clone(), key.clone(), value.clone(), scaling, out.clone()))
        return out, w

    AttentionInterface.register("rec_" + name, rec)
    AttentionMaskInterface.register("rec_" + name, sdpa_mask)
    return "rec_" + name, calls


@pytest.mark.parametrize("mode,kw", NATIVE_MODES, ids=[m for m, _ in NATIVE_MODES])
def test_native_mode_decode_equals_its_step(mode, kw):
    # the HF entry runs the mode's decode step per layer with the cache's K/V:
    # a fresh step fed the recorded decode calls of one layer reproduces the
    # outputs the model saw, step by step (the step's own state included)
    from transformers.cache_utils import DynamicCache

    name = hf.register_mode(mode, 512, **kw)
    rec_name, calls = _record(name)
    model = _model()
    prompt = torch.randint(0, 512, (2, 220), generator=torch.Generator().manual_seed(7)).to(DEV)
    logits = _decode(model, rec_name, DynamicCache(config=model.config), prompt, 5)
    assert all(torch.isfinite(x).all() for x in logits)
    assert len(calls) == 2 * 5
    cls = hf.native_step_class(mode)
    assert all(type(s) is cls for s in hf.ATTENTION_STEPS[name].values())
    for layer_module in {c[0] for c in calls}:
        seq = [c for c in calls if c[0] is layer_module]
        b, hq, _, d = seq[0][1].shape
        step = cls(mode, b, hq, seq[0][2].size(1), d, 512, device=DEV, **kw)
        for _, q, k, v, scaling, out in seq:
            got = step(q[:, :, 0, :], k, v, d ** -0.5 if scaling is None else scaling)
            assert torch.equal(got[:, None], out)


@pytest.mark.parametrize("mode,kw", [("qabs8cand100reuse", {"top_fraction": 1.0}), ("qabs8cand100attn", {}),
                                     ("qbb16q8s100cand100", {"top_fraction": 1.0})],
                         ids=["reuse", "attn", "qbb"])
def test_native_mode_keeping_everything_matches_dense(mode, kw):
    from transformers.cache_utils import DynamicCache

    name = hf.register_mode(mode, 512, **kw)
    model = _model()
    prompt = torch.randint(0, 512, (1, 180), generator=torch.Generator().manual_seed(8)).to(DEV)
    got = _decode(model, name, DynamicCache(config=model.config), prompt, 4)
    want = _decode(model, "sdpa", DynamicCache(config=model.config), prompt, 4)
    for g, w in zip(got, want):
        torch.testing.assert_close(g, w, rtol=3e-2, atol=3e-2)


def test_native_mode_generate_runs():
    from transformers.cache_utils import DynamicCache

    name = hf.register_mode("qabs8cand5reuse", 512, top_fraction=0.05)
    model = _model()
    model.config._attn_implementation = name
    prompt = torch.randint(0, 512, (1, 150), generator=torch.Generator().manual_seed(9)).to(DEV)
    with torch.no_grad():
        out = model.generate(prompt, past_key_values=DynamicCache(config=model.config), max_new_tokens=6,
                             do_sample=False)
    assert out.shape == (1, 156)


def test_register_mode_rejects_unknown_modes():
    with pytest.raises(ValueError):
        hf.register_mode("int4foo", 512)
