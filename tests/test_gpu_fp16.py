"""fp16 q/K/V through every 16-bit entry point: the int4 path (pack, slab,
query words, scoring, top-k, attention), the block selectors, the reuse and
candidate-attention steps, prefill query quantization, the drop-in
final_attention and the HF cache.  Same bars as the bf16 tests: integer,
index and mask work bit-exact against the oracle (which takes the fp16
values as exact fp32), attention within 1e-2 relative / 2e-2 absolute of
fp64; mixed dtypes and fp32 are refused."""

import numpy as np
import pytest
import torch

from kv_cache_amd import _lib
from kv_cache_amd import blocksel as BS
from kv_cache_amd import int4 as K
from kv_cache_amd import prefill as P
from kv_cache_amd import qabs_cuda_kernels as Q
from kv_cache_amd import reuse as RU
from oracle import qkv_oracle as O
from oracle import ref_semantics as R

pytestmark = pytest.mark.gpu
DEV = "cuda"
H = torch.float16
RTOL, ATOL = 1e-2, 2e-2


def f32(t):
    return t.float().cpu().numpy()


def bits16(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def rand_k(b, h, t, d, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((b, h, t, d), generator=g) * scale
    k[..., 3] *= 8.0
    return k.to(H)


# ---------------------------------------------------------------------------
# int4 structures
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("group", [32, 64, 128])
def test_pack_matches_oracle(group):
    key = rand_k(2, 3, 300, 128, seed=group + 1).to(DEV)
    packed, scales = K.int4_pack_k(key, group)
    want_p, want_s = O.int4_pack_k(f32(key), group)
    assert np.array_equal(packed[:, :, :300].cpu().numpy(), want_p)
    assert np.array_equal(bits16(scales[:, :, :300]), want_s)


def test_pack_fp16_range_ends():
    # the largest finite fp16, the smallest subnormal, a row of subnormals and
    # one mixing both ends: scales saturate / underflow exactly as the oracle says
    rows = torch.zeros((1, 1, 6, 128), dtype=torch.float32)
    tiny = 2.0 ** -24
    kat = [[65504.0, -65504.0, 7.0, 0.0], [tiny, 0, 0, 0], [7 * tiny, -3 * tiny, tiny, 0],
           [65504.0, tiny, -tiny, 1.0], [-0.0, 0.0, 0.0, 0.0], [6.1e-5, -6.1e-5, 3.0e-5, 0.0]]
    for t, vals in enumerate(kat):
        rows[0, 0, t, :4] = torch.tensor(vals)
    key = rows.to(H).to(DEV)
    packed, scales = K.int4_pack_k(key, 32)
    want_p, want_s = O.int4_pack_k(f32(key), 32)
    assert np.array_equal(packed[..., :6, :].cpu().numpy(), want_p)
    assert np.array_equal(bits16(scales[..., :6, :]), want_s)
    # 65504 / 7 -> fp16 9360; 2^-24 / 7 underflows to a zero scale (codes 0);
    # 7 * 2^-24 / 7 is the smallest subnormal exactly
    assert bits16(scales)[0, 0, :5, 0].tolist() == [0x7092, 0, 0x0001, 0x7092, 0]


@pytest.mark.parametrize("count", [16, 32, 64, 128])
def test_slab_matches_oracle(count):
    key = rand_k(1, 3, 513, 128, seed=200 + count).to(DEV)
    g = torch.Generator().manual_seed(count)
    chan = torch.stack([torch.randperm(128, generator=g)[:count].sort().values for _ in range(3)])
    chan = chan.view(1, 3, count).to(torch.int32).to(DEV)
    slab, ss = K.build_slab(key, chan)
    want, want_s = O.build_slab(f32(key).reshape(3, 513, 128), chan.cpu().numpy().reshape(3, count))
    stored = slab.cpu().numpy().reshape(3, -1)
    assert np.array_equal(O.unswizzle_slab(stored, count, 513), want)
    assert np.array_equal(bits16(ss[:, :, :513]).reshape(3, 513), want_s)


@pytest.mark.parametrize("count", [16, 32, 64, 128])
def test_query_words_match_oracle(count):
    g = torch.Generator().manual_seed(count + 5)
    b, hq, hkv = 2, 16, 4
    q = (torch.randn((b, hq, 128), generator=g) * 3).to(H)
    chan = torch.stack([torch.randperm(128, generator=g)[:count].sort().values for _ in range(b * hkv)])
    chan = chan.view(b, hkv, count).to(torch.int32)
    words, qs = K.query_words(q.to(DEV), chan.to(DEV), qscale=torch.empty((b, hkv), device=DEV))
    q8, want_qs = O.quantize_query_group(f32(q), chan.numpy().reshape(b * hkv, count), hkv)
    assert np.array_equal(words.cpu().numpy().reshape(b * hkv, count // 4).view(np.uint32), O.pack_query_words(q8))
    assert np.array_equal(qs.cpu().numpy().reshape(-1), want_qs)


@pytest.mark.parametrize("count,block", [(16, 1), (32, 16), (64, 64), (128, 16)])
def test_decode_scores_match_oracle(count, block):
    b, hq, hkv, t = 2, 8, 4, 1000
    g = torch.Generator().manual_seed(count * 3 + block)
    key = rand_k(b, hkv, t, 128, seed=count + block).to(DEV)
    q = torch.randn((b, hq, 128), generator=g).to(H).to(DEV)
    cache = K.Int4KCache.from_prefill(key, 32 if count <= 32 else 128, count)
    bmax, isum, keys, qs = K.decode_scores(q, cache.chan_idx, cache.slab, cache.slab_scales, t, block, debug=True)
    rows = b * hkv
    chan = cache.chan_idx.cpu().numpy().reshape(rows, count)
    slab = O.unswizzle_slab(cache.slab.cpu().numpy().reshape(rows, -1), count, t)
    sbits = bits16(cache.slab_scales[:, :, :t]).reshape(rows, t)
    q8, want_qs = O.quantize_query_group(f32(q), chan, hkv)
    want_i = O.partial_scores_i32(q8, slab)
    want_k = O.ranking_keys(want_i, sbits)
    assert np.array_equal(qs.cpu().numpy().reshape(rows), want_qs)
    assert np.array_equal(isum.cpu().numpy().reshape(rows, t), want_i)
    assert np.array_equal(keys.cpu().numpy().reshape(rows, t).view(np.uint32), want_k.view(np.uint32))
    assert np.array_equal(bmax.cpu().numpy().reshape(rows, -1), O.block_max(want_k, block))


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _qkv(b, hq, hkv, t, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((b, hq, 128), generator=gen).to(H)
    k = (torch.randn((b, hkv, t, 128), generator=gen) * 2).to(H)
    v = torch.randn((b, hkv, t, 128), generator=gen).to(H)
    return q, k, v, gen


@pytest.mark.parametrize("g_size", [1, 2, 4, 8])
@pytest.mark.parametrize("block,nsel", [(1, 300), (16, 128), (64, 7)])
def test_sparse_attention_matches_fp64(g_size, block, nsel):
    b, hkv, t = 2, 2, 3000
    q, k, v, gen = _qkv(b, hkv * g_size, hkv, t, g_size * 100 + block)
    nb = -(-t // block)
    sel = torch.stack([torch.randperm(nb, generator=gen)[:nsel].sort().values for _ in range(b * hkv)])
    sel = sel.view(b, hkv, nsel).to(torch.int32)
    sel[0, 0, 0] = -1
    sel[0, 1, -1] = nb - 1
    out = K.sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV), block, t, 128 ** -0.5)
    assert out.dtype == H
    want = O.sparse_attention(f32(q), f32(k), f32(v), sel.numpy(), block, t, 128 ** -0.5)
    assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("g_size,batch,t,block,nsel", [(2, 8, 20000, 16, 1024), (4, 2, 40000, 64, 300),
                                                       (8, 1, 9000, 1, 4000)])
def test_sparse_attention_long_selections(g_size, batch, t, block, nsel):
    # several splits per row: the merge of split partials in fp16 output
    hkv = 2
    q, k, v, gen = _qkv(batch, hkv * g_size, hkv, t, t + nsel)
    nb = -(-t // block)
    sel = torch.stack([torch.randperm(nb, generator=gen)[:nsel].sort().values for _ in range(batch * hkv)])
    sel = sel.view(batch, hkv, nsel).to(torch.int32)
    out = K.sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV), block, t, 0.09)
    for bi in range(min(batch, 2)):
        want = O.sparse_attention(f32(q[bi:bi + 1]), f32(k[bi:bi + 1]), f32(v[bi:bi + 1]), sel[bi:bi + 1].numpy(),
                                  block, t, 0.09)
        assert np.allclose(f32(out[bi:bi + 1]), want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("g_size", [1, 4])
def test_sparse_attention_select_and_protected(g_size):
    b, hkv, t, block, nsel = 2, 2, 2500, 16, 40
    q, k, v, gen = _qkv(b, hkv * g_size, hkv, t + 1, 77 + g_size)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    nb = -(-t // block)
    bmax = torch.randn((b, hkv, nb), generator=gen).to(DEV)
    sel = torch.empty((b, hkv, nsel), dtype=torch.int32, device=DEV)
    out = K.sparse_attention_select(qd, kd, vd, bmax, nsel, block, t, 0.088, sel_out=sel)
    assert torch.equal(sel, K.block_topk(bmax, nsel))
    torch.testing.assert_close(out, K.sparse_attention(qd, kd, vd, sel, block, t, 0.088), rtol=0, atol=0)
    prot = K.sparse_attention_select(qd, kd, vd, bmax, nsel, block, t, 0.088, protect_sink=4, protect_recent=9,
                                     keep_self=True)
    want = O.sparse_attention_protected(f32(q), f32(k), f32(v), sel.cpu().numpy(), block, t, 0.088, 4, 9, True)
    assert np.allclose(f32(prot), want, rtol=RTOL, atol=ATOL)


def test_decode_step_matches_oracle():
    b, hq, hkv, t, block, topk = 1, 16, 4, 5000, 16, 64
    q, k, v, _ = _qkv(b, hq, hkv, t, 31)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    cache = K.Int4KCache.from_prefill(kd[:, :, : t - 1], 32, 32, capacity=K.round_capacity(t))
    step = K.SparseDecodeStep(b, hq, hkv, 128, t, block, topk, protect_sink=2, protect_recent=8, keep_self=True,
                              dtype=H)
    out = step(qd, cache, kd, vd, 0.088)
    assert out.dtype == H
    rows = b * hkv
    chan = cache.chan_idx.cpu().numpy().reshape(rows, 32)
    slab = O.unswizzle_slab(cache.slab.cpu().numpy().reshape(rows, -1), 32, t - 1)
    sbits = bits16(cache.slab_scales[:, :, : t - 1]).reshape(rows, t - 1)
    *_, want_sel = O.decode_select(f32(q), slab, sbits, chan, hkv, block, topk)
    assert np.array_equal(step.sel.cpu().numpy().reshape(rows, topk), want_sel)
    want = O.sparse_attention_protected(f32(q), f32(k), f32(v), want_sel.reshape(b, hkv, topk), block, t - 1, 0.088,
                                        2, 8, True)
    assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL)


def test_mixed_and_fp32_dtypes_are_refused():
    q, k, v, _ = _qkv(1, 4, 2, 64, 5)
    sel = torch.zeros((1, 2, 1), dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="share one dtype"):
        K.sparse_attention(q.to(DEV), k.to(torch.bfloat16).to(DEV), v.to(DEV), sel, 16, 64, 0.1)
    with pytest.raises(RuntimeError, match="bfloat16 or float16"):
        K.int4_pack_k(k.float().to(DEV), 32)
    step = K.SparseDecodeStep(1, 4, 2, 128, 64, 16, 2)   # bf16 step
    cache = K.Int4KCache.from_prefill(k.to(DEV), 32, 32)
    with pytest.raises(RuntimeError, match="this step runs on torch.bfloat16"):
        step(q.to(DEV), cache, k.to(DEV), v.to(DEV), 0.1)


# ---------------------------------------------------------------------------
# block selectors, reuse and candidate attention steps
# ---------------------------------------------------------------------------

KINDS = {BS.QBB: "qbb", BS.BREP: "brep", BS.QBORACLE: "qboracle"}


def test_qbb_metadata_is_exact_fp16():
    lib = _lib.load()
    t, block = 700, 16
    _, k, _, _ = _qkv(1, 2, 2, t, 9)
    kd = k.to(DEV)
    mb = -(-t // block)
    meta = torch.zeros(lib.qkv_block_meta_bytes(BS.QBB, 1, 2, mb, 1), dtype=torch.uint8, device=DEV)
    _lib.check(lib.qkv_block_meta_update(BS.QBB, kd.data_ptr(), _lib.strides(*kd.stride()), 1, 2, 128, block, 1, 0, t,
                                         meta.data_ptr(), mb, 1, _lib.stream_of(kd)))
    rec = meta.view(torch.float16).view(1, 2, mb, 2, 128)
    lo, hi = R.block_minmax(f32(k), block)
    assert np.array_equal(f32(rec[:, :, :, 0]), lo)
    assert np.array_equal(f32(rec[:, :, :, 1]), hi)


@pytest.mark.parametrize("mode,hq,hkv,t,steps", [
    ("qbb16q8s12cand4", 8, 2, 3000, 2),
    ("brep16r2q8s12cand4", 8, 2, 3000, 2),
    ("qboracle16q8s12cand4", 8, 2, 3000, 2),
    ("qbb32q8s6p25cand2", 32, 8, 9000, 1),
])
def test_block_select_step_matches_oracle(mode, hq, hkv, t, steps):
    kind, block, reps, dims, scan, cand = BS.parse_block_mode(mode)
    gen = torch.Generator().manual_seed(hq * t + 1)
    k = (torch.randn((1, hkv, t + steps, 128), generator=gen) * 1.5).to(H)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(H)
    qs = torch.randn((steps, 1, hq, 128), generator=gen).to(H)
    kd, vd = k.to(DEV), v.to(DEV)
    step = BS.BlockSelectDecodeStep(mode, 1, hq, hkv, 128, t + steps + 40, top_fraction=0.02, protect_sink=3,
                                    protect_recent=5, keep_self=True, dtype=H)
    step.prefill(kd[:, :, : t - 3])
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        assert out.dtype == H
        want, keep = R.block_select_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), KINDS[kind], block, dims,
                                         scan, cand, 0.02, 128 ** -0.5, 3, 5, True, reps)
        assert np.array_equal(step.final_mask().cpu().numpy(), keep), (mode, s)
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
    with pytest.raises(RuntimeError, match="takes torch.float16"):
        step(qs[0].to(torch.bfloat16).to(DEV), kd[:, :, :t], vd[:, :, :t], 0.1)


@pytest.mark.parametrize("mode", ["qabs8cand5reuse", "qabs16cand10reusefinalblk32"])
def test_reuse_step_matches_oracle(mode):
    hq, hkv, t, steps = 8, 2, 3000, 3
    gen = torch.Generator().manual_seed(len(mode))
    s_dims, cand, use_pc, use_pf, block = RU.parse_reuse_mode(mode)
    k = torch.randn((1, hkv, t + steps, 128), generator=gen).to(H)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(H)
    qs = torch.randn((steps, 1, hq, 128), generator=gen).to(H)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.ReuseDecodeStep(mode, 1, hq, hkv, 128, t + steps + 64, top_fraction=0.02, protect_sink=4,
                              protect_recent=8, dtype=H)
    step.prefill(kd[:, :, : t - 1])
    pc = pf = None
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, wc, wf = R.reuse_decode_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), s_dims, cand, 0.02, 4, 8,
                                           True, 128 ** -0.5, pc if use_pc else None, pf if use_pf else None, block)
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
        pc, pf = wc, wf


@pytest.mark.parametrize("mode", ["lagtop2qabs8cand5", "qdriftheadqabs8cand5", "lagrefresh2qabs8cand5"])
def test_lagged_step_matches_oracle(mode):
    # queries drifting slowly on some heads and jumping on others; masks
    # bit-exact at every step (these kinds never round scores to the dtype)
    gen = torch.Generator().manual_seed(len(mode) * 5 + 2)
    t, steps, hq, hkv = 2000, 4, 8, 2
    kind, param, dims, cand = RU.parse_lagged_mode(mode)
    eps = torch.tensor([0.02, 3.0, 0.05, 0.3, 0.01, 2.0, 0.1, 1.0]).view(1, 1, hq, 1)
    base = torch.randn((1, 1, hq, 128), generator=gen)
    q = ((base + eps * torch.randn((steps, 1, hq, 128), generator=gen)) / torch.sqrt(1 + eps * eps)).to(H)
    k = torch.randn((1, hkv, t + steps, 128), generator=gen).to(H)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(H)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.LaggedReuseDecodeStep(mode, 1, hq, hkv, 128, t + 64, top_fraction=0.02, protect_sink=4,
                                    protect_recent=8, dtype=H)
    prev = None
    for s in range(steps):
        n = t + s + 1
        out = step(q[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, wc, wf, prev, _ = R.lagged_reuse_decode_step(f32(q[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), kind,
                                                           param, dims, cand, 0.02, 4, 8, True, 128 ** -0.5, prev)
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)


def test_candidate_attention_step_matches_oracle():
    gen = torch.Generator().manual_seed(4)
    t = 6000
    k = torch.randn((1, 2, t + 1, 128), generator=gen).to(H)
    v = torch.randn((1, 2, t + 1, 128), generator=gen).to(H)
    q = torch.randn((1, 8, 128), generator=gen).to(H)
    step = RU.QabsCandidateAttentionStep("qabs8cand3attn", 1, 8, 2, 128, t + 64, protect_sink=4, protect_recent=8,
                                         dtype=H)
    out = step(q.to(DEV), k.to(DEV), v.to(DEV), 128 ** -0.5)
    assert out.dtype == H
    want, keep = R.qabs_attn_step(f32(q), f32(k), f32(v), 8, 0.03, 128 ** -0.5, 4, 8, True)
    np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
    assert np.array_equal(step.final_mask().cpu().numpy(), keep[..., :t])


# ---------------------------------------------------------------------------
# prefill query, drop-in final attention, HF cache
# ---------------------------------------------------------------------------

def test_prefill_quantize_query_matches_oracle():
    g = torch.Generator().manual_seed(8)
    q = torch.randn((2, 3, 77, 128), generator=g)
    q[..., 7] *= 8.0
    q = q.to(H)
    q8, qs = P.quantize_query(q.to(DEV))
    want, want_s = O.quantize_query_rows(q.float().numpy())
    assert np.array_equal(q8.cpu().numpy(), O.permute_prefill_query(want))
    assert np.array_equal(qs.cpu().numpy(), want_s)
    # the strided (non-16-byte) row path
    wide = torch.randn((40, 132), generator=g).to(H).to(DEV)
    q8s, qss = P.quantize_query(wide[:, :128])
    want, want_s = O.quantize_query_rows(f32(wide[:, :128]))
    assert np.array_equal(q8s.cpu().numpy(), O.permute_prefill_query(want))
    assert np.array_equal(qss.cpu().numpy(), want_s)


@pytest.mark.parametrize("n", [37, 1000])
def test_final_attention_routes_fp16_to_the_list_attention(n):
    g = torch.Generator().manual_seed(n)
    b, h, t = 2, 4, 3000
    q = torch.randn((b, h, 128), generator=g).to(H)
    k = torch.randn((b, h, t, 128), generator=g).to(H)
    v = torch.randn((b, h, t, 128), generator=g).to(H)
    idx = torch.randint(0, t, (b, h, n), generator=g)
    valid = torch.rand((b, h, n), generator=g) < 0.9
    idx[0, 0, 0] = t + 5
    valid[1, 2] = False
    out = Q.final_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), valid.to(DEV), 128 ** -0.5)
    assert out.shape == (b, 1, h, 128) and out.dtype == H
    want = R.final_attention(f32(q), f32(k), f32(v), idx.numpy(), valid.numpy(), 128 ** -0.5)
    assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL)
    assert torch.count_nonzero(out[1, 0, 2].float()) == 0


def test_hf_fp16_model_keeping_every_block_matches_dense():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from transformers.cache_utils import DynamicCache

    from kv_cache_amd import hf

    hf.register()
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      rope_theta=1.0e6)
    model = Qwen3ForCausalLM(cfg).to(DEV, H).eval()
    prompt = torch.randint(0, 512, (2, 300), generator=torch.Generator().manual_seed(1)).to(DEV)

    def decode(impl, cache):
        model.config._attn_implementation = impl
        logits = []
        with torch.no_grad():
            out = model(prompt, past_key_values=cache, use_cache=True)
            nxt = out.logits[:, -1:].argmax(-1)
            for i in range(5):
                out = model(nxt, past_key_values=cache, use_cache=True)
                logits.append(out.logits[:, -1].float())
                nxt = torch.full_like(nxt, (37 * i + 11) % 512)
        return logits

    cache = hf.Int4SparseCache(capacity=1024, group=32, selected=32, block=16, topk=64)
    got = decode("int4_sparse", cache)
    want = decode("sdpa", DynamicCache(config=model.config))
    for a, w in zip(got, want):
        torch.testing.assert_close(a, w, rtol=3e-2, atol=3e-2)
    assert all(layer.int4 is not None and layer.keys.dtype == H for layer in cache.layers)
