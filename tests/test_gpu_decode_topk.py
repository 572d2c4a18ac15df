"""qkv_int4_decode_topk (token scoring whose launch also builds the top-k's
chunk histograms, then the top-k from the row's floor) against the two
separate calls it replaces, decode_scores with block 1 and block_topk:
the same scores and the same indices, bit for bit, on every top-k path
(one launch, three launches, short rows, the staged path past 64 chunks),
every built channel count and heavily tied rows."""

import numpy as np
import pytest
import torch

from kv_cache_amd import int4 as K
from oracle import qkv_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _keys(b, hkv, t, pattern, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    if pattern == "normal":
        k = torch.randn((b, hkv, t, 128), generator=g, device=DEV)
        k[..., 3] *= 8.0
    elif pattern == "equal":      # every token the same: every score of a row equal
        k = torch.randn((b, hkv, 1, 128), generator=g, device=DEV).expand(b, hkv, t, 128).clone()
    elif pattern == "five":       # five token vectors in turn: five scores per row, ties at the boundary
        base = torch.randn((b, hkv, 5, 128), generator=g, device=DEV)
        k = base[:, :, torch.arange(t, device=DEV) % 5]
    elif pattern == "planted":    # a few tokens far above the rest, in one chunk
        k = torch.randn((b, hkv, t, 128), generator=g, device=DEV)
        k[:, :, 4096 * 3 : 4096 * 3 + 700] *= 6.0
    else:
        raise ValueError(pattern)
    return k.to(torch.bfloat16)


def _case(b, hkv, t, count, k, pattern, dtype=torch.bfloat16, seed=7):
    hq = hkv * 4
    key = _keys(b, hkv, t, pattern, seed)
    q = torch.randn((b, hq, 128), generator=torch.Generator().manual_seed(seed)).to(dtype).to(DEV)
    cache = K.Int4KCache.from_prefill(key, 32 if count <= 32 else 128, count)
    want_s = K.decode_scores(q, cache.chan_idx, cache.slab, cache.slab_scales, t, 1)
    want = K.block_topk(want_s, k)
    scores = torch.full((b, hkv, t), 7.0, device=DEV)
    got = K.decode_topk(q, cache.chan_idx, cache.slab, cache.slab_scales, t, k, scores=scores)
    assert torch.equal(scores.view(torch.int32), want_s.view(torch.int32))
    assert torch.equal(got, want)
    return got, want_s


@pytest.mark.parametrize("b,hkv,t,count,k,pattern", [
    (1, 8, 131072, 64, 1024, "normal"),    # cfg4: 8 rows x 32 chunks, the one-launch top-k
    (1, 8, 131072, 64, 1024, "planted"),
    (2, 8, 131072, 64, 256, "normal"),     # 16 rows x 32 chunks: the three-launch top-k
    (1, 8, 50001, 16, 100, "normal"),      # 8 waves per chunk, a short last chunk
    (1, 4, 40000, 32, 1, "normal"),
    (1, 2, 70000, 128, 513, "normal"),
    (1, 8, 131072, 64, 1024, "equal"),     # every score of a row equal: the lowest indices
    (1, 8, 65536, 64, 1000, "five"),       # five scores per row: ties across every chunk
    (2, 8, 131072, 32, 64, "five"),        # ... on the three-launch grid
])
def test_decode_topk_equals_separate_calls(b, hkv, t, count, k, pattern):
    got, scores = _case(b, hkv, t, count, k, pattern)
    if pattern == "equal":   # every row's k lowest indices
        assert torch.equal(got.cpu(), torch.arange(k, dtype=torch.int32).expand(b, hkv, k))
    if t <= 65536:   # the oracle's own top-k on the same scores
        want = O.topk_lowest_index(scores.reshape(b * hkv, t).cpu().numpy(), k)
        assert np.array_equal(got.reshape(b * hkv, k).cpu().numpy(), want)


@pytest.mark.parametrize("t,k", [(4000, 64), (300000, 128), (20000, 2000)])
def test_decode_topk_other_topk_paths(t, k):
    # rows of one chunk, rows past 64 chunks (the staged top-k) and k > 1024:
    # the scoring launch builds no windows and the top-k runs as it stands
    _case(1, 2, t, 64, k, "normal")


def test_decode_topk_fp16_query():
    _case(1, 8, 131072, 64, 1024, "normal", dtype=torch.float16)


def test_decode_topk_workspace_reuse_and_step():
    # one workspace through several shapes, then the decode step (block 1 uses
    # decode_topk) against the step's own separate calls
    key = _keys(1, 8, 131072, "normal", 3)
    q = torch.randn((1, 32, 128), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    cache = K.Int4KCache.from_prefill(key, 128, 64)
    ws = K.topk_workspace(8, 131072, 1024, DEV)
    for t, k in [(131072, 1024), (90000, 512), (131072, 1024), (8193, 1000)]:
        want = K.block_topk(K.decode_scores(q, cache.chan_idx, cache.slab, cache.slab_scales, t, 1), k)
        got = K.decode_topk(q, cache.chan_idx, cache.slab, cache.slab_scales, t, k, workspace=ws)
        assert torch.equal(got, want)
    v = torch.randn((1, 8, 131072, 128), generator=torch.Generator(device=DEV).manual_seed(4), device=DEV)
    v = v.to(torch.bfloat16)
    step = K.SparseDecodeStep(1, 32, 8, 128, 131072, 1, 1024)
    out = step(q, cache, key, v, 0.088).clone()
    sel = K.block_topk(K.decode_scores(q, cache.chan_idx, cache.slab, cache.slab_scales, 131072, 1), 1024)
    assert torch.equal(step.sel, sel)
    want = K.sparse_attention(q, key, v, sel, 1, 131072, 0.088)
    assert torch.equal(out, want)
