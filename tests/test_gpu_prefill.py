"""GPU parity of chunked-prefill block selection (int8 MFMA) against the
CPU oracle: bit-exact int8 queries, block maxima and top-k block ids."""

import numpy as np
import pytest
import torch

from kv_cache_amd import int4 as K
from kv_cache_amd import prefill as P
from oracle import qkv_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(b, hq, hkv, nq, t, q_pos0, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, hq, nq, 128), generator=g)
    q[..., 7] *= 8.0
    k = torch.randn((b, hkv, t, 128), generator=g)
    k[..., [3, 40, 77, 120]] *= 8.0
    return q.to(torch.bfloat16), k.to(torch.bfloat16)


def test_quantize_query_matches_oracle():
    q, _ = _case(2, 3, 1, 77, 64, 0, seed=1)
    q8, qs = P.quantize_query(q.to(DEV))
    want, want_s = O.quantize_query_rows(q.float().numpy())
    assert np.array_equal(q8.cpu().numpy(), O.permute_prefill_query(want))
    assert np.array_equal(qs.cpu().numpy(), want_s)


@pytest.mark.parametrize("width,offset", [(132, 0), (136, 2), (256, 64)])
def test_quantize_query_strided_rows_match_oracle(width, offset):
    # rows that are not 16-byte aligned (stride 132, or 4 bytes in) take the
    # kernel that loads two channels a lane; stride 256 takes the 16-byte loads
    g = torch.Generator().manual_seed(width + offset)
    big = torch.randn((301, width), generator=g).to(torch.bfloat16)
    big[7] = 0.0                                     # a zero row: scale 0, codes 0
    q = big[:, offset:offset + 128]
    qd = big.to(DEV)[:, offset:offset + 128]          # the strided view itself, on the device
    assert qd.stride(0) == width
    q8, qs = P.quantize_query(qd)
    want, want_s = O.quantize_query_rows(q.float().numpy())
    assert np.array_equal(q8.cpu().numpy(), O.permute_prefill_query(want))
    assert np.array_equal(qs.cpu().numpy(), want_s)


@pytest.mark.parametrize("b,hq,hkv,nq,t,q_pos0", [
    (1, 4, 2, 100, 1000, 900),     # partial query tile, partial last block, causal cut
    (1, 8, 2, 64, 2500, 0),        # most blocks invisible to the first queries
    (2, 4, 4, 130, 4096, 3966),    # G = 1, last chunk of the context
    (1, 16, 4, 200, 3000, 2800),   # G = 4
    (1, 16, 2, 150, 3000, 2850),   # G = 8: two workgroups of 4 heads per query tile
    (1, 6, 2, 300, 2000, 1700),    # G = 3: one head per workgroup, three query tiles
])
def test_block_scores_match_oracle(b, hq, hkv, nq, t, q_pos0):
    q, k = _case(b, hq, hkv, nq, t, q_pos0, seed=nq + t)
    packed, scales = K.int4_pack_k(k.to(DEV), 128)
    q8, _ = P.quantize_query(q.to(DEV))
    bmax = P.block_scores(q8, packed, scales, t, q_pos0)
    want_q8, _ = O.quantize_query_rows(q.float().numpy())
    kp, ks = O.int4_pack_k(k.float().numpy(), 128)
    want = O.prefill_block_scores(want_q8, kp, ks[..., 0], 64, q_pos0)
    got = bmax.cpu().numpy()
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k", [1, 16, 47])
def test_block_topk_matches_oracle(k):
    q, kk = _case(1, 8, 2, 96, 3000, 200, seed=k)
    packed, scales = K.int4_pack_k(kk.to(DEV), 128)
    sel, bmax = P.select_blocks(q.to(DEV), packed, scales, 3000, 200, k)
    want = O.prefill_block_topk(bmax.cpu().numpy(), k)
    assert np.array_equal(sel.cpu().numpy(), want)
    # the first queries see only 4 blocks: the rest of their row is -1
    if k > 4:
        assert (sel[0, 0, 0, 4:] == -1).all()


def test_block_topk_ties_and_padding():
    vals = torch.full((3, 1000), -float("inf"))
    vals[0, :10] = 1.0                      # 10 finite ties
    vals[1] = torch.arange(1000).float() % 7
    got = P.block_topk(vals.to(DEV), 16).cpu().numpy()
    assert np.array_equal(got, O.prefill_block_topk(vals.numpy(), 16))
    assert got[0].tolist() == list(range(10)) + [-1] * 6
    assert (got[2] == -1).all()


def test_config5_slice():
    # cfg5 shape (32 q / 8 kv heads, head_dim 128, block 64, top-64) on a
    # slice the oracle scores in seconds: 128 queries at the end of 8192 keys.
    q, k = _case(1, 32, 8, 128, 8192, 8192 - 128, seed=5)
    packed, scales = K.int4_pack_k(k.to(DEV), 128)
    sel, bmax = P.select_blocks(q.to(DEV), packed, scales, 8192, 8192 - 128, 64)
    want_q8, _ = O.quantize_query_rows(q.float().numpy())
    kp, ks = O.int4_pack_k(k.float().numpy(), 128)
    want = O.prefill_block_scores(want_q8, kp, ks[..., 0], 64, 8192 - 128)
    assert np.array_equal(bmax.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(sel.cpu().numpy(), O.prefill_block_topk(want, 64))
