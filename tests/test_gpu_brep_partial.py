"""brep_partial_scores, the kernel the reference imports but never shipped
(wrapper EV:3847-3877, call EV:5419-5431), against the oracle: partial
scores bit-exact on the scanned blocks' tokens and -inf elsewhere, where the
scanned blocks are the best by their representatives' scores
(ref_semantics.brep_block_scores, pinned by the reference's brep drivers).
Then, through the caller's next steps (ref_semantics.brep_caller_final_mask:
candidate top-k, full-D rerank, protection; EV:5426-5505), every step of the
reference's brep golden scenarios reproduces the reference's final mask bit
for bit."""

import math

import numpy as np
import pytest
import torch

from kv_cache_amd import qabs_cuda_kernels as QK
from oracle import qkv_oracle as O
from oracle import ref_semantics as R
from tests.test_oracle_block import load_block_golden

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _want(q, k, ridx, rvalid, block, dims, scan):
    return R.brep_partial_scores(q, k, ridx, rvalid, block, dims, scan)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("block,reps,t,dims,scan", [(16, 2, 1000, 8, 0.25), (8, 1, 333, 16, 0.12),
                                                      (64, 5, 700, 12, 0.5), (4, 4, 37, 128, 1.0),
                                                      (16, 3, 4100, 8, 0.01)])
def test_brep_partial_scores_match_oracle(dtype, block, reps, t, dims, scan):
    g = torch.Generator().manual_seed(block * 1000 + t)
    k = (torch.randn((2, 4, t, 128), generator=g) * 1.5).to(dtype)
    k[0, 1, 5] = k[0, 1, 3]                       # equal norms: the lower position is the representative
    k[1, 2, 2 * block: 3 * block] = k[1, 2, :block]   # two blocks with equal scores: the lower one ranks first
    q = torch.randn((2, 4, 128), generator=g).to(dtype).float()   # the caller's fp32 query
    kf = k.float().numpy()
    ridx, rvalid = R.block_representatives(kf, block, reps)
    got = QK.brep_partial_scores(q.to(DEV), k.to(DEV), torch.from_numpy(ridx).to(DEV),
                                 torch.from_numpy(rvalid).to(DEV), block, dims, scan)
    want = _want(q.numpy(), kf, ridx, rvalid, block, dims, scan)
    assert np.array_equal(got.cpu().numpy(), want)


def test_brep_partial_scores_invalid_representatives():
    # blocks whose representatives are all invalid score finfo.min and come last
    g = torch.Generator().manual_seed(5)
    k = torch.randn((1, 2, 160, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((1, 2, 128), generator=g).to(torch.bfloat16).float()
    kf = k.float().numpy()
    ridx, rvalid = R.block_representatives(kf, 16, 2)
    rvalid[0, 0, 1:7] = False
    got = QK.brep_partial_scores(q.to(DEV), k.to(DEV), torch.from_numpy(ridx).to(DEV),
                                 torch.from_numpy(rvalid).to(DEV), 16, 8, 0.5)
    want = _want(q.numpy(), kf, ridx, rvalid, 16, 8, 0.5)
    assert np.array_equal(got.cpu().numpy(), want)
    # 5 of 10 blocks scanned: the 4 with representatives (0, 7, 8, 9), then
    # the lowest of the tied finfo.min blocks (1); blocks 2-6 stay -inf
    assert np.isfinite(want[0, 0, 16:32]).all() and np.isinf(want[0, 0, 32:112]).all()


@pytest.mark.parametrize("name", ["brep16r2q8s12cand4_fp32", "brep8r1q16s25cand6p25_fp32"])
def test_brep_partial_scores_reproduce_reference_steps(name):
    gd = load_block_golden(name)
    hq, hkv = gd["q"].shape[2], gd["k"].shape[1]
    gqa = hq // hkv
    for s in range(gd["steps"]):
        n = gd["t0"] + s + 1
        history = n - 1
        kh = np.repeat(gd["k"][:, :, :history], gqa, axis=1)          # the reference's GQA-expanded history
        q = gd["q"][s]
        dims = min(max(1, gd["dims"]), 128)
        ridx, rvalid = R.block_representatives(kh, gd["block"], gd["reps"])
        got = QK.brep_partial_scores(torch.from_numpy(q).to(DEV), torch.from_numpy(kh).to(DEV),
                                     torch.from_numpy(ridx).to(DEV), torch.from_numpy(rvalid).to(DEV), gd["block"],
                                     dims, gd["scan"]).cpu().numpy()
        assert np.array_equal(got, _want(q, kh, ridx, rvalid, gd["block"], dims, gd["scan"])), (name, s)
        for bi in range(q.shape[0]):
            for hi in range(hq):
                final = R.brep_caller_final_mask(got[bi, hi], q[bi, hi], kh[bi, hi], n, gd["cand"],
                                                 gd["top_fraction"], gd["scaling"], gd["sink"], gd["recent"],
                                                 gd["keep_self"])
                assert np.array_equal(final, gd["final"][s][bi, hi, :n]), (name, s, bi, hi)
