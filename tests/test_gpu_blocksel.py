"""GPU parity of the block selectors (qbb, brep, qboracle) against the
oracle, which the reference's own drivers pin (tests/test_oracle_block.py):
metadata, block scores and final masks bit-exact; attention within 1e-2 /
2e-2.  The reference's bf16 qboracle vectors also run through the GPU step."""

import numpy as np
import pytest
import torch

from kv_cache_amd import _lib
from kv_cache_amd import blocksel as BS
from oracle import qkv_oracle as O
from oracle import ref_semantics as R
from tests.test_oracle_block import load_block_golden

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2


KINDS = {BS.QBB: "qbb", BS.BREP: "brep", BS.QBORACLE: "qboracle"}


def f32(t):
    return t.float().cpu().numpy()


def _kv(b, hkv, t, seed):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn((b, hkv, t, 128), generator=g) * 1.5).to(torch.bfloat16)
    v = torch.randn((b, hkv, t, 128), generator=g).to(torch.bfloat16)
    return k, v, g


@pytest.mark.parametrize("block,t", [(16, 1000), (8, 333), (64, 700), (1, 50)])
def test_qbb_metadata_and_bounds(block, t):
    lib = _lib.load()
    k, _, g = _kv(2, 2, t, block + t)
    q = torch.randn((2, 4, 128), generator=g).to(torch.bfloat16)
    kd, qd = k.to(DEV), q.to(DEV)
    mb = -(-t // block) + 3
    meta = torch.zeros(lib.qkv_block_meta_bytes(BS.QBB, 2, 2, mb, 1), dtype=torch.uint8, device=DEV)
    ks = _lib.strides(*kd.stride())
    # built in two pieces: the second rebuilds the block the first ended inside
    for t0, t1 in ((0, t // 2 + 1), (t // 2 + 1, t)):
        _lib.check(lib.qkv_block_meta_update(BS.QBB, kd.data_ptr(), ks, 2, 2, 128, block, 1, t0, t1,
                                             meta.data_ptr(), mb, 0, _lib.stream_of(kd)))
    rec = meta.view(torch.int16).view(2, 2, mb, 2, 128)[:, :, : -(-t // block)]
    lo, hi = R.block_minmax(f32(k), block)
    assert np.array_equal(f32(rec[:, :, :, 0].view(torch.bfloat16)), lo)
    assert np.array_equal(f32(rec[:, :, :, 1].view(torch.bfloat16)), hi)
    nb = -(-t // block)
    out = torch.empty((8, nb + 5), dtype=torch.float32, device=DEV)
    _lib.check(lib.qkv_block_scores(BS.QBB, qd.data_ptr(), kd.data_ptr(), ks, meta.data_ptr(), mb, 2, 4, 2, t, 128,
                                    block, 1, 8, out.data_ptr(), nb + 5, 0, _lib.stream_of(kd)))
    want = R.qbb_block_bounds(f32(q), np.repeat(lo, 2, axis=1), np.repeat(hi, 2, axis=1), 8)
    assert np.array_equal(out[:, :nb].cpu().numpy().reshape(2, 4, nb), want)


@pytest.mark.parametrize("block,reps,t", [(16, 2, 1000), (8, 1, 333), (64, 5, 700), (16, 16, 40),
                                          # a workgroup per block: norms in registers, then past 16384 tokens
                                          # per block recomputed each round
                                          (128, 3, 1000), (1000, 8, 2500), (20000, 4, 41000)])
def test_brep_metadata_and_scores(block, reps, t):
    lib = _lib.load()
    k, _, g = _kv(1, 2, t, block * reps + t)
    k[0, 0, 3] = k[0, 0, 5]          # equal norms: the lower index first
    q = torch.randn((1, 8, 128), generator=g).to(torch.bfloat16)
    kd, qd = k.to(DEV), q.to(DEV)
    mb = -(-t // block)
    meta = torch.zeros(lib.qkv_block_meta_bytes(BS.BREP, 1, 2, mb, reps), dtype=torch.uint8, device=DEV)
    ks = _lib.strides(*kd.stride())
    for t0, t1 in ((0, 1), (1, t - 7), (t - 7, t)):
        _lib.check(lib.qkv_block_meta_update(BS.BREP, kd.data_ptr(), ks, 1, 2, 128, block, reps, t0, t1,
                                             meta.data_ptr(), mb, 0, _lib.stream_of(kd)))
    got = meta.view(torch.int32).view(1, 2, mb, reps).cpu().numpy()
    idx, valid = R.block_representatives(f32(k), block, reps)
    assert np.array_equal(np.where(valid, idx, -1), got)
    out = torch.empty((8, mb), dtype=torch.float32, device=DEV)
    _lib.check(lib.qkv_block_scores(BS.BREP, qd.data_ptr(), kd.data_ptr(), ks, meta.data_ptr(), mb, 1, 8, 2, t, 128,
                                    block, reps, 16, out.data_ptr(), mb, 0, _lib.stream_of(kd)))
    kx = np.repeat(f32(k), 4, axis=1)
    want = R.brep_block_scores(f32(q), kx, np.repeat(idx, 4, axis=1), np.repeat(valid, 4, axis=1), 16)
    assert np.array_equal(out.cpu().numpy().reshape(1, 8, mb), want)


@pytest.mark.parametrize("mode,hq,hkv,t,steps,sink,recent,keep_self", [
    ("qbb16q8s12cand4", 8, 2, 3000, 3, 3, 5, True),
    ("qbb8q16s25cand6p25", 4, 4, 1500, 2, 0, 0, False),
    ("qbb32q8s6p25cand2", 32, 8, 9000, 2, 4, 8, True),
    ("brep16r2q8s12cand4", 8, 2, 3000, 3, 3, 5, True),
    ("brep8r1q16s25cand6p25", 4, 1, 1200, 2, 0, 4, True),
    ("brep16r4q8s6p25cand2", 32, 8, 9000, 2, 4, 8, True),
    ("qbb16q8s40cand10", 8, 2, 20000, 1, 2, 2, True),          # 8000 scanned tokens, 2000 candidates
    ("brep32r2q8s90cand11", 4, 1, 36000, 1, 0, 0, True),       # 32400 scanned, 3960 candidates
    ("qboracle16q8s12cand4", 8, 2, 3000, 3, 3, 5, True),
    ("qboracle8q16s25cand6p25", 4, 4, 1500, 2, 0, 0, False),
    ("qboracle64q8s6p25cand2", 32, 8, 9000, 2, 4, 8, True),
    ("qboracle1q8s5cand3", 8, 2, 5000, 2, 2, 2, True),          # one-token blocks: 250 scanned tokens
])
def test_step_matches_oracle(mode, hq, hkv, t, steps, sink, recent, keep_self):
    kind, block, reps, dims, scan, cand = BS.parse_block_mode(mode)
    k, v, g = _kv(1, hkv, t + steps, hq * t)
    qs = torch.randn((steps, 1, hq, 128), generator=g).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = BS.BlockSelectDecodeStep(mode, 1, hq, hkv, 128, t + steps + 40, top_fraction=0.02, protect_sink=sink,
                                    protect_recent=recent, keep_self=keep_self)
    step.prefill(kd[:, :, : t - 3])
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, keep = R.block_select_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), KINDS[kind], block, dims,
                                         scan, cand, 0.02, 128 ** -0.5, sink, recent, keep_self, reps)
        assert np.array_equal(step.final_mask().cpu().numpy(), keep), (mode, s)
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("block,t,hq,hkv,dims", [(16, 1000, 8, 2, 8), (7, 333, 4, 4, 16), (64, 2100, 4, 1, 12),
                                                 (1, 300, 8, 2, 8), (300, 4000, 4, 2, 128), (2048, 5000, 2, 1, 8),
                                                 (3000, 10000, 2, 1, 8), (5000, 12001, 4, 2, 16)])
def test_qboracle_block_scores_match_oracle(block, t, hq, hkv, dims):
    # block maxima of the partial scores (EV:5030-5044), bit for bit
    from kv_cache_amd.reuse import dim_major_append

    lib = _lib.load()
    k, _, g = _kv(1, hkv, t, block + t)
    k[0, 0, 5] = k[0, 0, 3]
    q = torch.randn((1, hq, 128), generator=g).to(torch.bfloat16)
    kd, qd = k.to(DEV), q.to(DEV)
    kdm = torch.empty((1, hkv, 128, t + 64), dtype=torch.bfloat16, device=DEV)
    dim_major_append(kd, kdm, 0, t)
    nb = -(-t // block)
    out = torch.full((hq, nb + 3), 7.0, dtype=torch.float32, device=DEV)
    _lib.check(lib.qkv_block_max_partial_scores(qd.data_ptr(), kdm.data_ptr(), _lib.strides(*kdm.stride()), 1, hq, hkv,
                                                t, 128, block, dims, out.data_ptr(), nb + 3, 0, _lib.stream_of(kd)))
    want = O.block_max(R.partial_scores(f32(q), np.repeat(f32(k), hq // hkv, axis=1), dims), block)
    got = out.cpu().numpy()
    assert np.array_equal(got[:, :nb].reshape(1, hq, nb), want)
    assert (got[:, nb:] == 7.0).all()


@pytest.mark.parametrize("name", ["qboracle16q8s12cand4_bf16"])
def test_step_reproduces_reference_vectors(name):
    # the reference's qboracle driver on bf16 inputs, replayed through the GPU
    # step: every step's final mask bit-exact, outputs within tolerance
    g = load_block_golden(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    kd = torch.from_numpy(g["k"]).to(torch.bfloat16).to(DEV)
    vd = torch.from_numpy(g["v"]).to(torch.bfloat16).to(DEV)
    step = BS.BlockSelectDecodeStep(g["mode"], 1, hq, hkv, 128, kd.size(2) + 8, top_fraction=g["top_fraction"],
                                    protect_sink=g["sink"], protect_recent=g["recent"], keep_self=g["keep_self"])
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(torch.bfloat16).to(DEV)
        out = step(q, kd[:, :, :n], vd[:, :, :n], g["scaling"])
        assert np.array_equal(step.final_mask().cpu().numpy(), g["final"][s][..., :n]), (name, s)
        np.testing.assert_allclose(f32(out), g["out"][s], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("mode,hq,hkv,t,steps", [
    ("qboracle16q8s2cand10", 4, 2, 3000, 2),      # 10% candidates from 2% scanned: unscanned ones at finfo.min
    ("qboracle64q8s1cand3", 8, 2, 20000, 1),      # the same at 20000 tokens, 64-token blocks
    ("qbb16q8s50cand4", 4, 2, 90000, 1),          # 45000 scanned tokens per row
    ("qbb16q8s20cand10", 4, 1, 60000, 1),         # 6000 candidates per row
    ("brep20000r2q8s100cand2", 4, 2, 45000, 1),   # every block scanned (45000 tokens), 20000-token blocks
    ("brep256r2q8s30cand6", 8, 2, 20000, 2),      # 6000 scanned tokens, 1200 candidates: one workgroup
])
def test_step_past_the_one_workgroup_rerank_matches_oracle(mode, hq, hkv, t, steps):
    # rows the one-workgroup rerank cannot hold run the general rerank (dense
    # candidate scores, two staged top-k selections); masks still bit-exact
    kind, block, reps, dims, scan, cand = BS.parse_block_mode(mode)
    k, v, g = _kv(1, hkv, t + steps, hq * t + 5)
    qs = torch.randn((steps, 1, hq, 128), generator=g).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = BS.BlockSelectDecodeStep(mode, 1, hq, hkv, 128, t + steps + 8, top_fraction=0.02, protect_sink=3,
                                    protect_recent=5, keep_self=True)
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, keep = R.block_select_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), KINDS[kind], block, dims,
                                         scan, cand, 0.02, 128 ** -0.5, 3, 5, True, reps)
        assert np.array_equal(step.final_mask().cpu().numpy(), keep), (mode, s)
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)


def test_rerank_general_path_equals_one_workgroup_path():
    # Rows that fit both reranks: the qboracle flag with more candidates than
    # the fewest scanned history tokens a row could have (its last, partial
    # block scanned) takes the general path, but these rows never scan that
    # block, so their candidates are all scanned tokens and both paths must
    # write the same mask and token list; the partial scores carry ties.
    lib = _lib.load()
    hq, hkv, t, block, n_scan = 4, 2, 5000, 16, 40
    history = t - 1
    nb = -(-history // block)
    g = torch.Generator().manual_seed(5)
    k = torch.randn((1, hkv, t, 128), generator=g).to(torch.bfloat16).to(DEV)
    q = torch.randn((1, hq, 128), generator=g).to(torch.bfloat16).to(DEV)
    blocks = torch.stack([torch.randperm(nb - 1, generator=g)[:n_scan].sort().values for _ in range(hq)])
    blocks = blocks.to(torch.int32).to(DEV).contiguous()
    partial = (torch.randint(0, 50, (hq, n_scan * block), generator=g).float() / 4).to(DEV)
    n_cand, n_keep = n_scan * block - 2, 100
    n_out = int(lib.qkv_final_list_count(history, n_keep, 3, 5, 1))
    assert lib.qkv_block_rerank_workspace_bytes(hq, history, n_scan, block, n_cand, n_keep, 0) == 0
    need = int(lib.qkv_block_rerank_workspace_bytes(hq, history, n_scan, block, n_cand, n_keep, 1))
    assert need > 0
    outs = []
    for unscanned in (0, 1):
        keep = torch.zeros((hq, t + 8), dtype=torch.uint8, device=DEV)
        ids = torch.full((hq * n_out,), -7, dtype=torch.int32, device=DEV)
        ws = torch.empty((need + 3) // 4, dtype=torch.float32, device=DEV) if unscanned else None
        _lib.check(lib.qkv_block_rerank(
            q.data_ptr(), k.data_ptr(), _lib.strides(*k.stride()), 1, hq, hkv, t, 128, partial.data_ptr(), None,
            n_scan * block, blocks.data_ptr(), n_scan, block, n_cand, n_keep, 3, 5, 1, 0.088, keep.data_ptr(), t + 8,
            ids.data_ptr(), n_out, unscanned, _lib.ptr(ws), need if unscanned else 0, 0, _lib.stream_of(q)))
        outs.append((keep, ids))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert int(outs[0][0][:, :history].sum()) > hq * n_keep // 2


def test_new_sequence_resets():
    k, v, g = _kv(1, 2, 800, 3)
    q = torch.randn((1, 4, 128), generator=g).to(torch.bfloat16).to(DEV)
    kd, vd = k.to(DEV), v.to(DEV)
    step = BS.BlockSelectDecodeStep("qbb16q8s12cand4", 1, 4, 2, 128, 1024)
    step(q, kd[:, :, :700], vd[:, :, :700], 0.1)
    a = step(q, kd[:, :, :400], vd[:, :, :400], 0.1).clone()
    fresh = BS.BlockSelectDecodeStep("qbb16q8s12cand4", 1, 4, 2, 128, 1024)
    assert torch.equal(a, fresh(q, kd[:, :, :400], vd[:, :, :400], 0.1))
    assert torch.equal(step.final_mask(), fresh.final_mask())


def test_longer_new_sequence_resets():
    k, v, g = _kv(1, 2, 900, 4)
    k2, v2, _ = _kv(1, 2, 900, 8)
    q = torch.randn((1, 4, 128), generator=g).to(torch.bfloat16).to(DEV)
    kd, vd, kd2, vd2 = k.to(DEV), v.to(DEV), k2.to(DEV), v2.to(DEV)
    for mode in ("qbb16q8s12cand4", "brep16r2q8s12cand4", "qboracle16q8s12cand4"):
        step = BS.BlockSelectDecodeStep(mode, 1, 4, 2, 128, 1024)
        step(q, kd[:, :, :500], vd[:, :, :500], 0.1)
        a = step(q, kd2[:, :, :800], vd2[:, :, :800], 0.1).clone()     # another sequence, longer
        fresh = BS.BlockSelectDecodeStep(mode, 1, 4, 2, 128, 1024)
        assert torch.equal(a, fresh(q, kd2[:, :, :800], vd2[:, :, :800], 0.1)), mode
        assert torch.equal(step.final_mask(), fresh.final_mask()), mode


def test_bad_rerank_arguments_are_errors():
    lib = _lib.load()
    assert lib.qkv_block_rerank_workspace_bytes(4, 1000, 10, 16, 10, 11, 0) == -1     # n_keep > n_cand
    assert lib.qkv_block_rerank_workspace_bytes(4, 100000, 3000, 16, 100, 10, 0) > 0  # 48000 scanned tokens
    assert lib.qkv_block_rerank_workspace_bytes(4, 100000, 100, 16, 5000, 10, 0) > 0  # 5000 candidates
    assert lib.qkv_block_rerank_workspace_bytes(4, 10000, 10, 16, 200, 10, 1) > 0     # qboracle, 200 > 160 scanned
    assert lib.qkv_block_rerank_workspace_bytes(4, 10000, 10, 16, 100, 10, 1) == 0
    with pytest.raises(RuntimeError, match="at most 64 representatives"):
        BS.BlockSelectDecodeStep("brep128r65q8s6cand2", 1, 4, 2, 128, 4000)


@pytest.mark.parametrize("mode,t", [("qbb64q8s3cand3", 4000), ("brep16r4q8s12cand4", 3001)])
def test_rerank_with_and_without_scan_full_scores(mode, t):
    # The step hands the rerank the full-D scores its scan launch computed;
    # the rerank computing them itself (full = NULL) keeps the same masks and
    # token lists, and both match the step's.
    hq, hkv = 8, 2
    k, v, g = _kv(1, hkv, t, 41)
    q = torch.randn((1, hq, 128), generator=g).to(torch.bfloat16).to(DEV)
    step = BS.BlockSelectDecodeStep(mode, 1, hq, hkv, 128, t + 8, top_fraction=0.02, protect_sink=3,
                                    protect_recent=5, keep_self=True)
    kd, vd = k.to(DEV), v.to(DEV)
    step(q, kd, vd, 0.088)
    history = t - 1
    nb, n_scan, n_cand, n_keep = BS.step_counts(history, step.block, step.scan, step.cand, step.top_fraction)
    lib = _lib.load()
    rows, n_tok = hq, n_scan * step.block
    n_out = int(lib.qkv_final_list_count(history, n_keep, 3, 5, 1))
    want_mask, want_ids = step.keep[:, :t].clone(), step.attn_ids[: rows * n_out].clone()
    for full in (step.full[: rows * n_tok], None):
        keep = torch.zeros_like(step.keep)
        ids = torch.full((rows * n_out,), -7, dtype=torch.int32, device=DEV)
        _lib.check(lib.qkv_block_rerank(
            q.data_ptr(), kd.data_ptr(), _lib.strides(*kd.stride()), 1, hq, hkv, t, 128,
            step.partial[: rows * n_tok].data_ptr(), _lib.ptr(full), n_tok, step.blocks[: rows * n_scan].data_ptr(),
            n_scan, step.block, n_cand, n_keep, 3, 5, 1, 0.088, keep.data_ptr(), step.capacity, ids.data_ptr(), n_out,
            0, None, 0, 0, _lib.stream_of(q)))
        assert torch.equal(keep[:, :t], want_mask), full is None
        assert torch.equal(ids, want_ids), full is None
