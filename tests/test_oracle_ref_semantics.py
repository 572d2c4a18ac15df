"""Pins the restatement of the reference's fp32 kernels (oracle/ref_semantics.py)
against known answers and fp64 brute force, and checks the reference op
sequence used as the CPU baseline."""

import numpy as np
import torch

from oracle import ref_semantics as R


def test_select_dims_order_and_ties():
    # |q| = [1, 3, 3, 2]: the serial strict-'>' selector of the reference
    # takes dim 1 before dim 2 (equal magnitude, lower index first).
    q = np.array([1.0, -3.0, 3.0, 2.0], np.float32)
    assert R.select_dims_by_abs(q, 2).tolist() == [1, 2]
    assert R.select_dims_by_abs(q, 3).tolist() == [1, 2, 3]
    assert R.select_dims_by_abs(q, 0).tolist() == [1]          # clamped to >= 1
    assert R.select_dims_by_abs(q, 99).tolist() == [1, 2, 3, 0]  # clamped to D


def test_partial_scores_vs_fp64():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, 3, 16)).astype(np.float32)
    k = rng.standard_normal((2, 3, 40, 16)).astype(np.float32)
    got = R.partial_scores(q, k, 5)
    for b in range(2):
        for h in range(3):
            dims = np.argsort(-np.abs(q[b, h]), kind="stable")[:5]
            want = k[b, h][:, dims].astype(np.float64) @ q[b, h, dims].astype(np.float64)
            assert np.allclose(got[b, h], want, rtol=1e-5, atol=1e-5)
    # dim-major restatement agrees with the token-major one for the same dims
    dims = np.stack([np.stack([R.select_dims_by_abs(q[b, h], 5) for h in range(3)]) for b in range(2)])
    kdm = np.ascontiguousarray(k.transpose(0, 1, 3, 2))
    assert np.array_equal(R.partial_scores_dim_major(q, kdm, dims), got)


def test_partial_scores_sequential_order_known_answer():
    # fp32 accumulation in selection order: 2^24 + 1 - 2^24 in that order
    # loses the 1 (2^24 + 1 rounds to 2^24), in another order it would not.
    q = np.array([[[4.0, 2.0, 1.0]]], np.float32)            # order: dims 0, 1, 2
    k = np.array([[[[2.0 ** 22, 0.5, -2.0 ** 24]]]], np.float32)
    assert R.partial_scores(q, k, 3)[0, 0, 0] == np.float32(0.0)


def test_candidate_full_scores_masks():
    q = np.ones((1, 1, 2), np.float32)
    k = np.arange(12, dtype=np.float32).reshape(1, 1, 6, 2)
    cur = np.zeros((1, 1, 6), bool)
    cur[0, 0, 2] = True
    prev = np.zeros((1, 1, 6), bool)
    prev[0, 0, 3] = True
    out = R.candidate_full_scores(q, k, cur, prev, None, 1, 1, 0.5)
    # selected: sink {0}, current {2}, previous {3}, recent {5}
    want = [0.5 * (0 + 1), -np.inf, 0.5 * (4 + 5), 0.5 * (6 + 7), -np.inf, 0.5 * (10 + 11)]
    assert out[0, 0].tolist() == want


def test_final_attention_special_cases():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 2, 4))
    k = rng.standard_normal((1, 2, 6, 4))
    v = rng.standard_normal((1, 2, 6, 4))
    idx = np.array([[[1, 4, 9, -1], [0, 0, 2, 3]]])
    valid = np.array([[[1, 1, 1, 1], [0, 0, 0, 0]]], np.uint8)
    out = R.final_attention(q, k, v, idx, valid, 0.7)
    assert out.shape == (1, 1, 2, 4)
    # head 1: nothing valid -> zeros (QK:388, 404)
    assert np.all(out[0, 0, 1] == 0)
    # head 0: out-of-range 9 and -1 are skipped; only rows 1 and 4 count
    s = k[0, 0, [1, 4]] @ q[0, 0] * 0.7
    w = np.exp(s - s.max())
    w /= w.sum()
    assert np.allclose(out[0, 0, 0], w @ v[0, 0, [1, 4]])


def test_final_indices_from_selected():
    sel = torch.tensor([[[0, 5, 8, 3]]])
    idx, valid = R.final_indices_from_selected(sel, torch.ones_like(sel, dtype=torch.bool), 9, 10,
                                               sink=2, recent=2, keep_self=True)
    # 0 is in the sink range and 8 in the recent range: masked, then appended
    assert idx.tolist() == [[[0, 5, 8, 3, 0, 1, 7, 8, 9]]]
    assert valid.tolist() == [[[False, True, False, True, True, True, True, True, True]]]


def test_cpu_op_sequence_matches_fp64_on_its_own_selection():
    torch.manual_seed(0)
    b, hq, hkv, t, d = 1, 4, 2, 64, 16
    q = torch.randn(b, hq, 1, d)
    k = torch.randn(b, hkv, t, d)
    v = torch.randn(b, hkv, t, d)
    out = R.qabs_candidate_attention_cpu(q, k, v, dim_count=4, candidate_fraction=0.1, scaling=0.25)
    assert out.shape == (b, 1, hq, d)
    # reproduce the selection independently and compare against the fp64 kernel restatement
    kk = k.repeat_interleave(2, dim=1)
    vv = v.repeat_interleave(2, dim=1)
    hist = t - 1
    req = int(np.ceil(0.1 * hist))
    qn = q[:, :, 0].numpy()
    part = R.partial_scores(qn, kk[:, :, :hist].numpy(), 4)
    cand = np.argsort(-part, axis=-1, kind="stable")[..., :req]
    idx = np.concatenate([cand, np.full((b, hq, 1), t - 1)], axis=-1)
    want = R.final_attention(qn, kk.numpy(), vv.numpy(), idx, np.ones_like(idx, np.uint8), 0.25)
    assert np.allclose(out.numpy(), want, rtol=1e-4, atol=1e-4)
