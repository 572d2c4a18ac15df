"""Pins the candidate-reuse restatement (oracle/ref_semantics.py: reuse_select,
reuse_decode_step) against golden vectors written by the reference itself
(tests/golden/make_reuse_vectors.py: consecutive decode steps of the
reference's reuse driver, run on the CPU), plus known answers and invariants
of the selection."""

import re
from pathlib import Path

import numpy as np
import pytest

from oracle import ref_semantics as R

GOLDEN = Path(__file__).resolve().parent / "golden"
SCENARIOS = ["s8c5_fp32", "s16c10_final_fp32", "s8c3_2set_fp32", "s8c5_bf16",
             "s8c5_blk16_fp32", "s16c10_finalblk8_bf16", "s8c3_2setblk32_fp32",
             "s8c5_sample64_fp32", "s8c5_samplecover_fp32", "s8c10_prevthr_fp32"]


def load_golden(name):
    """Inputs and per-step outputs of one golden scenario."""
    z = np.load(GOLDEN / f"reuse_{name}.npz")
    t_max = int(z["t_max"])
    bf = lambda a: (a.astype(np.int32) << 16).view(np.float32)   # bf16 bits -> fp32
    m = re.fullmatch(r"qabs(\d+)cand(\d+)reuse(2set|final)?(?:blk(\d+))?", str(z["mode"]))
    return {
        "mode": str(z["mode"]), "dtype": str(z["dtype"]), "dims": int(m.group(1)), "cand": int(m.group(2)) / 100,
        # EV:955-960 test the suffix: a blk mode keeps both previous masks
        "use_prev_candidate": not str(z["mode"]).endswith("reusefinal"),
        "use_prev_final": not str(z["mode"]).endswith("reuse2set"),
        "block": int(m.group(4)) if m.group(4) else None,
        "q": z["q"][:, :, :, 0, :], "k": bf(z["k_bf16"]), "v": bf(z["v_bf16"]), "t0": int(z["t0"]),
        "steps": int(z["steps"]), "top_fraction": float(z["top_fraction"]), "sink": int(z["sink"]),
        "recent": int(z["recent"]), "keep_self": bool(z["keep_self"]), "scaling": float(z["scaling"]),
        "out": z["out"][:, :, 0],   # [steps, B, Hq, D]
        "candidate": np.unpackbits(z["candidate"], axis=-1)[..., :t_max].astype(bool),
        "final": np.unpackbits(z["final"], axis=-1)[..., :t_max].astype(bool),
        "selection": str(z["selection"]) if "selection" in z else "topk",
        "sample_size": int(z["sample_size"]) if "sample_size" in z else 256,
        "thresholds": z["thresholds"] if "thresholds" in z else None,   # [steps, B, Hq]
    }


@pytest.mark.parametrize("name", SCENARIOS)
def test_decode_steps_match_reference_vectors(name):
    g = load_golden(name)
    pc = pf = None
    # fp32: only the attention's summation order differs; bf16: the reference
    # rounds the softmax weights to bf16 (EV:4372-4373)
    tol = dict(rtol=1e-5, atol=1e-5) if g["dtype"] == "float32" else dict(rtol=1e-2, atol=2e-2)
    thr = None
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        got_thr = []
        out, cur, hf = R.reuse_decode_step(
            g["q"][s], g["k"][:, :, :n], g["v"][:, :, :n], g["dims"], g["cand"], g["top_fraction"], g["sink"],
            g["recent"], g["keep_self"], g["scaling"], pc if g["use_prev_candidate"] else None,
            pf if g["use_prev_final"] else None, g["block"], selection=g["selection"],
            sample_size=g["sample_size"], previous_thresholds=thr, thresholds_out=got_thr)
        thr = got_thr[0]
        if g["thresholds"] is not None:
            assert np.array_equal(thr[..., 0], g["thresholds"][s]), (name, s, "thresholds")
        assert np.array_equal(cur, g["candidate"][s][..., : n - 1]), (name, s)
        assert np.array_equal(hf, g["final"][s][..., : n - 1]), (name, s)
        np.testing.assert_allclose(out[:, 0], g["out"][s], **tol)
        pc, pf = cur, hf


def test_expand_to_blocks_known_answers():
    m = np.zeros((1, 1, 10), bool)
    m[0, 0, [1, 8]] = True
    # blocks of 4: [0,4) and [8,10) (the last one cut at the history)
    assert np.flatnonzero(R.expand_to_blocks(m, 4)[0, 0]).tolist() == [0, 1, 2, 3, 8, 9]
    assert np.flatnonzero(R.expand_to_blocks(m, 3)[0, 0]).tolist() == [0, 1, 2, 6, 7, 8]
    assert np.flatnonzero(R.expand_to_blocks(m, 16)[0, 0]).tolist() == list(range(10))
    for b in (None, 0, 1):
        assert np.array_equal(R.expand_to_blocks(m, b), m)
    one = np.ones((2, 1), bool)
    assert np.array_equal(R.expand_to_blocks(one, 8), one)
    assert not R.expand_to_blocks(np.zeros((3, 17), bool), 5).any()


def test_expand_to_blocks_is_idempotent_and_brute_force():
    rng = np.random.default_rng(3)
    m = rng.random((6, 97)) < 0.03
    for b in (2, 5, 16, 33, 97, 200):
        e = R.expand_to_blocks(m, b)
        assert np.array_equal(R.expand_to_blocks(e, b), e)
        for r in range(m.shape[0]):
            for t in range(m.shape[1]):
                assert e[r, t] == m[r, (t // b) * b:(t // b + 1) * b].any()


def test_indices_from_keep_mask_descending_and_padded():
    m = np.array([[False, True, True, False, True], [False, False, False, True, False]])
    idx, valid = R.indices_from_keep_mask(m)
    assert idx.tolist() == [[4, 2, 1], [3, 0, 0]]
    assert valid.tolist() == [[True, True, True], [True, False, False]]
    idx, valid = R.indices_from_keep_mask(np.zeros((2, 4), bool))
    assert idx.shape == (2, 0) and valid.shape == (2, 0)


def test_reuse_select_block_expansion():
    # scores 9 5 7 1 0 8 3 2 1 1; keep = 2 -> {0, 5}; blocks of 4 -> {0..3, 4..7};
    # sink 1 is in block 0, recent 1 (position 9) is block [8, 10)
    q, k = _row([9, 5, 7, 1, 0, 8, 3, 2, 1, 1])
    allm = _mask(10, range(10))
    fi, fv, hf = R.reuse_select(q, k, allm, None, None, sink=1, recent=1, top_fraction=0.2, keep_self=True,
                                scaling=1.0, block=4)
    assert np.flatnonzero(hf[0, 0]).tolist() == list(range(10))
    got = sorted(fi[0, 0][fv[0, 0]].tolist())
    assert got == list(range(11))           # all history + the current token 10
    assert len(got) == len(set(got))        # protected entries appear once
    fi, fv, hf = R.reuse_select(q, k, allm, None, None, sink=0, recent=0, top_fraction=0.2, keep_self=False,
                                scaling=1.0, block=4)
    assert np.flatnonzero(hf[0, 0]).tolist() == list(range(8))
    assert fi[0, 0][fv[0, 0]].tolist() == [7, 6, 5, 4, 3, 2, 1, 0]


def test_candidate_mask_selections_known_answers():
    p = np.array([[[5.0, 1.0, 4.0, 2.0, 3.0, 0.0, 6.0, 7.0]]], np.float32)
    m, thr, used = R.candidate_mask(p, 3, 0.3, "topk")
    assert used == "topk" and thr.tolist() == [[[5.0]]] and np.flatnonzero(m).tolist() == [0, 6, 7]
    m, thr, used = R.candidate_mask(p, 3, 0.3, "previous_threshold", np.array([[3.5]], np.float32))
    assert used == "previous_threshold" and np.flatnonzero(m).tolist() == [0, 2, 6, 7]
    m, thr, used = R.candidate_mask(p, 3, 0.3, "previous_threshold", None)      # no previous step: topk
    assert used == "topk" and thr.tolist() == [[[5.0]]]
    # a sample of 4 of the 8 columns: linspace(0, 7, 4) = 0, 2.33, 4.67, 7 -> 0, 2, 5, 7; values 5, 4, 0, 7;
    # ceil(0.3 * 4) = 2 -> threshold 5
    assert R.sample_columns(8, 4).tolist() == [0, 2, 5, 7]
    m, thr, used = R.candidate_mask(p, 3, 0.3, "sample_quantile", sample_size=4)
    assert used == "sample_quantile" and thr.tolist() == [[[5.0]]] and np.flatnonzero(m).tolist() == [0, 6, 7]
    assert R.sample_columns(8, 8) is None and R.sample_columns(8, 100) is None
    # a sample of one column: the middle is not sampled, column 0 is
    assert R.sample_columns(8, 1).tolist() == [0]


def test_sample_columns_are_the_rounded_linspace():
    # |position - i * (n - 1) / (s - 1)| <= 1/2 (+ float32 slack), ascending, unique, ends kept
    for n, size in [(1000, 256), (32768, 256), (257, 256), (5000, 7), (99, 2)]:
        cols = R.sample_columns(n, size)
        exact = np.arange(size) * (n - 1) / (size - 1)
        assert cols[0] == 0 and cols[-1] == n - 1 and np.all(np.diff(cols) > 0)
        if len(cols) == size:
            assert np.all(np.abs(cols - exact) <= 0.5 + 1e-3)


def test_threshold_mask_keeps_ties():
    p = np.array([[3.0, 1.0, 3.0, 2.0]], np.float32)
    assert R.threshold_mask(p, 1).tolist() == [[True, False, True, False]]
    assert R.threshold_mask(p, 3).tolist() == [[True, False, True, True]]
    assert R.budget_count(240, 0.05) == 12 and R.budget_count(10, 0.0) == 1 and R.budget_count(3, 2.0) == 3


def _row(scores):
    """q = e0, K[t] = (s_t, 0, ...) so that the full score of t is s_t."""
    t = len(scores)
    k = np.zeros((1, 1, t + 1, 4), np.float32)
    k[0, 0, :t, 0] = scores
    q = np.zeros((1, 1, 4), np.float32)
    q[0, 0, 0] = 1.0
    return q, k


def _mask(t, ids):
    m = np.zeros((1, 1, t), bool)
    m[0, 0, list(ids)] = True
    return m


def test_reuse_select_known_answer():
    q, k = _row([9, 5, 7, 1, 0, 8, 3, 2])
    fi, fv, hf = R.reuse_select(q, k, _mask(8, [1, 3, 5]), _mask(8, [2]), _mask(8, [6]), sink=1, recent=2,
                                top_fraction=0.3, keep_self=True, scaling=1.0)
    # union {1,2,3,5,6} scores {5,7,1,8,3}: top 3 = {5, 2, 1}, ascending
    assert fi.tolist() == [[[1, 2, 5, 0, 6, 7, 8]]]
    assert fv.tolist() == [[[True] * 7]]
    assert np.flatnonzero(hf[0, 0]).tolist() == [0, 1, 2, 5, 6, 7]


def test_reuse_select_protected_and_short_union():
    q, k = _row([9, 5, 7, 1, 0, 8, 3, 2])
    # union {1, 6}: 3 slots, the third is the lowest -inf index (0), invalid;
    # 6 lies in the recent range, so it is masked and the range appended
    fi, fv, hf = R.reuse_select(q, k, _mask(8, [1]), None, _mask(8, [6]), sink=0, recent=2, top_fraction=0.3,
                                keep_self=False, scaling=1.0)
    assert fi.tolist() == [[[0, 1, 6, 6, 7]]]
    assert fv.tolist() == [[[False, True, False, True, True]]]
    assert np.flatnonzero(hf[0, 0]).tolist() == [1, 6, 7]


def test_reuse_select_ties_take_lower_index():
    q, k = _row([4, 4, 4, 4, 4, 4])
    fi, fv, _ = R.reuse_select(q, k, _mask(6, [5, 3, 1, 2]), None, None, 0, 0, 0.5, False, 1.0)
    assert fi.tolist() == [[[1, 2, 3]]] and fv.all()


def test_reuse_select_invariants():
    rng = np.random.default_rng(3)
    b, h, t, d = 2, 3, 97, 16
    q = rng.standard_normal((b, h, d)).astype(np.float32)
    k = rng.standard_normal((b, h, t + 1, d)).astype(np.float32)
    masks = [rng.random((b, h, t)) < p for p in (0.1, 0.05, 0.03)]
    fi, fv, hf = R.reuse_select(q, k, *masks, 3, 4, 0.1, True, 0.25)
    union = masks[0] | masks[1] | masks[2]
    keep = R.budget_count(t, 0.1)
    full = np.einsum("bhd,bhtd->bht", q.astype(np.float64), k[:, :, :t].astype(np.float64)) * 0.25
    for bi in range(b):
        for hi in range(h):
            sel = fi[bi, hi, :keep]
            ok = np.isfinite(np.where(union[bi, hi], full[bi, hi], -np.inf))[sel]
            chosen = set(sel[ok].tolist())
            assert len(chosen) == min(keep, int(union[bi, hi].sum()))
            rest = [x for x in np.flatnonzero(union[bi, hi]) if x not in chosen]
            if rest and chosen:
                assert min(full[bi, hi, list(chosen)]) >= max(full[bi, hi, rest]) - 1e-5
            assert hf[bi, hi, :3].all() and hf[bi, hi, t - 4:].all()
            assert set(np.flatnonzero(hf[bi, hi]).tolist()) == chosen | {0, 1, 2} | set(range(t - 4, t))
            assert fi[bi, hi, -1] == t and fv[bi, hi, -1]


@pytest.mark.parametrize("name", SCENARIOS)
def test_cpu_baseline_op_sequence_matches_reference_vectors(name):
    # The torch op sequence bench.py times as the reuse CPU baseline leaves
    # the reference's state and output at every step.
    import torch

    g = load_golden(name)
    if g["selection"] != "topk":
        pytest.skip("the CPU baseline times the default candidate selection")
    dt = torch.float32 if g["dtype"] == "float32" else torch.bfloat16
    k, v = torch.from_numpy(g["k"]).to(dt), torch.from_numpy(g["v"]).to(dt)
    pc = pf = None
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(dt)[:, :, None, :]
        fit = lambda m: None if m is None else torch.cat([m, torch.zeros_like(m[..., :1])], dim=-1)
        out, cur, hf = R.qabs_reuse_step_cpu(q, k[:, :, :n], v[:, :, :n], g["dims"], g["cand"], g["top_fraction"],
                                             g["scaling"], g["sink"], g["recent"], g["keep_self"],
                                             fit(pc) if g["use_prev_candidate"] else None,
                                             fit(pf) if g["use_prev_final"] else None, g["block"])
        assert np.array_equal(cur.numpy(), g["candidate"][s][..., : n - 1]), (name, s)
        assert np.array_equal(hf.numpy(), g["final"][s][..., : n - 1]), (name, s)
        np.testing.assert_allclose(out.float().numpy()[:, 0], g["out"][s], rtol=1e-5, atol=1e-6)
        pc, pf = cur, hf
