"""Pins the block-metadata selectors of oracle/ref_semantics.py (qbb: Quest-style
channel bounds; brep: block representatives) against golden vectors written
by the reference's own drivers (tests/golden/make_reuse_vectors.py), the
upper-bound property that defines the Quest bound, and known answers."""

import re
from pathlib import Path

import numpy as np
import pytest

from oracle import ref_semantics as R

GOLDEN = Path(__file__).resolve().parent / "golden"
BLOCK_SCENARIOS = ["qbb16q8s12cand4_fp32", "qbb8q16s25cand6p25_fp32", "brep16r2q8s12cand4_fp32",
                   "brep8r1q16s25cand6p25_fp32", "qboracle16q8s12cand4_fp32", "qboracle8q16s25cand6p25_fp32",
                   "qboracle16q8s12cand4_bf16"]
ATTN_SCENARIOS = ["qabs8cand3attn_fp32", "qabs16cand10attn_fp32", "qabs8cand5attn_bf16"]
APPEND_SCENARIOS = ["qabs8cand5appendattn_fp32", "qabs16cand10appendattn_bf16"]
PERIODIC_SCENARIOS = ["qabs8cand5r3attn_fp32", "qabs8cand3r2attn_bf16"]


def parse_block_mode(mode):
    """(kind, block, reps, dims, scan fraction, candidate fraction) of a qbb / brep /
    qboracle mode; ("qabs", 1, 1, dims, 1.0, candidate fraction) of a qabs{S}cand{pct}attn mode."""
    pct = lambda x: float(x.replace("p", ".")) / 100.0   # noqa: E731
    m = re.fullmatch(r"qbb(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)", mode)
    if m:
        return "qbb", int(m.group(1)), 1, int(m.group(2)), pct(m.group(3)), pct(m.group(4))
    m = re.fullmatch(r"qboracle(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)", mode)
    if m:
        return "qboracle", int(m.group(1)), 1, int(m.group(2)), pct(m.group(3)), pct(m.group(4))
    m = re.fullmatch(r"qabs(\d+)cand(\d+(?:p\d+)?)(?:append|r\d+)?attn", mode)
    if m:
        return "qabs", 1, 1, int(m.group(1)), 1.0, pct(m.group(2))
    m = re.fullmatch(r"brep(\d+)r(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)", mode)
    return "brep", int(m.group(1)), int(m.group(2)), int(m.group(3)), pct(m.group(4)), pct(m.group(5))


def load_block_golden(name):
    z = np.load(GOLDEN / f"block_{name}.npz")
    t_max = int(z["t_max"])
    bf = lambda a: (a.astype(np.int32) << 16).view(np.float32)   # noqa: E731
    kind, block, reps, dims, scan, cand = parse_block_mode(str(z["mode"]))
    return {
        "mode": str(z["mode"]), "kind": kind, "block": block, "reps": reps, "dims": dims, "scan": scan,
        "cand": cand, "q": z["q"][:, :, :, 0, :], "k": bf(z["k_bf16"]), "v": bf(z["v_bf16"]), "t0": int(z["t0"]),
        "steps": int(z["steps"]), "top_fraction": float(z["top_fraction"]), "sink": int(z["sink"]),
        "recent": int(z["recent"]), "keep_self": bool(z["keep_self"]), "scaling": float(z["scaling"]),
        "out": z["out"][:, :, 0], "final": np.unpackbits(z["final"], axis=-1)[..., :t_max].astype(bool),
        "append": str(z["mode"]).endswith("appendattn"),
        "interval": (int(re.fullmatch(r"qabs\d+cand\d+(?:p\d+)?r(\d+)attn", str(z["mode"])).group(1))
                     if re.fullmatch(r"qabs\d+cand\d+(?:p\d+)?r\d+attn", str(z["mode"])) else None),
    }


@pytest.mark.parametrize("name", BLOCK_SCENARIOS)
def test_block_steps_match_reference_vectors(name):
    g = load_block_golden(name)
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        out, keep = R.block_select_step(g["q"][s], g["k"][:, :, :n], g["v"][:, :, :n], g["kind"], g["block"],
                                        g["dims"], g["scan"], g["cand"], g["top_fraction"], g["scaling"], g["sink"],
                                        g["recent"], g["keep_self"], g["reps"])
        assert np.array_equal(keep, g["final"][s][..., :n]), (name, s)
        tol = dict(rtol=1e-2, atol=2e-2) if name.endswith("bf16") else dict(rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(out[:, 0], g["out"][s], **tol)


@pytest.mark.parametrize("name", ATTN_SCENARIOS + APPEND_SCENARIOS)
def test_qabs_attn_steps_match_reference_vectors(name):
    # the timed qabs{S}cand{pct}attn mode: every step's final index set
    # bit-exact, outputs to 1e-5 (fp32) / the bf16 attention tolerance
    g = load_block_golden(name)
    tol = dict(rtol=1e-5, atol=1e-5) if name.endswith("fp32") else dict(rtol=1e-2, atol=2e-2)
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        out, keep = R.qabs_attn_step(g["q"][s], g["k"][:, :, :n], g["v"][:, :, :n], g["dims"], g["cand"],
                                     g["scaling"], g["sink"], g["recent"], g["keep_self"], g["append"])
        assert np.array_equal(keep, g["final"][s][..., :n]), (name, s)
        np.testing.assert_allclose(out[:, 0], g["out"][s], **tol)
        if g["append"]:   # the vectors hold selected copies of protected tokens, which count twice
            plain, _ = R.qabs_attn_step(g["q"][s], g["k"][:, :, :n], g["v"][:, :, :n], g["dims"], g["cand"],
                                        g["scaling"], g["sink"], g["recent"], g["keep_self"])
            assert np.abs(plain - out).max() > 1e-3, (name, s)


@pytest.mark.parametrize("name", PERIODIC_SCENARIOS)
def test_qabs_periodic_steps_match_reference_vectors(name):
    # qabs{S}cand{pct}r{N}attn: the selection made at a multiple of N (or on
    # the first step) is reused until the next one, with the protected tokens
    # of each step's own history; every step's final set and output
    g = load_block_golden(name)
    tol = dict(rtol=1e-5, atol=1e-5) if name.endswith("fp32") else dict(rtol=1e-2, atol=2e-2)
    prev, reused = None, 0
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        out, keep, sel = R.qabs_periodic_step(g["q"][s], g["k"][:, :, :n], g["v"][:, :, :n], g["dims"], g["cand"],
                                              g["interval"], g["scaling"], g["sink"], g["recent"], g["keep_self"],
                                              prev)
        reused += prev is not None and sel is prev
        assert np.array_equal(keep, g["final"][s][..., :n]), (name, s)
        np.testing.assert_allclose(out[:, 0], g["out"][s], **tol)
        prev = sel
    assert 0 < reused < g["steps"] - 1   # the steps both reuse and reselect


@pytest.mark.parametrize("name", ATTN_SCENARIOS)
def test_qabs_attn_cpu_baseline_matches_reference_vectors(name):
    # the torch op sequence bench.py times as the decode CPU baseline
    # (qabs_candidate_attention_cpu) gives the reference driver's outputs
    import torch

    g = load_block_golden(name)
    dt = torch.bfloat16 if name.endswith("bf16") else torch.float32
    k, v = torch.from_numpy(g["k"]).to(dt), torch.from_numpy(g["v"]).to(dt)
    tol = dict(rtol=1e-5, atol=1e-6) if dt == torch.float32 else dict(rtol=0, atol=0)
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s])[:, :, None, :].to(dt)
        out = R.qabs_candidate_attention_cpu(q, k[:, :, :n], v[:, :, :n], g["dims"], g["cand"], g["scaling"],
                                             g["sink"], g["recent"], g["keep_self"])
        np.testing.assert_allclose(out.float().numpy()[:, 0], g["out"][s], **tol)


def test_block_minmax_brute_force():
    rng = np.random.default_rng(0)
    k = rng.standard_normal((2, 37, 5)).astype(np.float32)
    lo, hi = R.block_minmax(k, 8)
    assert lo.shape == (2, 5, 5)
    for j in range(5):
        seg = k[:, 8 * j: min(37, 8 * j + 8)]
        assert np.array_equal(lo[:, j], seg.min(axis=1)) and np.array_equal(hi[:, j], seg.max(axis=1))


def test_qbb_bound_is_an_upper_bound():
    # q.k over the selected dims never exceeds the block's bound, and a block
    # holding the maximizing corner reaches it (a sign slip breaks one of them)
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 3, 16)).astype(np.float32)
    k = rng.standard_normal((1, 3, 96, 16)).astype(np.float32)
    lo, hi = R.block_minmax(k, 16)
    bound = R.qbb_block_bounds(q, lo, hi, 6)
    part = R.partial_scores(q, k, 6)
    for h in range(3):
        for j in range(6):
            assert part[0, h, 16 * j: 16 * j + 16].max() <= bound[0, h, j] + 1e-5
    dims = R.select_dims_by_abs(q[0, 0], 6)
    corner = np.where(q[0, 0] >= 0, hi[0, 0, 2], lo[0, 0, 2])
    kc = k.copy()
    kc[0, 0, 32] = corner                       # block 2 now holds its own corner
    assert np.isclose(R.partial_scores(q, kc, 6)[0, 0, 32], bound[0, 0, 2], rtol=1e-6)
    assert dims.size == 6


def test_block_representatives_known_answer():
    # norms 1, 9, 4, 9 | 16, 0 : ties to the lower position, descending norm
    k = np.array([1, 3, 2, -3, 4, 0], np.float32).reshape(1, 6, 1)
    idx, valid = R.block_representatives(k, 4, 2)
    assert idx.tolist() == [[[1, 3], [4, 5]]] and valid.all()
    idx, valid = R.block_representatives(k[:, :5], 4, 3)
    assert idx.tolist() == [[[1, 3, 2], [4, 0, 0]]]
    assert valid.tolist() == [[[True, True, True], [True, False, False]]]


def test_brep_score_is_max_over_representatives():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 2, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 40, 8)).astype(np.float32)
    idx, valid = R.block_representatives(k, 16, 3)
    sc = R.brep_block_scores(q, k, idx, valid, 4)
    part = R.partial_scores(q, k, 4)
    for h in range(2):
        for j in range(3):
            reps = idx[0, h, j][valid[0, h, j]]
            assert sc[0, h, j] == part[0, h, reps].max()


@pytest.mark.parametrize("name", BLOCK_SCENARIOS)
def test_cpu_baseline_op_sequence_matches_reference_vectors(name):
    # the torch op sequence bench.py times as the block-selector CPU baseline
    import torch

    g = load_block_golden(name)
    dt = torch.bfloat16 if name.endswith("bf16") else torch.float32
    k, v = torch.from_numpy(g["k"]).to(dt), torch.from_numpy(g["v"]).to(dt)
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s])[:, :, None, :].to(dt)
        out, keep = R.block_select_step_cpu(q, k[:, :, :n], v[:, :, :n], g["kind"], g["block"], g["dims"], g["scan"],
                                            g["cand"], g["top_fraction"], g["scaling"], g["sink"], g["recent"],
                                            g["keep_self"], g["reps"])
        assert np.array_equal(keep.numpy(), g["final"][s][..., :n]), (name, s)
        np.testing.assert_allclose(out.float().numpy()[:, 0], g["out"][s], rtol=1e-5, atol=1e-6)   # same ops


@pytest.mark.parametrize("name", ["brep16r2q8s12cand4_fp32", "brep8r1q16s25cand6p25_fp32"])
def test_brep_partial_scores_drive_the_reference_caller(name):
    # brep_partial_scores' oracle, fed through the caller's remaining steps
    # (EV:5426-5505), gives the final mask the reference's brep driver wrote
    import math
    g = load_block_golden(name)
    gqa = g["q"].shape[2] // g["k"].shape[1]
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        kh = np.repeat(g["k"][:, :, : n - 1], gqa, axis=1)
        q = g["q"][s]
        ridx, rvalid = R.block_representatives(kh, g["block"], g["reps"])
        part = R.brep_partial_scores(q, kh, ridx, rvalid, g["block"], g["dims"], g["scan"])
        nb = -(-(n - 1) // g["block"])
        n_scan = min(nb, max(1, math.ceil(g["scan"] * (n - 1) / g["block"])))
        assert (np.isfinite(part).sum(axis=-1) <= n_scan * g["block"]).all()
        for bi in range(q.shape[0]):
            for hi in range(q.shape[1]):
                final = R.brep_caller_final_mask(part[bi, hi], q[bi, hi], kh[bi, hi], n, g["cand"], g["top_fraction"],
                                                 g["scaling"], g["sink"], g["recent"], g["keep_self"])
                assert np.array_equal(final, g["final"][s][bi, hi, :n]), (name, s, bi, hi)


def test_brep_partial_scores_known_answer():
    # 2 blocks of 2 tokens, one dim: representative = larger |k|; block 1 wins
    q = np.array([[[2.0]]], np.float32)
    k = np.array([[[[1.0], [-3.0], [2.0], [0.5]]]], np.float32)
    idx, valid = R.block_representatives(k, 2, 1)
    assert idx.tolist() == [[[[1], [2]]]]
    part = R.brep_partial_scores(q, k, idx, valid, 2, 1, 0.25)     # ceil(0.25 * 4 / 2) = 1 block
    assert part.tolist() == [[[-np.inf, -np.inf, 4.0, 1.0]]]

