"""Pins the lagged reuse restatement (oracle/ref_semantics.py:
lagged_reuse_decode_step, previous_final_ess_fraction) against golden vectors
written by the reference's own reuse driver on the CPU
(tests/golden/make_reuse_vectors.py, LAG_SCENARIOS), plus known answers of
the refresh tests."""

import math
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import ref_semantics as R

GOLDEN = Path(__file__).resolve().parent / "golden"
LAG_SCENARIOS = ["lagtop2_s8c5_bf16", "lagrefresh3_s8c5_bf16", "qdrift_s8c5_bf16", "qdriftmaj_s8c5_bf16",
                 "qdrifthead_s8c5_bf16", "qdriftshare_s8c5_bf16", "qdriftcos_s16c10_bf16",
                 "qdriftcoshead_s8c5_bf16", "pconf50_s8c5_bf16", "pconf37p5_s16c10_fp32", "qdrifthead_s8c5_fp32",
                 # the sample_quantile / previous_threshold candidate selections
                 "qdrift_sample64_s8c5_bf16", "qdrifthead_sample64_s8c5_bf16", "lagrefresh1_prevthr_s8c5_bf16",
                 "qdriftmaj_prevthr_s8c5_bf16", "qdriftcos_prevthr_s8c5_bf16"]
_MODE = re.compile(r"(lagtop2|lagrefresh(\d+)|qdrift(?:maj|head|share|cos|coshead)?|pconf(\d+(?:p\d+)?))"
                   r"qabs(\d+)cand(\d+(?:p\d+)?)")


def parse_lagged(mode):
    """(kind, param, dims, candidate fraction) of a lagged mode string (EV:475, 918-955)."""
    m = _MODE.fullmatch(mode)
    assert m, mode
    head = m.group(1)
    kind = "lagrefresh" if m.group(2) else "pconf" if m.group(3) else head
    param = int(m.group(2)) if m.group(2) else float(m.group(3).replace("p", ".")) / 100 if m.group(3) else None
    return kind, param, int(m.group(4)), float(m.group(5).replace("p", ".")) / 100


def load_lagged(name):
    """Inputs and per-step outputs of one lagged golden scenario."""
    z = np.load(GOLDEN / f"reuse_{name}.npz")
    t_max = int(z["t_max"])
    bf = lambda a: (a.astype(np.int32) << 16).view(np.float32)   # bf16 bits -> fp32
    kind, param, dims, cand = parse_lagged(str(z["mode"]))
    return {
        "mode": str(z["mode"]), "kind": kind, "param": param, "dims": dims, "cand": cand,
        "dtype": str(z["dtype"]), "q": z["q"][:, :, :, 0, :], "k": bf(z["k_bf16"]), "v": bf(z["v_bf16"]),
        "t0": int(z["t0"]), "steps": int(z["steps"]), "top_fraction": float(z["top_fraction"]),
        "sink": int(z["sink"]), "recent": int(z["recent"]), "keep_self": bool(z["keep_self"]),
        "scaling": float(z["scaling"]), "out": z["out"][:, :, 0],
        "candidate": np.unpackbits(z["candidate"], axis=-1)[..., :t_max].astype(bool),
        "final": np.unpackbits(z["final"], axis=-1)[..., :t_max].astype(bool),
        "qdims": z["qdim_indices"], "qvals": z["qdim_values"], "refresh_count": z["refresh_head_count"],
        "selection": str(z["selection"]), "sample_size": int(z["sample_size"]), "thresholds": z["thresholds"],
    }


@pytest.mark.parametrize("name", LAG_SCENARIOS)
def test_lagged_steps_match_reference_vectors(name):
    g = load_lagged(name)
    bf16 = g["dtype"] == "bfloat16"
    tol = dict(rtol=1e-2, atol=2e-2) if bf16 else dict(rtol=1e-5, atol=1e-5)
    prev = None
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        hist = n - 1
        if g["kind"] == "pconf" and prev is not None:
            # the decision is a float comparison: the vectors keep clear of it
            kx = np.repeat(g["k"][:, :, :n], g["q"].shape[2] // g["k"].shape[1], axis=1)
            ess = R.previous_final_ess_fraction(g["q"][s], kx, prev["final"], g["scaling"], bf16)
            assert np.abs(ess - g["param"]).min() > 1e-3, (s, ess)
        out, cur, hf, prev, flagged = R.lagged_reuse_decode_step(
            g["q"][s], g["k"][:, :, :n], g["v"][:, :, :n], g["kind"], g["param"], g["dims"], g["cand"],
            g["top_fraction"], g["sink"], g["recent"], g["keep_self"], g["scaling"], prev, bf16,
            selection=g["selection"], sample_size=g["sample_size"])
        assert np.array_equal(cur, g["candidate"][s][..., :hist]), (s, "candidate")
        # thresholds are recorded exactly by the steps that thresholded every
        # head; their last bit follows the order of the S-term partial sums,
        # which the reference's CPU fallback takes in torch's vector order and
        # the oracle in the CUDA kernel's sequential one (QK:91-94)
        want_thr = g["thresholds"][s]
        assert ("thresholds" in prev) == bool(np.isfinite(want_thr).all()), (s, "thresholds recorded")
        if "thresholds" in prev:
            np.testing.assert_allclose(prev["thresholds"].reshape(want_thr.shape), want_thr, rtol=1e-6, atol=0)
        assert np.array_equal(hf, g["final"][s][..., :hist]), (s, "final")
        assert np.array_equal(np.sort(prev["dims"], axis=-1), np.sort(g["qdims"][s], axis=-1)), (s, "dims")
        order = np.argsort(g["qdims"][s], axis=-1)
        mine = np.argsort(prev["dims"], axis=-1)
        assert np.array_equal(np.take_along_axis(prev["values"], mine, -1),
                              np.take_along_axis(g["qvals"][s], order, -1)), (s, "values")
        np.testing.assert_allclose(out[:, 0], g["out"][s], **tol)
        # the flagged heads of the per-head kinds are the ones the state counts
        if g["kind"] in ("qdrifthead", "qdriftcoshead", "pconf") and flagged is not None:
            assert int(flagged.sum()) == int(g["refresh_count"][s] - g["refresh_count"][s - 1]), s


def test_lagged_refresh_patterns_are_mixed():
    # the vectors exercise every branch: steps that reuse the previous final
    # selection alone, steps that refresh every head, and per-head refreshes
    seen = set()
    for name in LAG_SCENARIOS:
        g = load_lagged(name)
        for s in range(1, g["steps"]):
            rows = g["candidate"][s][..., : g["t0"] + s].any(axis=-1)
            seen.add("none" if not rows.any() else "all" if rows.all() else "some")
    assert seen == {"none", "all", "some"}


def test_ess_fraction_known_answers():
    # equal scores: ESS = count, fraction 1; one dominant token: ESS -> 1;
    # an empty previous set counts as 1e12 (all weights 0, EV:4080-4084)
    q = np.zeros((1, 2, 4), np.float32)
    k = np.zeros((1, 2, 6, 4), np.float32)
    m = np.zeros((1, 2, 6), bool)
    m[0, 0, [1, 3, 4]] = True
    assert R.previous_final_ess_fraction(q, k, m, 1.0)[0, 0] == pytest.approx(1.0)
    assert R.previous_final_ess_fraction(q, k, m, 1.0)[0, 1] == 1e12
    q[0, 0, 0] = 1.0
    k[0, 0, 3, 0] = 100.0
    assert R.previous_final_ess_fraction(q, k, m, 1.0)[0, 0] == pytest.approx(1 / 3, rel=1e-6)
    # two tokens with weights p, 1-p: ESS = 1 / (p^2 + (1-p)^2)
    k[0, 0, 3, 0] = math.log(3.0)
    m[0, 0] = False
    m[0, 0, [1, 3]] = True
    p = 0.75
    assert R.previous_final_ess_fraction(q, k, m, 1.0)[0, 0] == pytest.approx(1 / (p * p + (1 - p) ** 2) / 2)


def test_ess_fraction_at_the_pconf_threshold():
    # fractions exactly at a threshold (pconf flags only above it, EV:4085), in
    # the reference's float32: weights (1, 0) give exactly 0.5; four equal
    # weights exactly 1.0; three equal weights 1/3 each, whose squares sum to
    # 0.33333337 in float32, 0.99999994 (float64 would give 1.0000000000000002)
    q = np.zeros((1, 3, 128), np.float32)
    q[..., 0] = 1.0
    k = np.zeros((1, 3, 5, 128), np.float32)
    k[0, 0, 1, 0] = -2000.0          # score -177: exp underflows to 0
    m = np.zeros((1, 3, 4), bool)
    m[0, 0, :2] = True
    m[0, 1, :4] = True
    m[0, 2, :3] = True
    fr = R.previous_final_ess_fraction(q, k, m, 128 ** -0.5, bf16_scores=True)[0]
    assert fr.dtype == np.float32
    assert fr[0] == np.float32(0.5) and fr[1] == np.float32(1.0)
    assert fr[2] == np.float32(1.0) - np.float32(2.0 ** -24)
    assert (fr > np.float32(0.5)).tolist() == [False, True, True]
    assert (fr > np.float32(1.0)).tolist() == [False, False, False]


def test_drift_cosine_at_the_threshold():
    # q on the previous dims (1, 0, 0, 0) against previous values (1, 1, 1, 1):
    # cosine exactly 0.5, not flagged (the test is cos < 0.5, EV:4056); a
    # slightly larger last value takes it below 0.5
    q = np.zeros((1, 2, 16), np.float32)
    q[0, :, 0] = 1.0                 # top-4 |q| dims: 0 then the zeros 1, 2, 3 (lowest index first)
    k = np.zeros((1, 2, 20, 16), np.float32)
    prev = {"final": np.ones((1, 2, 18), bool), "dims": np.array([[[0, 1, 2, 3], [0, 1, 2, 3]]]),
            "values": np.array([[[1, 1, 1, 1], [1, 1, 1, 1.01]]], np.float32)}
    *_, flagged = R.lagged_reuse_decode_step(q, k, k, "qdriftcoshead", None, 4, 0.1, 0.1, 0, 0, True, 0.25, prev)
    assert flagged.tolist() == [[False, True]]


def test_drift_flags_known_answers():
    # S = 4 dims: a head whose top dims keep 2 of 4 is not flagged (2 >= ceil(4/2)),
    # one keeping 1 is; the cosine test flags a head whose q on the previous
    # dims turned against the previous values
    q = np.zeros((1, 2, 16), np.float32)
    q[0, 0, [0, 1, 8, 9]] = [4, 3, 2, 1]
    q[0, 1, [0, 10, 11, 12]] = [-4, 3, 2, 1]
    k = np.random.default_rng(0).standard_normal((1, 2, 20, 16)).astype(np.float32)
    prev = {"final": np.ones((1, 2, 18), bool), "dims": np.array([[[0, 1, 2, 3], [0, 1, 2, 3]]]),
            "values": np.array([[[4, 3, 2, 1], [4, 3, 2, 1]]], np.float32)}
    args = (k, k, 4, 0.1, 0.1, 0, 0, True, 0.25, prev)
    *_, flagged = R.lagged_reuse_decode_step(q, *args[:1], args[1], "qdrifthead", None, *args[2:])
    assert flagged.tolist() == [[False, True]]
    q[0, 0, [0, 1]] = [-4, -3]           # same dims, opposite direction: cosine -1
    *_, flagged = R.lagged_reuse_decode_step(q, k, k, "qdriftcoshead", None, 4, 0.1, 0.1, 0, 0, True, 0.25, prev)
    assert flagged.tolist() == [[True, True]]
    *_, flagged = R.lagged_reuse_decode_step(q, k, k, "qdrifthead", None, 4, 0.1, 0.1, 0, 0, True, 0.25, prev)
    assert flagged.tolist() == [[False, True]]


def test_lagged_union_known_answers():
    # lagtop2 with a previous final mask: no new candidates, the union is the
    # previous selection plus sink and recent, so with a keep budget as large
    # as the union the final mask equals that union
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 2, 8)).astype(np.float32)
    k = rng.standard_normal((1, 1, 41, 8)).astype(np.float32)
    pf = np.zeros((1, 2, 39), bool)
    pf[0, 0, [5, 17]] = True
    pf[0, 1, [30]] = True
    prev = {"final": pf, "dims": np.zeros((1, 2, 2), np.int64), "values": np.zeros((1, 2, 2), np.float32)}
    _, cur, hf, _, flagged = R.lagged_reuse_decode_step(q, k, k, "lagtop2", None, 2, 0.1, 1.0, 2, 3, True, 0.3,
                                                        prev)
    assert not cur.any() and flagged is None
    want = np.zeros((1, 2, 40), bool)
    want[..., :2] = want[..., 37:] = True
    want[0, 0, [5, 17]] = want[0, 1, 30] = True
    assert np.array_equal(hf, want)
    # lagrefresh5 at history 40 refreshes: candidates are the top-4 partial scores
    _, cur, hf, _, _ = R.lagged_reuse_decode_step(q, k, k, "lagrefresh", 5, 2, 0.1, 1.0, 2, 3, True, 0.3, prev)
    assert cur.sum(axis=-1).min() >= 4 and (hf >= cur).all() and (hf >= want).all()
