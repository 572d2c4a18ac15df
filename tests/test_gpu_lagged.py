"""GPU parity of the lagged reuse modes (lagtop2, lagrefresh{N}, qdrift*,
pconf{T}) against the reference's own golden vectors and the oracle: masks,
refresh flags and recorded dims bit-exact, attention within 1e-2 relative /
2e-2 absolute (bf16)."""

import numpy as np
import pytest
import torch

from kv_cache_amd import qabs_cuda_kernels as Q
from kv_cache_amd import reuse as RU
from oracle import ref_semantics as R
from tests.test_oracle_lagged import LAG_SCENARIOS, load_lagged

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2


def f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("name", [n for n in LAG_SCENARIOS if n.endswith("bf16")])
def test_lagged_step_matches_reference_vectors(name):
    # The GQA-native step on the reference's bf16 scenarios: at every step the
    # candidates, the final mask, the recorded top-|q| dims and the output
    # equal the reference's.
    g = load_lagged(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k = torch.from_numpy(g["k"]).to(torch.bfloat16).to(DEV)
    v = torch.from_numpy(g["v"]).to(torch.bfloat16).to(DEV)
    step = RU.LaggedReuseDecodeStep(g["mode"], 1, hq, hkv, 128, 1024, top_fraction=g["top_fraction"],
                                    protect_sink=g["sink"], protect_recent=g["recent"], keep_self=g["keep_self"],
                                    candidate_selection=g["selection"], threshold_sample_size=g["sample_size"])
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(torch.bfloat16).to(DEV)
        out = step(q, k[:, :, :n], v[:, :, :n], g["scaling"])
        assert np.array_equal(step.candidate_mask().cpu().numpy(), g["candidate"][s][..., : n - 1]), s
        assert np.array_equal(step.final_mask().cpu().numpy(), g["final"][s][..., : n - 1]), s
        want_thr = g["thresholds"][s].reshape(-1)
        if g["selection"] != "topk":
            # the step keeps thresholds only after thresholding every row
            assert step.thr_valid == bool(np.isfinite(want_thr).all()), s
            if step.thr_valid:   # the partial sums' order sets the last bit (QK:91-94 vs the CPU fallback)
                np.testing.assert_allclose(step.thresholds.cpu().numpy(), want_thr, rtol=1e-6, atol=0)
        if RU.LAGGED_KINDS[g["kind"]][0] is not None:
            dims = step.qdims[1 - step.flip].view(1, hq, -1).cpu().numpy()
            assert np.array_equal(np.sort(dims, axis=-1), np.sort(g["qdims"][s], axis=-1)), s
        np.testing.assert_allclose(f32(out), g["out"][s], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("name", [n for n in LAG_SCENARIOS if n.endswith("fp32")])
def test_lagged_pieces_match_reference_vectors(name):
    # The fp32 scenarios through the C-ABI pieces on GQA-expanded K (the
    # reference's hook expands it): refresh flags, union, rerank and final
    # mask equal the reference's at every step.
    g = load_lagged(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k_all = torch.from_numpy(np.repeat(g["k"], hq // hkv, axis=1)).to(DEV)
    v_all = torch.from_numpy(np.repeat(g["v"], hq // hkv, axis=1)).to(DEV)
    test, per = RU.LAGGED_KINDS[g["kind"]]
    t_max = k_all.shape[2]
    s_count = g["dims"]
    dims = [torch.zeros((hq, s_count), dtype=torch.int32, device=DEV) for _ in range(2)]
    vals = [torch.zeros((hq, s_count), dtype=torch.float32, device=DEV) for _ in range(2)]
    flags = torch.zeros(hq, dtype=torch.uint8, device=DEV)
    cur = torch.zeros((hq, t_max), dtype=torch.uint8, device=DEV)
    fin = torch.zeros((hq, t_max), dtype=torch.uint8, device=DEV)
    uni = torch.zeros((hq, t_max), dtype=torch.uint8, device=DEV)
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        hist = n - 1
        q = torch.from_numpy(g["q"][s]).to(DEV)
        k, v = k_all[:, :, :n], v_all[:, :, :n]
        has_prev = s > 0
        run = test if has_prev else "dims"
        RU.lag_flags(q, hq, run, s_count, dims[s % 2], vals[s % 2], flags, previous_dims=dims[1 - s % 2],
                     previous_values=vals[1 - s % 2], key=k, history=hist, previous_final=fin,
                     scaling=g["scaling"], ess_threshold=g["param"] or 0.0)
        refresh = per if has_prev else "all"
        part = Q.partial_scores(q, k[:, :, :hist], s_count).view(hq, hist)
        req = R.budget_count(hist, g["cand"])
        ws = torch.empty(max(1, Q._lib.load().qkv_threshold_mask_workspace_bytes(hq, hist, req)) // 4 + 1,
                         dtype=torch.float32, device=DEV)
        RU.threshold_mask(part, hist, req, cur, ws)
        RU.lag_union(cur, fin if has_prev else None, flags, 1, hq, hist, refresh,
                     g["kind"] == "qdriftshare" and has_prev, g["sink"], g["recent"], uni)
        assert np.array_equal(cur[:, :hist].cpu().numpy().astype(bool), g["candidate"][s][0, :, :hist]), s
        fi, fv, hf = Q.reuse_select(q, k, uni[:, :hist].view(torch.bool).view(1, hq, hist), None, None, g["sink"],
                                    g["recent"], g["top_fraction"], g["keep_self"], g["scaling"])
        assert np.array_equal(hf.cpu().numpy(), g["final"][s][..., :hist]), s
        np.testing.assert_allclose(f32(Q.final_attention(q, k, v, fi, fv, g["scaling"]))[:, 0], g["out"][s],
                                   rtol=1e-3, atol=1e-3)
        fin.zero_()
        fin[:, :hist] = hf.view(hq, hist).view(torch.uint8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,hkv,hist,dens", [(8, 2, 3000, 0.03), (4, 4, 70000, 0.2), (6, 3, 37, 0.5),
                                                 (2, 1, 20000, 0.0)])
def test_lag_flags_ess_matches_oracle(dtype, rows, hkv, hist, dens):
    # the ESS statistic over a random previous final mask, every pass size:
    # rows longer than one 32768-position pass, lists past the 8192-entry LDS
    # list, empty masks (flagged); rows within 1e-4 of the threshold are left out
    gen = torch.Generator().manual_seed(rows * 7 + hist)
    q = (torch.randn((1, rows, 128), generator=gen) * 0.5).to(dtype)
    k = torch.randn((1, hkv, hist + 1, 128), generator=gen).to(dtype)
    m = torch.rand((rows, hist), generator=gen) < dens
    if rows > 2:
        m[1] = False
    ld = hist + 13 if hist % 2 else (hist + 15) // 16 * 16 + 16   # byte loads, then 16-byte loads
    mask = torch.zeros((rows, ld), dtype=torch.uint8)
    mask[:, :hist] = m.to(torch.uint8)
    mask[:, hist:] = 1   # past the history: never read
    kx = np.repeat(f32(k), rows // hkv, axis=1)
    ess = R.previous_final_ess_fraction(f32(q), kx, m.numpy()[None], 128 ** -0.5, dtype == torch.bfloat16)[0]
    thr = float(np.median(ess[ess < 1e11])) if (ess < 1e11).any() else 0.5
    flags = torch.full((rows,), 7, dtype=torch.uint8, device=DEV)
    dims = torch.empty((rows, 8), dtype=torch.int32, device=DEV)
    vals = torch.empty((rows, 8), dtype=torch.float32, device=DEV)
    RU.lag_flags(q.to(DEV), hkv, "ess", 8, dims, vals, flags, key=k.to(DEV), history=hist,
                 previous_final=mask.to(DEV), scaling=128 ** -0.5, ess_threshold=thr)
    got = flags.cpu().numpy()
    assert set(got.tolist()) <= {0, 1}
    clear = np.abs(ess - thr) > 1e-4
    assert np.array_equal(got[clear].astype(bool), (ess > thr)[clear])
    if rows > 2:
        assert got[1] == 1   # an empty previous selection refreshes


def test_lag_flags_known_answers_at_the_thresholds():
    # pconf: ESS / count exactly 0.5 (weights 1, 0) and exactly 1.0 (four equal
    # weights) are not above thresholds 0.5 and 1.0 and are above just smaller
    # ones; qdrift cos: cosine exactly 0.5 is not below 0.5, a smaller one is
    q = torch.zeros((1, 2, 128), dtype=torch.bfloat16)
    q[..., 0] = 1.0
    k = torch.zeros((1, 2, 5, 128), dtype=torch.bfloat16)
    k[0, 0, 1, 0] = -2000.0          # score -177: its weight underflows to 0
    mask = torch.zeros((2, 16), dtype=torch.uint8)
    mask[0, :2] = 1
    mask[1, :4] = 1
    dims = torch.empty((2, 8), dtype=torch.int32, device=DEV)
    vals = torch.empty((2, 8), dtype=torch.float32, device=DEV)
    for thr, want in ((0.5, [0, 1]), (0.49999997, [1, 1]), (1.0, [0, 0]), (0.99999994, [0, 1])):
        flags = torch.full((2,), 7, dtype=torch.uint8, device=DEV)
        RU.lag_flags(q.to(DEV), 2, "ess", 8, dims, vals, flags, key=k.to(DEV), history=4,
                     previous_final=mask.to(DEV), scaling=128 ** -0.5, ess_threshold=thr)
        assert flags.cpu().tolist() == want, thr
    qc = torch.zeros((1, 2, 128), dtype=torch.bfloat16, device=DEV)
    qc[..., 0] = 1.0                 # top-4 |q| dims 0, 1, 2, 3
    pd = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 3]], dtype=torch.int32, device=DEV)
    pv = torch.tensor([[1, 1, 1, 1], [1, 1, 1, 1.01]], dtype=torch.float32, device=DEV)
    flags = torch.full((2,), 7, dtype=torch.uint8, device=DEV)
    RU.lag_flags(qc, 2, "cos", 4, dims[:, :4].contiguous(), vals[:, :4].contiguous(), flags, previous_dims=pd,
                 previous_values=pv)
    assert flags.cpu().tolist() == [0, 1]


@pytest.mark.parametrize("s_count", [1, 4, 8, 16, 33, 128])
def test_lag_flags_overlap_and_cos_match_oracle(s_count):
    gen = torch.Generator().manual_seed(s_count)
    rows = 16
    base = torch.randn((1, rows, 128), generator=gen)
    eps = torch.linspace(0, 3, rows).view(1, rows, 1)
    q0 = base.to(torch.bfloat16)
    q1 = (base + eps * torch.randn((1, rows, 128), generator=gen)).to(torch.bfloat16)
    q1[0, 3] = -q0[0, 3]   # same dims, opposite direction: only the cosine test flags it
    dims = [torch.empty((rows, s_count), dtype=torch.int32, device=DEV) for _ in range(2)]
    vals = [torch.empty((rows, s_count), dtype=torch.float32, device=DEV) for _ in range(2)]
    RU.lag_flags(q0.to(DEV), 1, "dims", s_count, dims[0], vals[0])
    want_d = np.stack([R.select_dims_by_abs(f32(q0)[0, r], s_count) for r in range(rows)])
    assert np.array_equal(dims[0].cpu().numpy(), want_d)
    assert np.array_equal(vals[0].cpu().numpy(), np.take_along_axis(f32(q0)[0], want_d, -1))
    prev = {"final": np.ones((1, rows, 4), bool), "dims": want_d[None], "values": vals[0].cpu().numpy()[None]}
    kk = np.zeros((1, 1, 5, 128), np.float32)
    for test, kind in (("overlap", "qdrifthead"), ("cos", "qdriftcoshead")):
        flags = torch.full((rows,), 9, dtype=torch.uint8, device=DEV)
        RU.lag_flags(q1.to(DEV), 1, test, s_count, dims[1], vals[1], flags, previous_dims=dims[0],
                     previous_values=vals[0])
        *_, want = R.lagged_reuse_decode_step(f32(q1), kk, kk, kind, None, s_count, 0.5, 0.5, 0, 0, True, 0.1,
                                              prev)
        assert np.array_equal(flags.cpu().numpy().astype(bool), want[0]), test
        assert 0 < int(flags.sum()) < rows or s_count == 128
        if test == "cos":
            assert flags[3].item() == 1


@pytest.mark.parametrize("refresh,share", [("none", False), ("all", False), ("per_row", False), ("per_row", True),
                                           ("any", False), ("majority", False)])
@pytest.mark.parametrize("batch,hq,hist,ld", [(2, 4, 1000, 1024), (1, 3, 37, 37), (3, 2, 4113, 4200)])
def test_lag_union_matches_numpy(refresh, share, batch, hq, hist, ld):
    gen = torch.Generator().manual_seed(hist + hq)
    rows = batch * hq
    cur = (torch.rand((rows, ld), generator=gen) < 0.05).to(torch.uint8)
    fin = (torch.rand((rows, ld), generator=gen) < 0.03).to(torch.uint8)
    flags = (torch.rand(rows, generator=gen) < 0.4).to(torch.uint8)
    if refresh == "majority":
        flags[: rows // 2 + 1] = 1
    sink, recent = 3, 11
    c, f, fl = cur.numpy().astype(bool)[:, :hist], fin.numpy().astype(bool)[:, :hist], flags.numpy().astype(bool)
    fresh = {"none": np.zeros(rows, bool), "all": np.ones(rows, bool), "per_row": fl,
             "any": np.full(rows, fl.any()), "majority": np.full(rows, fl.sum() * 2 > rows)}[refresh]
    want_cur = c & fresh[:, None]
    want = want_cur | f
    if share:
        want |= np.repeat(want_cur.reshape(batch, hq, hist).any(axis=1), hq, axis=0)
    want[:, :sink] = True
    want[:, max(0, hist - recent):] = True
    cur_d = cur.to(DEV)
    out = torch.full((rows, ld), 5, dtype=torch.uint8, device=DEV)
    RU.lag_union(cur_d, fin.to(DEV), flags.to(DEV), batch, hq, hist, refresh, share, sink, recent, out)
    assert np.array_equal(out[:, :hist].cpu().numpy().astype(bool), want)
    assert (out[:, hist:] == 5).all()
    got_cur = cur_d.cpu().numpy()
    assert np.array_equal(got_cur[:, :hist].astype(bool), want_cur)
    assert np.array_equal(got_cur[:, hist:], cur.numpy()[:, hist:])   # past the history: untouched
    # no previous final mask (a sequence's first step)
    out2 = torch.zeros((rows, ld), dtype=torch.uint8, device=DEV)
    RU.lag_union(cur.to(DEV), None, flags.to(DEV), batch, hq, hist, "all", False, 0, 0, out2)
    assert np.array_equal(out2[:, :hist].cpu().numpy().astype(bool), c)


def _to_words(m):
    # bool [rows, n] -> int64 bitset words [rows, ceil(n / 64)] (bit t % 64 of word t // 64)
    rows, n = m.shape
    n_w = -(-n // 64)
    pad = torch.zeros((rows, n_w * 64), dtype=torch.bool, device=m.device)
    pad[:, :n] = m
    by = (pad.view(rows, -1, 8).to(torch.uint8) << torch.arange(8, dtype=torch.uint8, device=m.device)).sum(-1)
    return by.to(torch.uint8).contiguous().view(torch.int64)


@pytest.mark.parametrize("refresh,share", [("none", False), ("all", False), ("per_row", False), ("per_row", True),
                                           ("any", False), ("majority", False)])
@pytest.mark.parametrize("batch,hq,hist", [(2, 4, 1000), (1, 3, 37), (3, 2, 4113), (1, 2, 128)])
def test_lag_union_bits_equals_bytes(refresh, share, batch, hq, hist):
    # qkv_reuse_lag_union_bits against the byte-mask union on the same masks:
    # the same union and the same cleared candidates, words past the history untouched
    gen = torch.Generator().manual_seed(hist * 3 + hq)
    rows = batch * hq
    cur = (torch.rand((rows, hist), generator=gen) < 0.05).to(DEV)
    fin = (torch.rand((rows, hist), generator=gen) < 0.03).to(DEV)
    flags = (torch.rand(rows, generator=gen) < 0.4).to(torch.uint8).to(DEV)
    if refresh == "majority":
        flags[: rows // 2 + 1] = 1
    cur_b, out_b = cur.to(torch.uint8), torch.zeros((rows, hist), dtype=torch.uint8, device=DEV)
    RU.lag_union(cur_b, fin.to(torch.uint8), flags, batch, hq, hist, refresh, share, 3, 11, out_b)
    n_w = -(-hist // 64)
    cur_w = torch.cat([_to_words(cur), torch.full((rows, 1), 5, dtype=torch.int64, device=DEV)], 1)
    fin_w = torch.cat([_to_words(fin), torch.zeros((rows, 1), dtype=torch.int64, device=DEV)], 1)
    out_w = torch.full((rows, n_w + 1), 7, dtype=torch.int64, device=DEV)
    RU.lag_union(cur_w, fin_w, flags, batch, hq, hist, refresh, share, 3, 11, out_w)
    assert torch.equal(RU.expand_bits(out_w, hist), out_b.bool())
    assert torch.equal(RU.expand_bits(cur_w, hist), cur_b.bool())
    assert bool((out_w[:, n_w] == 7).all()) and bool((cur_w[:, n_w] == 5).all())
    if hist % 64:   # no bit past the history in the last word
        assert not RU.expand_bits(out_w[:, :n_w], n_w * 64)[:, hist:].any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,hkv,hist,dens", [(8, 2, 3000, 0.03), (4, 4, 70000, 0.2), (6, 3, 37, 0.5)])
def test_lag_flags_ess_bits_equals_bytes(dtype, rows, hkv, hist, dens):
    gen = torch.Generator().manual_seed(rows * 11 + hist)
    q = (torch.randn((1, rows, 128), generator=gen) * 0.5).to(dtype).to(DEV)
    k = torch.randn((1, hkv, hist + 1, 128), generator=gen).to(dtype).to(DEV)
    m = (torch.rand((rows, hist), generator=gen) < dens).to(DEV)
    outs = []
    for fin in (m.to(torch.uint8), _to_words(m)):
        flags = torch.full((rows,), 7, dtype=torch.uint8, device=DEV)
        dims = torch.empty((rows, 8), dtype=torch.int32, device=DEV)
        vals = torch.empty((rows, 8), dtype=torch.float32, device=DEV)
        RU.lag_flags(q, hkv, "ess", 8, dims, vals, flags, key=k, history=hist, previous_final=fin,
                     scaling=128 ** -0.5, ess_threshold=0.3)
        outs.append((flags, dims, vals))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("refresh", ["all", "per_row", "any", "majority", "none"])
@pytest.mark.parametrize("hist", [3000, 32790, 50000])
def test_lag_candidates_bits_equals_bytes(refresh, hist):
    # the refreshing rows' candidate bits equal the byte path's mask; past
    # 40960 positions the rows take the one-workgroup path; the workspace
    # state is left zero
    gen = torch.Generator().manual_seed(hist + 17)
    b, hq, hkv, d, s_count = 2, 4, 2, 128, 8
    rows = b * hq
    k = torch.randn((b, hkv, hist + 1, d), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16).to(DEV)
    kdm = torch.zeros((b, hkv, d, hist + 64), dtype=torch.bfloat16, device=DEV)
    RU.dim_major_append(k, kdm, 0, hist)
    flags = torch.tensor([1, 0, 0, 1, 0, 1, 0, 0], dtype=torch.uint8, device=DEV)
    if refresh == "majority":
        flags[:5] = 1
    lib = Q._lib.load()
    req = R.budget_count(hist, 0.05)
    ws = torch.empty(lib.qkv_threshold_mask_workspace_bytes(rows, hist, req) // 4 + 1, dtype=torch.float32,
                     device=DEV)
    part = torch.full((rows, hist + 64), -7.0, device=DEV)
    mask = torch.full((rows, hist + 64), 9, dtype=torch.uint8, device=DEV)
    RU.lag_candidates(q, kdm, hist, s_count, req, flags, refresh, part, mask, ws)
    n_w = -(-hist // 64)
    cws = torch.zeros(lib.qkv_reuse_candidates_workspace_bytes(rows, hist, req) // 4 + 1, dtype=torch.float32,
                      device=DEV)
    part_b = torch.full((rows, hist + 64), -7.0, device=DEV)
    words = torch.full((rows, n_w + 1), 3, dtype=torch.int64, device=DEV)
    for _ in range(2):   # twice through one workspace
        RU.lag_candidates(q, kdm, hist, s_count, req, flags, refresh, part_b, words, cws)
    assert not cws[: rows * 4096].any()   # the per-row histograms are clear again
    fl = flags.cpu().numpy().astype(bool)
    fresh = {"all": np.ones(rows, bool), "none": np.zeros(rows, bool), "per_row": fl,
             "any": np.full(rows, fl.any()), "majority": np.full(rows, 2 * fl.sum() > rows)}[refresh]
    got = RU.expand_bits(words[:, :n_w], hist)
    for r in range(rows):
        if fresh[r]:
            assert torch.equal(part_b[r, :hist], part[r, :hist]), r
            assert torch.equal(got[r], mask[r, :hist].bool()), r
        elif hist <= 40960:   # rows that keep are not touched
            assert bool((part_b[r] == -7.0).all()) and bool((words[r] == 3).all()), r
    assert bool((words[:, n_w] == 3).all())


def test_lag_entry_points_reject_bad_arguments():
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device=DEV)
    d = torch.zeros((4, 8), dtype=torch.int32, device=DEV)
    v = torch.zeros((4, 8), dtype=torch.float32, device=DEV)
    fl = torch.zeros(4, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="need the previous dims"):
        RU.lag_flags(q, 2, "overlap", 8, d, v, fl)
    with pytest.raises(RuntimeError, match="ESS test needs K"):
        RU.lag_flags(q, 2, "ess", 8, d, v, fl, history=10)
    with pytest.raises(RuntimeError, match="head_dim must be in"):
        RU.lag_flags(torch.zeros((1, 4, 256), dtype=torch.bfloat16, device=DEV), 2, "dims", 8, d, v)
    m = torch.zeros((4, 64), dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="null flags"):
        RU.lag_union(m, None, None, 1, 4, 64, "any", False, 0, 0, m.clone())
    with pytest.raises(RuntimeError, match="mask_ld and union_ld"):
        RU.lag_union(m, None, fl, 1, 4, 65, "all", False, 0, 0, m.clone())
    with pytest.raises(RuntimeError, match="not a lagged reuse mode"):
        RU.LaggedReuseDecodeStep("qabs8cand5reuse", 1, 4, 2, 128, 256)
    with pytest.raises(RuntimeError, match="unknown candidate selection"):
        RU.LaggedReuseDecodeStep("pconf50qabs8cand5", 1, 4, 2, 128, 256, candidate_selection="median")


@pytest.mark.parametrize("mode", ["pconf50qabs8cand5", "qdriftmajqabs8cand5", "lagrefresh2qabs8cand5"])
def test_lagged_step_graph_replays(mode):
    # a lagged step captured at a fixed history: every replay, with a new query
    # copied in and the outputs cleared between replays, matches the eager launch
    gen = torch.Generator().manual_seed(len(mode))
    t = 2000
    k = torch.randn((1, 2, t + 3, 128), generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn((1, 2, t + 3, 128), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((1, 8, 128), generator=gen).to(torch.bfloat16).to(DEV)
    step = RU.LaggedReuseDecodeStep(mode, 1, 8, 2, 128, t + 64, top_fraction=0.02, protect_sink=4, protect_recent=8)
    for n in (t, t + 1, t + 2):
        step(q, k[:, :, :n], v[:, :, :n], 128 ** -0.5)
    cur = step.cand[step.flip]
    fin_prev = step.fin.clone()
    kk, vv = k[:, :, : t + 3], v[:, :, : t + 3]
    if step.kdm_len < t + 2:
        RU.dim_major_append(kk, step.kdm, step.kdm_len, t + 2)
        step.kdm_len = t + 2

    def launch():
        step.fin.copy_(fin_prev)
        step.launch(q, kk, vv, 128 ** -0.5, cur, None, step.fin)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    outs = (cur, step.fin, step.flags, step.out, step.union)
    for rep in range(4):
        q.copy_(torch.randn((1, 8, 128), generator=gen).to(torch.bfloat16))
        launch()
        want = [x.clone() for x in outs]
        for x in outs:
            x.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for w, x in zip(want, outs):
            assert torch.equal(w, x), rep


@pytest.mark.parametrize("refresh", ["all", "per_row", "any", "majority", "none"])
@pytest.mark.parametrize("hist", [3000, 50000])   # one workgroup per row; past it, every row is computed
def test_lag_candidates_skip_rows_that_keep(refresh, hist):
    gen = torch.Generator().manual_seed(hist)
    b, hq, hkv, d, s_count = 2, 4, 2, 128, 8
    rows = b * hq
    k = torch.randn((b, hkv, hist + 1, d), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16).to(DEV)
    kdm = torch.zeros((b, hkv, d, hist + 64), dtype=torch.bfloat16, device=DEV)
    RU.dim_major_append(k, kdm, 0, hist)
    flags = torch.tensor([1, 0, 0, 1, 0, 1, 0, 0], dtype=torch.uint8, device=DEV)
    if refresh == "majority":
        flags[:5] = 1
    req = R.budget_count(hist, 0.05)
    ws = torch.empty(Q._lib.load().qkv_threshold_mask_workspace_bytes(rows, hist, req) // 4 + 1,
                     dtype=torch.float32, device=DEV)
    part = torch.full((rows, hist + 64), -7.0, device=DEV)
    mask = torch.full((rows, hist + 64), 9, dtype=torch.uint8, device=DEV)
    RU.lag_candidates(q, kdm, hist, s_count, req, flags, refresh, part, mask, ws)
    want_p = RU.reuse_partial_scores(q, kdm, hist, s_count)
    want_m = torch.zeros((rows, hist), dtype=torch.uint8, device=DEV)
    RU.threshold_mask(want_p, hist, req, want_m, ws)
    fl = flags.cpu().numpy().astype(bool)
    fresh = {"all": np.ones(rows, bool), "none": np.zeros(rows, bool), "per_row": fl,
             "any": np.full(rows, fl.any()), "majority": np.full(rows, 2 * fl.sum() > rows)}[refresh]
    for r in range(rows):
        if fresh[r]:
            assert torch.equal(part[r, :hist], want_p[r]), r
            assert torch.equal(mask[r, :hist], want_m[r]), r
        elif hist <= 40960:   # rows that keep are not touched
            assert bool((part[r] == -7.0).all()) and bool((mask[r] == 9).all()), r
    assert bool((mask[:, hist:] == 9).all())


@pytest.mark.parametrize("mode", ["lagtop2qabs8cand5", "lagrefresh2qabs8cand5", "qdriftqabs8cand5",
                                  "qdriftmajqabs8cand5", "qdriftheadqabs8cand5", "qdriftshareqabs8cand5",
                                  "qdriftcosqabs16cand10", "qdriftcosheadqabs8cand5", "pconf60qabs8cand5"])
def test_lagged_step_matches_oracle_multistep(mode):
    # every lagged kind over 5 steps at 3000 history tokens, GQA 4, queries
    # drifting slowly on some heads and jumping on others (refreshes of no,
    # some and every head); masks bit-exact to the oracle at every step
    gen = torch.Generator().manual_seed(len(mode) * 7 + 1)
    t, steps, hq, hkv = 3000, 5, 8, 2
    kind, param, dims, cand = RU.parse_lagged_mode(mode)
    eps = torch.tensor([0.02, 3.0, 0.05, 0.3, 0.01, 2.0, 0.1, 1.0]).view(1, 1, hq, 1)
    base = torch.randn((1, 1, hq, 128), generator=gen)
    q = ((base + eps * torch.randn((steps, 1, hq, 128), generator=gen)) / torch.sqrt(1 + eps * eps)).to(torch.bfloat16)
    k = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.LaggedReuseDecodeStep(mode, 1, hq, hkv, 128, t + 64, top_fraction=0.02, protect_sink=4,
                                    protect_recent=8)
    prev = None
    for s in range(steps):
        n = t + s + 1
        if kind == "pconf" and prev is not None:   # the seed keeps every row's ESS clear of the threshold
            kx = np.repeat(f32(k[:, :, :n]), hq // hkv, axis=1)
            ess = R.previous_final_ess_fraction(f32(q[s]), kx, prev["final"], 128 ** -0.5, True)
            assert np.abs(ess - param).min() > 1e-3, s
        out = step(q[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, wc, wf, prev, flagged = R.lagged_reuse_decode_step(f32(q[s]), f32(k[:, :, :n]), f32(v[:, :, :n]),
                                                                 kind, param, dims, cand, 0.02, 4, 8, True,
                                                                 128 ** -0.5, prev, True)
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        if flagged is not None and kind in ("qdrifthead", "qdriftcoshead", "qdriftshare", "pconf"):
            assert np.array_equal(step.flags.cpu().numpy().astype(bool), flagged.reshape(-1)), s
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("mode", ["qdriftheadqabs8cand5", "qdriftmajqabs8cand5"])
def test_lagged_step_long_rows_match_oracle(mode):
    # 45000 history tokens: past the one-workgroup selection, the candidates of
    # every row are thresholded by the staged top-k (rows that keep included,
    # their scores stale) and the union clears the rows that keep
    gen = torch.Generator().manual_seed(len(mode) * 11)
    t, steps, hq, hkv = 45000, 3, 8, 2
    kind, param, dims, cand = RU.parse_lagged_mode(mode)
    eps = torch.tensor([0.02, 3.0, 0.05, 0.3, 0.01, 2.0, 0.1, 1.0]).view(1, 1, hq, 1)
    base = torch.randn((1, 1, hq, 128), generator=gen)
    q = ((base + eps * torch.randn((steps, 1, hq, 128), generator=gen)) / torch.sqrt(1 + eps * eps)).to(torch.bfloat16)
    k = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.LaggedReuseDecodeStep(mode, 1, hq, hkv, 128, t + 64, top_fraction=0.02, protect_sink=4,
                                    protect_recent=8)
    prev = None
    for s in range(steps):
        n = t + s + 1
        out = step(q[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, wc, wf, prev, _ = R.lagged_reuse_decode_step(f32(q[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), kind,
                                                           param, dims, cand, 0.02, 4, 8, True, 128 ** -0.5, prev,
                                                           True)
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
