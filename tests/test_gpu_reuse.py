"""GPU parity of candidate reuse and exact rerank against the oracle and the
reference's own golden vectors: masks and final index sets bit-exact,
attention within 1e-2 relative / 2e-2 absolute."""

import numpy as np
import pytest
import torch

from kv_cache_amd import qabs_cuda_kernels as Q
from kv_cache_amd import reuse as RU
from oracle import ref_semantics as R
from tests.test_oracle_reuse import SCENARIOS, load_golden

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2
DT = {"float32": torch.float32, "bfloat16": torch.bfloat16}


def f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("name", SCENARIOS)
def test_pieces_match_reference_vectors(name):
    # The step composed from the C-ABI pieces in the scenario's dtype, on
    # GQA-expanded K as the reference's hook passes it; every step's masks
    # equal the reference's, the attention is within tolerance.
    g = load_golden(name)
    dt = DT[g["dtype"]]
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k_all = torch.from_numpy(np.repeat(g["k"], hq // hkv, axis=1)).to(dt).to(DEV)
    v_all = torch.from_numpy(np.repeat(g["v"], hq // hkv, axis=1)).to(dt).to(DEV)
    pc = pf = None
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        hist = n - 1
        q = torch.from_numpy(g["q"][s]).to(dt).to(DEV)
        k, v = k_all[:, :, :n], v_all[:, :, :n]
        partial = Q.partial_scores(q, k[:, :, :hist], g["dims"])
        req = R.budget_count(hist, g["cand"])
        ws = torch.empty(max(1, Q._lib.load().qkv_threshold_mask_workspace_bytes(hq, hist, req)) // 4 + 1,
                         dtype=torch.float32, device=DEV)
        cur = torch.empty((1, hq, hist), dtype=torch.bool, device=DEV)
        if g["selection"] == "topk":
            RU.threshold_mask(partial.view(hq, hist), hist, req, cur.view(torch.uint8).view(hq, hist), ws)
        else:   # the candidate selections of EV:3958-3989, thresholds carried between steps
            cols = RU.sample_columns(hist, g["sample_size"]) if g["selection"] == "sample_quantile" else None
            use_prev = g["selection"] == "previous_threshold" and s > 0
            sel = "previous_threshold" if use_prev else "sample_quantile" if cols is not None else "topk"
            n_s = cols.numel() if cols is not None else 0
            kk = R.budget_count(n_s, g["cand"]) if cols is not None else req
            ws = torch.empty(max(1, Q._lib.load().qkv_candidate_mask_workspace_bytes(
                hq, hist, RU.CANDIDATE_SELECTIONS[sel], kk, n_s)) // 4 + 1, dtype=torch.float32, device=DEV)
            if s == 0:
                thr = torch.zeros(hq, dtype=torch.float32, device=DEV)
            RU.candidate_mask(partial.view(hq, hist), hist, sel, kk, cur.view(torch.uint8).view(hq, hist), thr, ws,
                              cols.to(DEV) if cols is not None else None, n_s)
            assert np.array_equal(thr.cpu().numpy(), g["thresholds"][s].reshape(-1)), (name, s, "thresholds")
        assert np.array_equal(cur.cpu().numpy(), g["candidate"][s][..., :hist]), (name, s, "candidate")
        fi, fv, hf = Q.reuse_select(q, k, cur, pc if g["use_prev_candidate"] else None,
                                    pf if g["use_prev_final"] else None, g["sink"], g["recent"], g["top_fraction"],
                                    g["keep_self"], g["scaling"])
        if g["block"] is not None:   # the blk modes expand the selection to whole blocks (EV:4314-4316)
            fi, fv, _ = RU.expand_blocks(hf.view(torch.uint8).view(hq, hist), n, g["block"], g["sink"],
                                         g["recent"], g["top_fraction"], g["keep_self"])
            fi, fv = fi.view(1, hq, -1), fv.view(1, hq, -1)
        assert np.array_equal(hf.cpu().numpy(), g["final"][s][..., :hist]), (name, s, "final")
        out = Q.final_attention(q, k, v, fi, fv, g["scaling"])
        np.testing.assert_allclose(f32(out)[:, 0], g["out"][s], rtol=RTOL, atol=ATOL)
        # the next step reads them padded with False to its history (EV:1645-1662)
        pc, pf = (torch.cat([m, torch.zeros_like(m[..., :1])], dim=-1) for m in (cur, hf))


@pytest.mark.parametrize("name", ["s8c5_bf16", "s16c10_finalblk8_bf16"])
def test_step_matches_reference_vectors_bf16(name):
    # The GQA-native step (dim-major K, no head expansion) on the bf16
    # scenarios: the state it leaves equals the reference's at every step.
    g = load_golden(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k = torch.from_numpy(g["k"]).to(torch.bfloat16).to(DEV)
    v = torch.from_numpy(g["v"]).to(torch.bfloat16).to(DEV)
    step = RU.ReuseDecodeStep(g["mode"], 1, hq, hkv, 128, 1024, top_fraction=g["top_fraction"],
                              protect_sink=g["sink"], protect_recent=g["recent"], keep_self=g["keep_self"])
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(torch.bfloat16).to(DEV)
        out = step(q, k[:, :, :n], v[:, :, :n], g["scaling"])
        assert np.array_equal(step.candidate_mask().cpu().numpy(), g["candidate"][s][..., : n - 1]), s
        assert np.array_equal(step.final_mask().cpu().numpy(), g["final"][s][..., : n - 1]), s
        np.testing.assert_allclose(f32(out), g["out"][s], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("b,h,t,sink,recent,frac,keep_self", [
    (2, 4, 5000, 4, 16, 0.02, True),
    (1, 3, 777, 0, 0, 0.3, False),       # keep larger than the union: invalid -inf picks
    (1, 2, 2, 1, 1, 1.0, True),          # history 1
    (1, 2, 9000, 100, 100, 0.01, True),  # protected ranges overlap the selection
    (1, 2, 40961, 3, 3, 0.02, True),     # the longest row selected in one workgroup
    (1, 1, 45001, 0, 7, 0.05, False),    # longer rows: staged top-k
])
def test_reuse_select_matches_oracle(dtype, b, h, t, sink, recent, frac, keep_self):
    gen = torch.Generator().manual_seed(t + h)
    q = torch.randn((b, h, 128), generator=gen).to(dtype)
    k = torch.randn((b, h, t, 128), generator=gen).to(dtype)
    hist = t - 1
    masks = [torch.rand((b, h, hist), generator=gen) < p for p in (0.05, 0.04, 0.02)]
    fi, fv, hf = Q.reuse_select(q.to(DEV), k.to(DEV), masks[0].to(DEV), masks[1].to(DEV), masks[2].to(DEV), sink,
                                recent, frac, keep_self, 0.088)
    wi, wv, whf = R.reuse_select(f32(q), f32(k), masks[0].numpy(), masks[1].numpy(), masks[2].numpy(), sink, recent,
                                 frac, keep_self, 0.088)
    assert fi.shape == wi.shape
    assert np.array_equal(fi.cpu().numpy(), wi)        # same order: ascending selection, then the ranges
    assert np.array_equal(fv.cpu().numpy(), wv)
    assert np.array_equal(hf.cpu().numpy(), whf)


@pytest.mark.parametrize("t,dens,frac", [
    (8001, (0.4, 0.3, 0.1), 0.05),      # union ~60% of the row: beyond the compacted lists, the whole row is ranked
    (8001, (0.08, 0.0, 0.0), 0.05),     # union just above keep
    (30001, (0.06, 0.05, 0.02), 0.02),  # the bench's proportions
    (8001, (0.3, 0.1, 0.05), 0.05),     # union ~40%: the wider compacted form (2048-4096 keys at this width)
    (30001, (0.12, 0.08, 0.04), 0.02),  # union ~22%: the wider form at 32 keys per thread (4096-8192)
    (40001, (0.15, 0.05, 0.02), 0.02),  # union ~21%: the wider form at 40 keys per thread (5120-10240)
])
def test_reuse_select_union_sizes(t, dens, frac):
    gen = torch.Generator().manual_seed(t + int(100 * dens[0]))
    q = torch.randn((1, 4, 128), generator=gen).to(torch.bfloat16)
    k = torch.randn((1, 4, t, 128), generator=gen).to(torch.bfloat16)
    hist = t - 1
    masks = [torch.rand((1, 4, hist), generator=gen) < p for p in dens]
    fi, fv, hf = Q.reuse_select(q.to(DEV), k.to(DEV), *(m.to(DEV) for m in masks), 3, 5, frac, True, 0.088)
    wi, wv, whf = R.reuse_select(f32(q), f32(k), *(m.numpy() for m in masks), 3, 5, frac, True, 0.088)
    assert np.array_equal(fi.cpu().numpy(), wi)
    assert np.array_equal(fv.cpu().numpy(), wv)
    assert np.array_equal(hf.cpu().numpy(), whf)


def test_reuse_select_exact_ties():
    # K rows repeat every 37 tokens, so union scores tie exactly: the lower
    # token wins, whether the union is ranked compacted (up to 2048 keys, the
    # wider form up to 4096 at this width) or over the whole row
    gen = torch.Generator().manual_seed(12)
    q = torch.randn((1, 2, 128), generator=gen).to(torch.bfloat16)
    base = torch.randn((1, 2, 37, 128), generator=gen).to(torch.bfloat16)
    t = 5181
    k = base.repeat(1, 1, 141, 1)[:, :, :t].contiguous()
    hist = t - 1
    for dens in ((0.1, 0.05, 0.02), (0.5, 0.0, 0.0), (0.9, 0.0, 0.0)):
        masks = [torch.rand((1, 2, hist), generator=gen) < p for p in dens]
        fi, fv, hf = Q.reuse_select(q.to(DEV), k.to(DEV), *(m.to(DEV) for m in masks), 0, 0, 0.03, False, 0.088)
        wi, wv, whf = R.reuse_select(f32(q), f32(k), *(m.numpy() for m in masks), 0, 0, 0.03, False, 0.088)
        assert np.array_equal(fi.cpu().numpy(), wi) and np.array_equal(fv.cpu().numpy(), wv)
        assert np.array_equal(hf.cpu().numpy(), whf)


@pytest.mark.parametrize("rows,n,k,ld", [(3, 1000, 50, 1000), (2, 16384, 1, 16400), (2, 16385, 819, 16385),
                                         (1, 40960, 2048, 40960), (2, 45000, 2250, 45056), (4, 7, 7, 9)])
def test_threshold_mask_matches_oracle(rows, n, k, ld):
    gen = torch.Generator().manual_seed(n + k)
    vals = torch.randint(-30, 30, (rows, ld), generator=gen).float()      # heavy ties at the threshold
    vals[0] = torch.randn(ld, generator=gen)
    mask = torch.full((rows, ld + 5), 7, dtype=torch.uint8)
    lib = Q._lib.load()
    ws = torch.empty(lib.qkv_threshold_mask_workspace_bytes(rows, n, k) // 4 + 1, dtype=torch.float32, device=DEV)
    md = mask.to(DEV)
    RU.threshold_mask(vals.to(DEV), n, k, md, ws)
    got = md.cpu().numpy()
    assert np.array_equal(got[:, :n].astype(bool), R.threshold_mask(vals[:, :n].numpy(), k))
    assert set(np.unique(got[:, :n]).tolist()) <= {0, 1} and (got[:, n:] == 7).all()   # nothing past n


@pytest.mark.parametrize("rows,n,n_s,frac,ld", [(3, 1000, 256, 0.05, 1000), (2, 32790, 256, 0.05, 32800),
                                               (2, 5000, 255, 0.5, 5003), (2, 300, 64, 1.0, 300),
                                               (4, 9000, 1, 0.05, 9000), (2, 20000, 257, 0.05, 20000),
                                               (2, 50000, 4000, 0.05, 50000)])
def test_sample_quantile_mask_matches_oracle(rows, n, n_s, frac, ld):
    # the sample's k-th largest and the mask over the row: one launch up to
    # 256 samples, the gather + selection + compare launches above; integer
    # scores put many ties at the threshold, one row has signed zeros there
    gen = torch.Generator().manual_seed(n + n_s)
    vals = torch.randint(-20, 20, (rows, ld), generator=gen).float()
    vals[0] = torch.randn(ld, generator=gen)
    vals[-1, ::3] = -0.0
    vals[-1, 1::3] = 0.0
    cols = RU.sample_columns(n, n_s)
    k = R.budget_count(cols.numel(), frac)
    want_m, want_t, _ = R.candidate_mask(vals[:, :n].numpy(), R.budget_count(n, frac), frac, "sample_quantile",
                                         sample_size=n_s)
    lib = Q._lib.load()
    ws = torch.empty(max(1, lib.qkv_candidate_mask_workspace_bytes(rows, n, 1, k, cols.numel())) // 4 + 1,
                     dtype=torch.float32, device=DEV)
    mask = torch.full((rows, ld + 3), 7, dtype=torch.uint8, device=DEV)
    thr = torch.full((rows,), 5.0, device=DEV)
    for c in (cols.to(DEV), cols):   # device columns as given, host columns checked and copied
        RU.candidate_mask(vals.to(DEV), n, "sample_quantile", k, mask, thr, ws, c, cols.numel())
        got = mask.cpu().numpy()
        assert np.array_equal(got[:, :n].astype(bool), want_m)
        assert set(np.unique(got[:, :n]).tolist()) <= {0, 1} and (got[:, n:] == 7).all()
        assert np.array_equal(thr.cpu().numpy(), want_t.reshape(-1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d,hist,dims", [(128, 32790, 8), (128, 5, 8), (128, 4103, 16), (64, 1001, 8),
                                         (200, 333, 12)])
def test_reuse_partial_scores_ties_and_ragged_tails(dtype, d, hist, dims):
    # GQA-native partial scores from the dim-major copy: queries with many
    # equal magnitudes (the lower dim first), histories whose last 8-token
    # group is short, head sizes under 128 (padded ranking keys) and above
    # it (the general ranking)
    gen = torch.Generator().manual_seed(d * 7 + hist + dims)
    b, hq, hkv = 2, 4, 2
    q = torch.randint(-3, 4, (b, hq, d), generator=gen).float() * 0.5
    q[0, 1] = torch.randn(d, generator=gen)
    k = torch.randn((b, hkv, hist, d), generator=gen).to(dtype)
    kdm = torch.zeros((b, hkv, d, hist + 40), dtype=dtype, device=DEV)
    RU.dim_major_append(k.to(DEV), kdm, 0, hist)
    got = RU.reuse_partial_scores(q.to(dtype).to(DEV), kdm, hist, dims).cpu().numpy().reshape(b, hq, hist)
    want = R.partial_scores(f32(q.to(dtype)), np.repeat(f32(k), hq // hkv, axis=1), dims)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype,b,hist,dims,gated,bits", [
    (torch.bfloat16, 4, 32790, 8, False, False),    # 128 rows: the one-launch kernel, five 8192-token chunks
    (torch.float16, 4, 5001, 16, False, False),     # one chunk, a short last 8-token group
    (torch.float32, 8, 20003, 8, False, False),     # 256 rows, three chunks
    (torch.bfloat16, 4, 9000, 8, True, False),      # lagged steps: rows whose flag is clear stay untouched
    (torch.bfloat16, 1, 9000, 8, False, False),     # 32 rows: the two-launch form
    (torch.bfloat16, 4, 32790, 8, False, True),     # bitsets: one launch
    (torch.float16, 1, 5001, 16, False, True),      # bitsets: two launches, a partial last word
    (torch.bfloat16, 1, 45001, 8, False, True),     # bitsets past the one-workgroup selection
])
def test_reuse_candidates_match_oracle(dtype, b, hist, dims, gated, bits):
    # partial scores, the k-th largest and the mask in one call: scores bit-exact
    # to the oracle, mask = score >= the k-th largest (ties all kept), threshold
    from kv_cache_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(hist + b + dims)
    hq, hkv, d = 32, 8, 128
    rows = b * hq
    q = torch.randn((b, hq, d), generator=gen).to(dtype)
    k = torch.randn((b, hkv, hist, d), generator=gen)
    k[0, 0, 7] = k[0, 0, 3]   # equal scores at the threshold's neighbourhood are kept together
    k = k.to(dtype)
    kdm = torch.zeros((b, hkv, d, hist + 24), dtype=dtype, device=DEV)
    RU.dim_major_append(k.to(DEV), kdm, 0, hist)
    kk = -(-hist * 5 // 100)
    part = torch.full((rows, hist + 9), 7.0, device=DEV)
    mask = torch.full((rows, hist + 9), 9, dtype=torch.uint8, device=DEV)
    words = torch.full((rows, -(-hist // 64) + 3), -1, dtype=torch.int64, device=DEV)
    thr = torch.zeros(rows, device=DEV)
    if gated:
        ws = torch.empty((lib.qkv_threshold_mask_workspace_bytes(rows, hist, kk) + 3) // 4, device=DEV)
    else:   # zero-filled: the selection state starts at zero
        ws = torch.zeros((lib.qkv_reuse_candidates_workspace_bytes(rows, hist, kk) + 3) // 4, device=DEV)
    flags = (torch.arange(rows) % 3 == 0).to(torch.uint8).to(DEV)
    qd = q.to(DEV)
    if gated:
        _lib.check(lib.qkv_reuse_lag_candidates(
            qd.data_ptr(), kdm.data_ptr(), _lib.strides(*kdm.stride()), _lib.DTYPE_CODES[dtype], b, hq, hkv, hist, d,
            dims, kk, flags.data_ptr(), 2, part.data_ptr(), part.stride(0), mask.data_ptr(), mask.stride(0),
            ws.data_ptr(), ws.numel() * 4, _lib.stream_of(qd)))
    else:
        _lib.check(lib.qkv_reuse_candidates(
            qd.data_ptr(), kdm.data_ptr(), _lib.strides(*kdm.stride()), _lib.DTYPE_CODES[dtype], b, hq, hkv, hist, d,
            dims, kk, part.data_ptr(), part.stride(0), None if bits else mask.data_ptr(), mask.stride(0),
            words.data_ptr() if bits else None, words.stride(0), thr.data_ptr(), ws.data_ptr(), ws.numel() * 4,
            _lib.stream_of(qd)))
    if bits:   # the words of [0, ceil(hist / 64)) hold the mask, bits past the history clear
        n_w = -(-hist // 64)
        exp = RU.expand_bits(words[:, :n_w], n_w * 64).cpu().numpy()
        mask[:, :hist] = torch.from_numpy(exp[:, :hist].astype(np.uint8)).to(DEV)
        assert not exp[:, hist:].any()
        assert (words[:, n_w:] == -1).all()
    want = R.partial_scores(f32(q), np.repeat(f32(k), hq // hkv, axis=1), dims).reshape(rows, hist)
    kth = -np.sort(-want, axis=1)[:, kk - 1 : kk]
    got_p, got_m = part.cpu().numpy(), mask.cpu().numpy()
    on = flags.cpu().numpy().astype(bool) if gated else np.ones(rows, bool)
    assert np.array_equal(got_p[on, :hist], want[on])
    assert np.array_equal(got_m[on, :hist].astype(bool), (want >= kth)[on])
    assert (got_p[:, hist:] == 7.0).all() and (got_m[:, hist:] == 9).all()   # nothing past the history
    if gated:
        assert (got_p[~on] == 7.0).all() and (got_m[~on] == 9).all()
    else:
        assert np.array_equal(thr.cpu().numpy(), kth[:, 0])
        _assert_cand_state_zero(ws, rows)


def _assert_cand_state_zero(ws, rows):
    # the parts of qkv_reuse_candidates' workspace that are zero between
    # calls: the 4096 first-digit bins per row at its start, then (after 48
    # state words per row: 40 list counts, the ticket, padding) each row's ticket
    assert not ws[: rows * 4096].any()
    state = ws[rows * 4096 : rows * 4096 + rows * 48].view(torch.int32).view(rows, 48)
    assert not state[:, 40].any()


def _cand_case(b, hist, dims, pattern, seed):
    # (q, K) whose partial scores follow `pattern`: K[t] = c_t * (a fixed
    # vector), so the scores are c_t times the row's sum over its dims
    gen = torch.Generator().manual_seed(seed)
    hq, hkv, d = 32, 8, 128
    q = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16)
    if pattern == "normal":
        k = torch.randn((b, hkv, hist, d), generator=gen)
    else:
        if pattern == "equal":          # every score of a row equal: the whole row in one bin
            c = torch.ones(hist)
        elif pattern == "narrow":       # 256 values in [1, 2): about an eighth of a row per bin
            c = 1.0 + torch.randint(0, 256, (hist,), generator=gen).float() / 256.0
        elif pattern == "coarse":       # 16 values in [1, 1.125): one bin, heavy ties
            c = 1.0 + torch.randint(0, 16, (hist,), generator=gen).float() / 128.0
        else:
            raise ValueError(pattern)
        k = c.view(1, 1, hist, 1).expand(b, hkv, hist, d).clone()
    return q, k.to(torch.bfloat16)


def _run_candidates(lib, q, kdm, hist, dims, kk, words, thr, ws, part):
    from kv_cache_amd import _lib

    b, hq, d = q.shape
    _lib.check(lib.qkv_reuse_candidates(
        q.data_ptr(), kdm.data_ptr(), _lib.strides(*kdm.stride()), _lib.DTYPE_CODES[q.dtype], b, hq, kdm.shape[1],
        hist, d, dims, kk, part.data_ptr(), part.stride(0), None, 0, words.data_ptr(), words.stride(0),
        thr.data_ptr(), ws.data_ptr(), ws.numel() * 4, _lib.stream_of(q)))


def _check_candidates(q, k, hist, dims, kk, words, thr):
    b, hq, _ = q.shape
    rows = b * hq
    want = R.partial_scores(f32(q), np.repeat(f32(k), hq // k.shape[1], axis=1), dims).reshape(rows, hist)
    kth = -np.sort(-want, axis=1)[:, kk - 1 : kk]
    n_w = -(-hist // 64)
    got = RU.expand_bits(words[:, :n_w], n_w * 64).cpu().numpy()
    assert not got[:, hist:].any()
    assert np.array_equal(got[:, :hist], want >= kth)
    assert np.array_equal(thr.cpu().numpy(), kth[:, 0])


@pytest.mark.parametrize("b,hist,pattern,frac", [
    (1, 20000, "equal", 5),      # the boundary bin holds the whole row: the list selected from memory
    (1, 20000, "narrow", 5),     # a list of a few thousand: eight scores per thread
    (1, 30011, "coarse", 5),     # one bin and 16 distinct scores: ties at the threshold
    (2, 40960, "normal", 2),     # 64 rows at the longest one-workgroup row
    (1, 1000, "normal", 50),     # one slice per row
    (3, 777, "narrow", 100),     # k = the whole row
])
def test_reuse_candidates_slices(b, hist, pattern, frac):
    # the partial scores' first-digit counts and the selection across several
    # workgroups per row: the bitset = score >= the k-th largest, the threshold
    # exact, the workspace's state zero afterwards
    from kv_cache_amd import _lib

    lib = _lib.load()
    dims = 8
    q, k = _cand_case(b, hist, dims, pattern, hist + b)
    rows = b * 32
    kdm = torch.zeros((b, 8, 128, hist + 24), dtype=torch.bfloat16, device=DEV)
    RU.dim_major_append(k.to(DEV), kdm, 0, hist)
    kk = min(hist, -(-hist * frac // 100))
    part = torch.zeros((rows, hist + 9), device=DEV)
    words = torch.full((rows, -(-hist // 64) + 3), -1, dtype=torch.int64, device=DEV)
    thr = torch.zeros(rows, device=DEV)
    ws = torch.zeros((lib.qkv_reuse_candidates_workspace_bytes(rows, hist, kk) + 3) // 4, device=DEV)
    qd = q.to(DEV)
    _run_candidates(lib, qd, kdm, hist, dims, kk, words, thr, ws, part)
    _check_candidates(q, k, hist, dims, kk, words, thr)
    assert (words[:, -(-hist // 64):] == -1).all()
    _assert_cand_state_zero(ws, rows)


def test_reuse_candidates_workspace_reused():
    # one zero-filled workspace through calls of growing and shrinking history
    # (and a byte-mask call between them): every call exact, the state zero
    # after each
    from kv_cache_amd import _lib

    lib = _lib.load()
    b, cap, dims = 1, 33000, 8
    rows = b * 32
    q, k = _cand_case(b, cap, dims, "normal", 11)
    kdm = torch.zeros((b, 8, 128, cap + 8), dtype=torch.bfloat16, device=DEV)
    RU.dim_major_append(k.to(DEV), kdm, 0, cap)
    ws = torch.zeros((lib.qkv_reuse_candidates_workspace_bytes(rows, cap, cap) + 3) // 4, device=DEV)
    part = torch.zeros((rows, cap), device=DEV)
    words = torch.zeros((rows, -(-cap // 64)), dtype=torch.int64, device=DEV)
    thr = torch.zeros(rows, device=DEV)
    qd = q.to(DEV)
    for hist in (32768, 32769, 4097, 33000, 100):
        kk = -(-hist * 2 // 100)
        _run_candidates(lib, qd, kdm, hist, dims, kk, words, thr, ws, part)
        _check_candidates(q, k[:, :, :hist], hist, dims, kk, words, thr)
        _assert_cand_state_zero(ws, rows)
        if hist == 4097:   # the byte mask takes the other path through the same workspace
            mask = torch.zeros((rows, hist), dtype=torch.uint8, device=DEV)
            _lib.check(lib.qkv_reuse_candidates(
                qd.data_ptr(), kdm.data_ptr(), _lib.strides(*kdm.stride()), _lib.DTYPE_CODES[qd.dtype], b, 32, 8,
                hist, 128, dims, kk, part.data_ptr(), part.stride(0), mask.data_ptr(), mask.stride(0), None, 0,
                None, ws.data_ptr(), ws.numel() * 4, _lib.stream_of(qd)))
            assert np.array_equal(mask.cpu().numpy().astype(bool), RU.expand_bits(words, cap)[:, :hist].cpu().numpy())


@pytest.mark.parametrize("hist,sink,recent,frac,prev,dens,ties,dtype", [
    (3000, 4, 8, 0.02, True, 0.03, False, torch.bfloat16),
    (1001, 0, 0, 0.05, False, 0.03, False, torch.bfloat16),
    (45000, 10, 10, 0.02, True, 0.03, False, torch.bfloat16),   # past the one-workgroup rows
    (32768, 10, 10, 0.02, True, 0.03, False, torch.float16),    # the bench's proportions, fp16
    (40960, 10, 10, 0.02, True, 0.03, False, torch.bfloat16),   # the longest one-workgroup row
    (8000, 3, 5, 0.05, True, 0.25, False, torch.bfloat16),      # a union past the compacted keys: the whole row
    (777, 0, 0, 0.3, True, 0.03, False, torch.bfloat16),        # keep larger than the union: -inf picks
    (3700, 0, 0, 0.03, True, 0.1, True, torch.bfloat16),        # K rows repeat every 37 tokens: exact ties
])
def test_reuse_select_bits_equals_bytes(hist, sink, recent, frac, prev, dens, ties, dtype):
    # the same masks as bytes and as bitsets (the bitset selection forms and
    # scores the union in its own workgroup): the same final list and final mask
    from kv_cache_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(hist)
    b, hq, hkv, d = 1, 8, 2, 128
    rows, t = b * hq, hist + 1
    q = torch.randn((b, hq, d), generator=gen).to(dtype).to(DEV)
    if ties:
        k = torch.randn((b, hkv, 37, d), generator=gen).repeat(1, 1, -(-t // 37), 1)[:, :, :t]
        k = k.contiguous().to(dtype).to(DEV)
    else:
        k = torch.randn((b, hkv, t, d), generator=gen).to(dtype).to(DEV)
    masks = [(torch.rand((rows, hist), generator=gen) < dens).to(DEV) for _ in range(3)]
    n_w = -(-hist // 64)

    def to_words(m):
        pad = torch.zeros((rows, n_w * 64), dtype=torch.bool, device=DEV)
        pad[:, :hist] = m
        by = (pad.view(rows, -1, 8).to(torch.uint8) << torch.arange(8, dtype=torch.uint8, device=DEV)).sum(-1)
        return by.to(torch.uint8).contiguous().view(torch.int64)

    n_out = int(lib.qkv_reuse_final_count(hist, sink, recent, frac, 1))
    ws = torch.empty((lib.qkv_reuse_select_workspace_bytes(rows, hist, frac) + 3) // 4, device=DEV)
    outs = []
    for bits in (False, True):
        ms = [to_words(m) if bits else m.to(torch.uint8).contiguous() for m in masks]
        fin = torch.zeros_like(ms[2]) if bits else torch.zeros((rows, hist), dtype=torch.uint8, device=DEV)
        fi = torch.empty((rows, n_out), dtype=torch.int64, device=DEV)
        fv = torch.empty((rows, n_out), dtype=torch.uint8, device=DEV)
        ids = torch.empty((rows, n_out), dtype=torch.int32, device=DEV)
        select = lib.qkv_reuse_select_bits if bits else lib.qkv_reuse_select
        extra = (None, None, None) if bits else ()
        _lib.check(select(q.data_ptr(), k.data_ptr(), _lib.strides(*k.stride()), _lib.DTYPE_CODES[dtype], b, hq,
                          hkv, t, d,
                          ms[0].data_ptr(), ms[1].data_ptr() if prev else None, ms[2].data_ptr(), ms[0].stride(0),
                          sink, recent, frac, 1, 0.088, ws.data_ptr(), ws.numel() * 4, fi.data_ptr(), fv.data_ptr(),
                          ids.data_ptr(), n_out, fin.data_ptr(), fin.stride(0), *extra, _lib.stream_of(q)))
        hf = RU.expand_bits(fin, hist) if bits else fin.bool()
        outs.append((fi, fv, ids, hf))
    for a, w in zip(*outs):
        assert torch.equal(a, w)


@pytest.mark.parametrize("dtype,hist,frac,fused", [(torch.bfloat16, 3000, 0.02, True), (torch.float16, 9000, 0.05, True),
                                                   (torch.bfloat16, 40000, 0.11, False)])
def test_step_attention_in_the_final_selection(dtype, hist, frac, fused):
    # the final selection's workgroups attend over the list they wrote (one launch);
    # past 4096 list entries the separate token attention runs -- either way the
    # output equals the token attention over the step's own list
    from kv_cache_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(hist)
    hq, hkv = 8, 2
    k = torch.randn((1, hkv, hist + 1, 128), generator=gen).to(dtype).to(DEV)
    v = torch.randn((1, hkv, hist + 1, 128), generator=gen).to(dtype).to(DEV)
    q = torch.randn((1, hq, 128), generator=gen).to(dtype).to(DEV)
    step = RU.ReuseDecodeStep("qabs8cand5reuse", 1, hq, hkv, 128, hist + 8, top_fraction=frac, protect_sink=4,
                              protect_recent=8, dtype=dtype, fused_attention=True)
    out = step(q, k, v, 0.088).clone()
    n_out = step.n_out
    assert (n_out <= 4096) == fused
    ids = step.attn_ids[: hq * n_out].view(hq, n_out)
    want = RU.token_attention(q, k, v, ids, 0.088, workspace=step.attn_ws)
    torch.testing.assert_close(out.float(), want.float(), rtol=2e-2, atol=2e-3)
    fi, fv = (x.cpu().numpy() for x in step.final_indices())
    o = R.final_attention(f32(q), np.repeat(f32(k), hq // hkv, axis=1), np.repeat(f32(v), hq // hkv, axis=1),
                          fi, fv, 0.088)
    np.testing.assert_allclose(f32(out), o[:, 0], rtol=RTOL, atol=ATOL)


def test_reuse_select_ties_and_missing_masks():
    # Duplicate keys give equal scores: the lower index wins; previous masks absent.
    gen = torch.Generator().manual_seed(1)
    q = torch.randn((1, 2, 128), generator=gen).to(torch.bfloat16)
    base = torch.randn((1, 2, 40, 128), generator=gen).to(torch.bfloat16)
    k = base.repeat(1, 1, 50, 1)[:, :, :1999]          # every row repeats 50 times
    cur = torch.rand((1, 2, 1998), generator=gen) < 0.3
    fi, fv, hf = Q.reuse_select(q.to(DEV), k.to(DEV), cur.to(DEV), None, None, 0, 0, 0.05, True, 0.1)
    wi, wv, whf = R.reuse_select(f32(q), f32(k), cur.numpy(), None, None, 0, 0, 0.05, True, 0.1)
    assert np.array_equal(fi.cpu().numpy(), wi) and np.array_equal(fv.cpu().numpy(), wv)
    assert np.array_equal(hf.cpu().numpy(), whf)


@pytest.mark.parametrize("hq,hkv,t,steps,mode", [
    (8, 2, 3000, 4, "qabs8cand5reuse"),
    (32, 8, 9000, 3, "qabs16cand10reusefinal"),
    (4, 4, 1500, 3, "qabs8cand3reuse2set"),
    (8, 2, 3000, 4, "qabs8cand5reuseblk16"),
    (32, 8, 9000, 3, "qabs16cand10reusefinalblk32"),
    (4, 4, 1500, 3, "qabs8cand3reuse2setblk64"),
    (4, 2, 1000, 3, "qabs8cand5reuseblk7"),
    (4, 2, 50000, 2, "qabs8cand2reuseblk64"),     # staged selection, 13 expansion tiles
])
def test_step_matches_oracle(hq, hkv, t, steps, mode):
    gen = torch.Generator().manual_seed(hq * t)
    s_dims, cand, use_pc, use_pf, block = RU.parse_reuse_mode(mode)
    k = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    qs = torch.randn((steps, 1, hq, 128), generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.ReuseDecodeStep(mode, 1, hq, hkv, 128, t + steps + 64, top_fraction=0.02, protect_sink=4,
                              protect_recent=8)
    step.prefill(kd[:, :, :t - 1])
    pc = pf = None
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        want, wc, wf = R.reuse_decode_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), s_dims, cand, 0.02, 4, 8,
                                           True, 128 ** -0.5, pc if use_pc else None, pf if use_pf else None, block)
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        # the final list: the final mask plus the current token, each once
        fi, fv = (x.cpu().numpy() for x in step.final_indices())
        for r in range(hq):
            got = fi[0, r][fv[0, r]]
            assert len(got) == len(set(got.tolist())), (s, r)
            assert set(got.tolist()) == set(np.flatnonzero(wf[0, r]).tolist()) | {n - 1}, (s, r)
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
        pc, pf = wc, wf


@pytest.mark.parametrize("hq,hkv,t,steps,mode,selection,sample", [
    (8, 2, 3000, 4, "qabs8cand5reuse", "sample_quantile", 256),
    (4, 2, 1000, 3, "qabs16cand10reusefinal", "sample_quantile", 2000),   # the sample covers the row
    (4, 2, 50000, 2, "qabs8cand5reuse", "sample_quantile", 45000),        # staged threshold of the sample
    (8, 2, 3000, 4, "qabs8cand5reuse", "previous_threshold", 256),
    (4, 2, 50000, 3, "qabs8cand2reuseblk16", "previous_threshold", 256),  # staged first threshold
])
def test_step_selections_match_oracle(hq, hkv, t, steps, mode, selection, sample):
    gen = torch.Generator().manual_seed(hq * t + len(selection))
    s_dims, cand, use_pc, use_pf, block = RU.parse_reuse_mode(mode)
    k = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((1, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    qs = torch.randn((steps, 1, hq, 128), generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.ReuseDecodeStep(mode, 1, hq, hkv, 128, t + steps + 64, top_fraction=0.02, protect_sink=4,
                              protect_recent=8, candidate_selection=selection, threshold_sample_size=sample)
    pc = pf = thr = None
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 128 ** -0.5)
        got = []
        want, wc, wf = R.reuse_decode_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), s_dims, cand, 0.02, 4, 8,
                                           True, 128 ** -0.5, pc if use_pc else None, pf if use_pf else None, block,
                                           selection=selection, sample_size=sample, previous_thresholds=thr,
                                           thresholds_out=got)
        thr = got[0]
        assert np.array_equal(step.thresholds.cpu().numpy(), thr.reshape(-1)), s
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
        pc, pf = wc, wf


def test_step_sample_quantile_graph_replays():
    # the sample_quantile step reads its sampled columns from a device table,
    # so it can be captured: every replay, with a new query copied in and the
    # outputs cleared between replays, matches the eager launch bit for bit
    gen = torch.Generator().manual_seed(17)
    t = 3000
    k = torch.randn((1, 2, t + 3, 128), generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn((1, 2, t + 3, 128), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((1, 8, 128), generator=gen).to(torch.bfloat16).to(DEV)
    step = RU.ReuseDecodeStep("qabs8cand5reuse", 1, 8, 2, 128, t + 64, top_fraction=0.02, protect_sink=4,
                              protect_recent=8, candidate_selection="sample_quantile", threshold_sample_size=256)
    for n in (t, t + 1, t + 2):
        step(q, k[:, :, :n], v[:, :, :n], 128 ** -0.5)
    cur, prev = step.cand[1 - step.flip], step.cand[step.flip]
    kk, vv = k[:, :, : t + 2], v[:, :, : t + 2]

    def launch():
        step.launch(q, kk, vv, 128 ** -0.5, cur, prev, None)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for rep in range(4):
        q.copy_(torch.randn((1, 8, 128), generator=gen).to(torch.bfloat16))
        launch()
        want = [x.clone() for x in (cur, step.fin, step.thresholds, step.out)]
        for x in (cur, step.fin, step.thresholds, step.out):
            x.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for w, x in zip(want, (cur, step.fin, step.thresholds, step.out)):
            assert torch.equal(w, x), rep
    assert int(cur.count_nonzero()) > 0


@pytest.mark.parametrize("mode,selection", [("qabs8cand5reuseblk8", "previous_threshold"),
                                            ("qabs16cand10reusefinal", "sample_quantile"),
                                            ("qabs8cand5reuse2setblk32", "topk")])
def test_step_batches_match_oracle(mode, selection):
    # two sequences: rows b * Hq + h read their own K/V, dim-major copy and masks
    gen = torch.Generator().manual_seed(len(mode) * 31 + len(selection))
    b, hq, hkv, t, steps = 2, 4, 2, 700, 3
    s_dims, cand, use_pc, use_pf, block = RU.parse_reuse_mode(mode)
    k = torch.randn((b, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((b, hkv, t + steps, 128), generator=gen).to(torch.bfloat16)
    qs = torch.randn((steps, b, hq, 128), generator=gen).to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    step = RU.ReuseDecodeStep(mode, b, hq, hkv, 128, t + steps + 8, top_fraction=0.03, protect_sink=2,
                              protect_recent=5, candidate_selection=selection, threshold_sample_size=64)
    pc = pf = thr = None
    for s in range(steps):
        n = t + s + 1
        out = step(qs[s].to(DEV), kd[:, :, :n], vd[:, :, :n], 0.09)
        got = []
        want, wc, wf = R.reuse_decode_step(f32(qs[s]), f32(k[:, :, :n]), f32(v[:, :, :n]), s_dims, cand, 0.03, 2, 5,
                                           True, 0.09, pc if use_pc else None, pf if use_pf else None, block,
                                           selection=selection, sample_size=64, previous_thresholds=thr,
                                           thresholds_out=got)
        thr = got[0]
        assert np.array_equal(step.candidate_mask().cpu().numpy(), wc), s
        assert np.array_equal(step.final_mask().cpu().numpy(), wf), s
        np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)
        pc, pf = wc, wf


@pytest.mark.parametrize("rows,history,block,sink,recent,keep_self,density", [
    (3, 1000, 16, 4, 8, True, 0.01),
    (2, 9000, 64, 0, 0, False, 0.002),      # three tiles of 4096
    (4, 777, 7, 3, 5, True, 0.02),          # blocks that do not divide the tile or the history
    (2, 300, 4096, 2, 2, True, 0.01),       # one block wider than the history
    (2, 5000, 1, 10, 10, True, 0.05),       # no expansion: the list is the mask
    (3, 40, 8, 50, 0, True, 0.2),           # the sink covers the history
    (2, 50, 8, 0, 60, False, 0.2),          # the recent range covers the history
    (1, 1, 16, 0, 0, True, 1.0),
    (2, 5000, 32, 5, 5, True, 0.0),         # only the protected ranges
])
def test_expand_blocks_matches_oracle(rows, history, block, sink, recent, keep_self, density):
    gen = torch.Generator().manual_seed(history + block)
    # a final mask as qkv_reuse_select leaves it: selections plus the protected ranges
    mask = torch.rand((rows, history), generator=gen) < density
    mask[:, :min(sink, history)] = True
    mask[:, max(0, history - recent):] = True
    keep = int(mask.sum(dim=1).max())
    top_fraction = keep / history
    buf = torch.zeros((rows, history + 37), dtype=torch.uint8)   # padded row stride
    buf[:, :history] = mask.to(torch.uint8)
    dbuf = buf.to(DEV)
    idx, valid, ids = RU.expand_blocks(dbuf, history + 1, block, sink, recent, top_fraction, keep_self)
    want = R.expand_to_blocks(mask.numpy(), block)
    assert np.array_equal(dbuf[:, :history].cpu().numpy().astype(bool), want)
    assert int(torch.count_nonzero(dbuf[:, history:])) == 0
    sel, sv = R.indices_from_keep_mask(want)
    wi, wv = R.final_indices_np(sel, sv, history, history + 1, sink, recent, keep_self)
    idx, valid, ids = idx.cpu().numpy(), valid.cpu().numpy(), ids.cpu().numpy()
    assert np.array_equal(np.where(valid, idx, -1), ids)
    for r in range(rows):
        got = idx[r][valid[r]]
        assert sorted(got.tolist()) == sorted(wi[r][wv[r]].tolist()), r
        sink_end = min(sink, history)
        rec_begin = max(history - recent, sink_end)
        body = idx.shape[1] - sink_end - (history - rec_begin if recent > 0 else 0) - int(keep_self)
        assert np.all(np.diff(idx[r, :body][valid[r, :body]]) > 0), r      # ascending body


@pytest.mark.parametrize("hist,sink,recent,frac,prev,dens,block,keep_self,dtype", [
    (3000, 4, 8, 0.02, True, 0.03, 16, True, torch.bfloat16),
    (32768, 10, 10, 0.02, True, 0.03, 16, True, torch.bfloat16),   # the bench's blk16 proportions
    (40960, 10, 10, 0.02, True, 0.03, 100, True, torch.bfloat16),  # the longest row; blocks across words
    (5000, 0, 0, 0.05, False, 0.1, 1, False, torch.float16),       # blocks of one position: no expansion
    (9000, 3, 5, 0.02, True, 0.03, 4096, True, torch.bfloat16),    # the largest block
    (777, 0, 0, 0.3, True, 0.03, 64, True, torch.bfloat16),        # keep above the union
    (10000, 20, 30, 0.05, True, 0.25, 8, True, torch.bfloat16),    # a union past the compacted forms
    (12345, 10, 10, 0.02, True, 0.03, 24, False, torch.bfloat16),
])
def test_reuse_select_bits_blocks_equals_bytes(hist, sink, recent, frac, prev, dens, block, keep_self, dtype):
    # the selection and its block expansion in one launch on bitsets against
    # qkv_reuse_select + qkv_reuse_expand_blocks on the same masks as bytes:
    # the same expanded list, validity, attention ids and expanded final mask
    from kv_cache_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(hist + block)
    b, hq, hkv, d = 1, 8, 2, 128
    rows, t = b * hq, hist + 1
    q = torch.randn((b, hq, d), generator=gen).to(dtype).to(DEV)
    k = torch.randn((b, hkv, t, d), generator=gen).to(dtype).to(DEV)
    masks = [(torch.rand((rows, hist), generator=gen) < dens).to(DEV) for _ in range(3)]
    n_w = -(-hist // 64)

    def to_words(m):
        pad = torch.zeros((rows, n_w * 64), dtype=torch.bool, device=DEV)
        pad[:, :hist] = m
        by = (pad.view(rows, -1, 8).to(torch.uint8) << torch.arange(8, dtype=torch.uint8, device=DEV)).sum(-1)
        return by.to(torch.uint8).contiguous().view(torch.int64)

    n_sel = int(lib.qkv_reuse_final_count(hist, sink, recent, frac, int(keep_self)))
    n_out = int(lib.qkv_reuse_block_final_count(hist, block, sink, recent, frac, int(keep_self)))
    ws = torch.empty((lib.qkv_reuse_select_workspace_bytes(rows, hist, frac) + 3) // 4, device=DEV)
    outs = []
    for bits in (False, True):
        ms = [to_words(m) if bits else m.to(torch.uint8).contiguous() for m in masks]
        fin = torch.zeros_like(ms[2]) if bits else torch.zeros((rows, hist), dtype=torch.uint8, device=DEV)
        fi = torch.full((rows, n_out), 7, dtype=torch.int64, device=DEV)
        fv = torch.full((rows, n_out), 7, dtype=torch.uint8, device=DEV)
        ids = torch.full((rows, n_out), 7, dtype=torch.int32, device=DEV)
        head = (q.data_ptr(), k.data_ptr(), _lib.strides(*k.stride()), _lib.DTYPE_CODES[dtype], b, hq, hkv, t, d,
                ms[0].data_ptr(), ms[1].data_ptr() if prev else None, ms[2].data_ptr(), ms[0].stride(0), sink,
                recent, frac, int(keep_self), 0.088)
        if bits:
            _lib.check(lib.qkv_reuse_select_bits_blocks(
                *head, block, ws.data_ptr(), ws.numel() * 4, fi.data_ptr(), fv.data_ptr(), ids.data_ptr(), n_out,
                fin.data_ptr(), fin.stride(0), _lib.stream_of(q)))
        else:
            _lib.check(lib.qkv_reuse_select(*head, ws.data_ptr(), ws.numel() * 4, fi.data_ptr(), fv.data_ptr(),
                                            ids.data_ptr(), n_sel, fin.data_ptr(), fin.stride(0), _lib.stream_of(q)))
            _lib.check(lib.qkv_reuse_expand_blocks(fin.data_ptr(), fin.stride(0), rows, t, block, sink, recent, frac,
                                                   int(keep_self), fi.data_ptr(), fv.data_ptr(), ids.data_ptr(),
                                                   n_out, _lib.stream_of(q)))
        hf = RU.expand_bits(fin, hist) if bits else fin.bool()
        outs.append((fi, fv, ids, hf))
    for a, w in zip(*outs):
        assert torch.equal(a, w)
    if bits:   # nothing set past the history in the last word
        tail = RU.expand_bits(fin, n_w * 64)[:, hist:]
        assert int(tail.count_nonzero()) == 0


def test_reuse_select_bits_blocks_rejects():
    from kv_cache_amd import _lib

    lib = _lib.load()
    hist = 40961
    rows, t = 2, hist + 1
    q = torch.zeros((1, 2, 128), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((1, 1, t, 128), dtype=torch.bfloat16, device=DEV)
    words = torch.zeros((rows, -(-hist // 64)), dtype=torch.int64, device=DEV)
    ws = torch.empty((lib.qkv_reuse_select_workspace_bytes(rows, hist, 0.02) + 3) // 4, device=DEV)
    out = torch.empty(rows * 8192, dtype=torch.int64, device=DEV)
    n_out = int(lib.qkv_reuse_block_final_count(hist, 16, 0, 0, 0.02, 1))

    def call(block, n, key_count=t):
        return lib.qkv_reuse_select_bits_blocks(
            q.data_ptr(), k.data_ptr(), _lib.strides(*k.stride()), 0, 1, 2, 1, key_count, 128, words.data_ptr(),
            None, None, words.stride(0), 0, 0, 0.02, 1, 0.088, block, ws.data_ptr(), ws.numel() * 4, out.data_ptr(),
            out.data_ptr(), None, n, words.data_ptr(), words.stride(0), _lib.stream_of(q))

    unsupported, invalid = -3, -1   # QKV_ERR_UNSUPPORTED, QKV_ERR_INVALID
    assert call(16, n_out) == unsupported   # past the rows held in one workgroup
    assert call(5000, n_out) == invalid     # block beyond 4096
    assert call(0, n_out) == invalid
    n_small = int(lib.qkv_reuse_block_final_count(4000, 16, 0, 0, 0.02, 1))
    assert call(16, n_small + 1, 4001) == invalid   # index rows of the wrong width
    torch.cuda.synchronize()


@pytest.mark.parametrize("history,block,sink,recent,keep_self,density", [
    (50000, 16, 10, 10, True, 0.02), (70001, 100, 3, 5, False, 0.01), (3000, 7, 0, 0, True, 0.05),
    (9000, 64, 4, 8, True, 0.03), (45000, 4096, 10, 10, True, 0.001), (1000, 1, 2, 2, True, 0.1),
])
def test_expand_blocks_bits_equals_bytes(history, block, sink, recent, keep_self, density):
    # qkv_reuse_expand_blocks_bits (any history) against the byte expansion
    # on the same final mask: the same expanded mask, list, validity and ids
    from kv_cache_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(history + block)
    rows = 4
    mask = torch.rand((rows, history), generator=gen) < density
    mask[:, :min(sink, history)] = True
    mask[:, max(0, history - recent):] = True
    keep = int(mask.sum(dim=1).max())
    frac = keep / history
    n_out = int(lib.qkv_reuse_block_final_count(history, block, sink, recent, frac, int(keep_self)))
    by = mask.to(torch.uint8).to(DEV)
    n_w = -(-history // 64)
    pad = torch.zeros((rows, n_w * 64), dtype=torch.bool)
    pad[:, :history] = mask
    words = ((pad.view(rows, -1, 8).to(torch.uint8) << torch.arange(8, dtype=torch.uint8)).sum(-1).to(torch.uint8)
             .contiguous().view(torch.int64)).to(DEV)
    outs = []
    for bits in (False, True):
        buf = words if bits else by
        fi = torch.full((rows, n_out), 7, dtype=torch.int64, device=DEV)
        fv = torch.full((rows, n_out), 7, dtype=torch.uint8, device=DEV)
        ids = torch.full((rows, n_out), 7, dtype=torch.int32, device=DEV)
        fn = lib.qkv_reuse_expand_blocks_bits if bits else lib.qkv_reuse_expand_blocks
        _lib.check(fn(buf.data_ptr(), buf.stride(0), rows, history + 1, block, sink, recent, frac, int(keep_self),
                      fi.data_ptr(), fv.data_ptr(), ids.data_ptr(), n_out, _lib.stream_of(buf)))
        outs.append((fi, fv, ids, RU.expand_bits(buf, history) if bits else buf.bool()))
    for a, w in zip(*outs):
        assert torch.equal(a, w)
    if history % 64:   # nothing set past the history in the last word
        assert not RU.expand_bits(words, n_w * 64)[:, history:].any()


def test_expand_blocks_rejects_bad_arguments():
    m = torch.zeros((2, 100), dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="block must be"):
        RU.expand_blocks(m, 101, 5000, 0, 0, 0.1, True)
    with pytest.raises(RuntimeError, match="need history >= 1"):
        RU.expand_blocks(m, 101, 0, 0, 0, 0.1, True)


def test_step_resets_on_shorter_history():
    gen = torch.Generator().manual_seed(5)
    k = torch.randn((1, 2, 600, 128), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((1, 4, 128), generator=gen).to(torch.bfloat16).to(DEV)
    step = RU.ReuseDecodeStep("qabs8cand5reuse", 1, 4, 2, 128, 1024)
    step(q, k[:, :, :500], k[:, :, :500], 0.1)
    step(q, k[:, :, :501], k[:, :, :501], 0.1)
    a = step(q, k[:, :, :300], k[:, :, :300], 0.1).clone()       # new sequence: no previous masks
    fresh = RU.ReuseDecodeStep("qabs8cand5reuse", 1, 4, 2, 128, 1024)
    assert torch.equal(a, fresh(q, k[:, :, :300], k[:, :, :300], 0.1))
    assert torch.equal(step.final_mask(), fresh.final_mask())


def test_step_resets_on_longer_new_sequence():
    # a second sequence with a longer history, without reset(): its dim-major
    # copy must be rebuilt and no previous mask read, as for a fresh step
    gen = torch.Generator().manual_seed(6)
    k1 = torch.randn((1, 2, 600, 128), generator=gen).to(torch.bfloat16).to(DEV)
    k2 = torch.randn((1, 2, 900, 128), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((1, 4, 128), generator=gen).to(torch.bfloat16).to(DEV)
    for n2 in (502, 800):       # the previous history + 1, and a jump past it
        step = RU.ReuseDecodeStep("qabs8cand5reusefinal", 1, 4, 2, 128, 1024)
        step(q, k1[:, :, :500], k1[:, :, :500], 0.1)
        step(q, k1[:, :, :501], k1[:, :, :501], 0.1)
        if n2 == 502:
            step.reset()        # the very next length: only an explicit reset marks a new sequence
        a = step(q, k2[:, :, :n2], k2[:, :, :n2], 0.1).clone()
        fresh = RU.ReuseDecodeStep("qabs8cand5reusefinal", 1, 4, 2, 128, 1024)
        assert torch.equal(a, fresh(q, k2[:, :, :n2], k2[:, :, :n2], 0.1))
        assert torch.equal(step.final_mask(), fresh.final_mask())


def test_dim_major_append_and_token_attention():
    gen = torch.Generator().manual_seed(7)
    k = torch.randn((2, 3, 700, 128), generator=gen).to(torch.bfloat16).to(DEV)
    kdm = torch.zeros((2, 3, 128, 1024), dtype=torch.bfloat16, device=DEV)
    RU.dim_major_append(k, kdm, 0, 333)
    RU.dim_major_append(k, kdm, 333, 700)
    assert torch.equal(kdm[..., :700], k.transpose(-1, -2))
    assert int(torch.count_nonzero(kdm[..., 700:])) == 0
    # token attention: per-head lists with invalid (-1) and out-of-range ids skipped
    q = torch.randn((2, 6, 128), generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn((2, 3, 700, 128), generator=gen).to(torch.bfloat16).to(DEV)
    ids = torch.randint(0, 700, (12, 50), generator=gen, dtype=torch.int32)
    ids[0, :10] = -1
    ids[3, 5] = 900
    ws = torch.zeros(Q._lib.load().qkv_sparse_attention_workspace_bytes(2, 6, 6, 128, 50, 1) // 4,
                     dtype=torch.float32, device=DEV)
    out = RU.token_attention(q, k, v, ids.to(DEV), 0.09, workspace=ws)
    idx = ids.view(2, 6, 50).long()
    valid = (idx >= 0) & (idx < 700)
    kx, vx = k.repeat_interleave(2, dim=1), v.repeat_interleave(2, dim=1)
    want = R.final_attention(f32(q), f32(kx), f32(vx), idx.clamp(0, 699).numpy(), valid.numpy(), 0.09)
    np.testing.assert_allclose(f32(out), want[:, 0], rtol=RTOL, atol=ATOL)


def test_stream_of_follows_the_current_stream():
    # the raw handle the wrappers launch on is torch's current stream: the
    # default one, a side stream, and the capture stream of a graph
    from kv_cache_amd import _lib

    t = torch.zeros(4, device=DEV)
    assert _lib.stream_of(t) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert _lib.stream_of(t) == side.cuda_stream
    torch.cuda.synchronize()
    seen = []
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        seen.append((_lib.stream_of(t), torch.cuda.current_stream().cuda_stream))
        t.add_(1)
    assert seen[0][0] == seen[0][1]
    g.replay()
    torch.cuda.synchronize()
    assert float(t[0]) == 1.0
