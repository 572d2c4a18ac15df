"""GPU parity of the exact qabs{S}cand{pct}attn / appendattn decode step
(kv_cache_amd.reuse.QabsCandidateAttentionStep, qkv_qabs_candidate_select)
against the reference's own golden vectors and the oracle: selections and
final index lists bit-exact, attention within 1e-2 relative / 2e-2 absolute
(bf16) or 1e-4 (fp32)."""

import numpy as np
import pytest
import torch

from kv_cache_amd import qabs_cuda_kernels as Q
from kv_cache_amd import reuse as RU
from oracle import ref_semantics as R
from oracle.qkv_oracle import topk_lowest_index
from tests.test_oracle_block import APPEND_SCENARIOS, ATTN_SCENARIOS, PERIODIC_SCENARIOS, load_block_golden

pytestmark = pytest.mark.gpu
DEV = "cuda"


def f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("name", [n for n in ATTN_SCENARIOS + APPEND_SCENARIOS if n.endswith("bf16")])
def test_candidate_attention_step_matches_reference_vectors(name):
    # the GQA-native step (dim-major K copy, no head expansion) on the
    # reference's bf16 scenarios: every step's final set and output
    g = load_block_golden(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k = torch.from_numpy(g["k"]).to(torch.bfloat16).to(DEV)
    v = torch.from_numpy(g["v"]).to(torch.bfloat16).to(DEV)
    step = RU.QabsCandidateAttentionStep(g["mode"], 1, hq, hkv, 128, 1024, protect_sink=g["sink"],
                                         protect_recent=g["recent"], keep_self=g["keep_self"])
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(torch.bfloat16).to(DEV)
        out = step(q, k[:, :, :n], v[:, :, :n], g["scaling"])
        assert np.array_equal(step.final_mask().cpu().numpy(), g["final"][s][..., : n - 1]), s
        assert bool((g["final"][s][..., n - 1] == g["keep_self"]).all()), s
        np.testing.assert_allclose(f32(out), g["out"][s], rtol=1e-2, atol=2e-2)


@pytest.mark.parametrize("name", [n for n in ATTN_SCENARIOS + APPEND_SCENARIOS if n.endswith("fp32")])
def test_candidate_attention_pieces_match_reference_vectors(name):
    # the fp32 scenarios through the reference-signature kernels and the
    # C-ABI selection, on GQA-expanded K as the reference's hook passes it
    g = load_block_golden(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k_all = torch.from_numpy(np.repeat(g["k"], hq // hkv, axis=1)).to(DEV)
    v_all = torch.from_numpy(np.repeat(g["v"], hq // hkv, axis=1)).to(DEV)
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(DEV)
        k, v = k_all[:, :, :n], v_all[:, :, :n]
        part = Q.partial_scores(q, k[:, :, : n - 1], g["dims"]).view(hq, n - 1)
        fi, fv, ids, hf = RU.qabs_candidate_select(part, n, g["cand"], g["sink"], g["recent"], g["keep_self"],
                                                   g["append"])
        assert np.array_equal(hf.cpu().numpy(), g["final"][s][0, :, : n - 1]), s
        out = Q.final_attention(q, k, v, fi.view(1, hq, -1), fv.view(1, hq, -1), g["scaling"])
        np.testing.assert_allclose(f32(out)[:, 0], g["out"][s], rtol=1e-4, atol=1e-4)
        assert torch.equal(ids, torch.where(fv, fi, torch.full_like(fi, -1)).to(torch.int32))


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("rows,hist,frac,sink,recent,keep_self", [
    (4, 5000, 0.03, 4, 16, True),
    (2, 40960, 0.05, 0, 0, False),      # the longest row one workgroup selects
    (2, 50000, 0.02, 10, 10, True),     # the staged top-k
    (3, 300, 0.5, 100, 100, True),      # the protected ranges cover most of the selection
    (2, 1, 0.03, 1, 1, True),           # history 1
])
def test_candidate_select_matches_oracle(append, rows, hist, frac, sink, recent, keep_self):
    gen = torch.Generator().manual_seed(hist + rows)
    scores = torch.randint(-40, 40, (rows, hist + 7), generator=gen).float()   # ties at the boundary
    scores[0, :hist] = torch.randn(hist, generator=gen)
    fi, fv, ids, hf = RU.qabs_candidate_select(scores.to(DEV), hist + 1, frac, sink, recent, keep_self, append)
    keep = R.budget_count(hist, frac)
    sel = np.sort(topk_lowest_index(scores[:, :hist].numpy(), keep), axis=-1)
    sink_end = min(sink, hist)
    rec_begin = max(hist - recent, sink_end) if recent else hist
    tail = list(range(sink_end)) + list(range(rec_begin, hist)) + ([hist] if keep_self else [])
    want_i = np.concatenate([sel, np.tile(np.array(tail, dtype=np.int64), (rows, 1))], axis=-1)
    prot = (sel < sink_end) | ((sel >= hist - recent) if recent else np.zeros_like(sel, bool))
    want_v = np.concatenate([np.ones_like(sel, bool) if append else ~prot, np.ones((rows, len(tail)), bool)], -1)
    assert np.array_equal(fi.cpu().numpy(), want_i)
    assert np.array_equal(fv.cpu().numpy(), want_v)
    want_hf = np.zeros((rows, hist), bool)
    np.put_along_axis(want_hf, sel, True, axis=-1)
    want_hf[:, :sink_end] = True
    if recent:
        want_hf[:, max(0, hist - recent):] = True
    assert np.array_equal(hf.cpu().numpy(), want_hf)


def test_candidate_attention_step_resets_and_matches_oracle_at_length():
    # a longer history than the vectors (4 rows of 9000), GQA 4, and a new
    # sequence of the same length after reset: outputs from the oracle step
    gen = torch.Generator().manual_seed(3)
    t = 9000
    k = torch.randn((1, 2, t + 1, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((1, 2, t + 1, 128), generator=gen).to(torch.bfloat16)
    q = torch.randn((1, 8, 128), generator=gen).to(torch.bfloat16)
    step = RU.QabsCandidateAttentionStep("qabs8cand3attn", 1, 8, 2, 128, t + 64, protect_sink=4, protect_recent=8)
    out = step(q.to(DEV), k.to(DEV), v.to(DEV), 128 ** -0.5)
    want, keep = R.qabs_attn_step(f32(q), f32(k), f32(v), 8, 0.03, 128 ** -0.5, 4, 8, True)
    np.testing.assert_allclose(f32(out), want[:, 0], rtol=1e-2, atol=2e-2)
    assert np.array_equal(step.final_mask().cpu().numpy(), keep[..., :t])
    k2 = torch.randn((1, 2, t + 1, 128), generator=gen).to(torch.bfloat16)
    step.reset()
    out2 = step(q.to(DEV), k2.to(DEV), v.to(DEV), 128 ** -0.5)
    want2, _ = R.qabs_attn_step(f32(q), f32(k2), f32(v), 8, 0.03, 128 ** -0.5, 4, 8, True)
    np.testing.assert_allclose(f32(out2), want2[:, 0], rtol=1e-2, atol=2e-2)


def test_candidate_select_rejects_bad_arguments():
    s = torch.zeros((2, 10), device=DEV)
    with pytest.raises(RuntimeError, match="need 2 <= key_count"):
        RU.qabs_candidate_select(s, 1, 0.1, 0, 0, True)
    with pytest.raises(RuntimeError, match="not a qabs"):
        RU.QabsCandidateAttentionStep("qabs8cand3reuse", 1, 4, 2, 128, 256)


def _keep_of(fi, fv, key_count):
    fi, fv = fi.cpu().numpy(), fv.cpu().numpy().astype(bool)
    keep = np.zeros((*fi.shape[:-1], key_count), dtype=bool)
    for lead in np.ndindex(*fi.shape[:-1]):
        keep[lead][fi[lead][fv[lead]]] = True
    return keep


@pytest.mark.parametrize("name", [n for n in PERIODIC_SCENARIOS if n.endswith("bf16")])
def test_periodic_step_matches_reference_vectors(name):
    # qabs{S}cand{pct}r{N}attn: steps at a multiple of N reselect, the others
    # rebuild the list from the kept selection at their own history
    g = load_block_golden(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k = torch.from_numpy(g["k"]).to(torch.bfloat16).to(DEV)
    v = torch.from_numpy(g["v"]).to(torch.bfloat16).to(DEV)
    step = RU.QabsCandidateAttentionStep(g["mode"], 1, hq, hkv, 128, 1024, protect_sink=g["sink"],
                                         protect_recent=g["recent"], keep_self=g["keep_self"])
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(torch.bfloat16).to(DEV)
        out = step(q, k[:, :, :n], v[:, :, :n], g["scaling"])
        fi, fv = step.final_indices()
        assert np.array_equal(_keep_of(fi, fv, n), g["final"][s][..., :n]), s
        np.testing.assert_allclose(f32(out), g["out"][s], rtol=1e-2, atol=2e-2)


@pytest.mark.parametrize("name", [n for n in PERIODIC_SCENARIOS if n.endswith("fp32")])
def test_periodic_pieces_match_reference_vectors(name):
    g = load_block_golden(name)
    hq, hkv = g["q"].shape[2], g["k"].shape[1]
    k_all = torch.from_numpy(np.repeat(g["k"], hq // hkv, axis=1)).to(DEV)
    v_all = torch.from_numpy(np.repeat(g["v"], hq // hkv, axis=1)).to(DEV)
    kept = None
    for s in range(g["steps"]):
        n = g["t0"] + s + 1
        q = torch.from_numpy(g["q"][s]).to(DEV)
        k, v = k_all[:, :, :n], v_all[:, :, :n]
        if kept is not None and (n - 1) % g["interval"] != 0:
            fi, fv, ids = RU.final_indices_from_selected(kept, kept.size(1), n, g["sink"], g["recent"],
                                                         g["keep_self"])
        else:
            part = Q.partial_scores(q, k[:, :, : n - 1], g["dims"]).view(hq, n - 1)
            fi, fv, ids, _ = RU.qabs_candidate_select(part, n, g["cand"], g["sink"], g["recent"], g["keep_self"])
            keep_n = R.budget_count(n - 1, g["cand"])
            kept = fi[:, :keep_n].contiguous()
        assert np.array_equal(_keep_of(fi.view(1, hq, -1), fv.view(1, hq, -1), n), g["final"][s][..., :n]), s
        out = Q.final_attention(q, k, v, fi.view(1, hq, -1), fv.view(1, hq, -1), g["scaling"])
        np.testing.assert_allclose(f32(out)[:, 0], g["out"][s], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("hist,n_sel,sink,recent,keep_self", [(500, 40, 4, 8, True), (33, 20, 0, 0, False),
                                                              (100, 1, 60, 60, True), (2000, 0, 3, 3, True)])
def test_final_indices_from_selected_matches_oracle(hist, n_sel, sink, recent, keep_self):
    # selections with indices in the protected ranges, past the history and
    # negative; every entry and its validity as EV:2938-2982 builds them
    gen = torch.Generator().manual_seed(hist + n_sel)
    rows = 3
    sel = torch.randint(-3, hist + 5, (rows, n_sel + 2), generator=gen)
    fi, fv, ids = RU.final_indices_from_selected(sel.to(DEV), n_sel, hist + 1, sink, recent, keep_self)
    s = sel[:, :n_sel].numpy()
    want_i, want_v = R.final_indices_np(np.maximum(s, 0), (s >= 0) & (s < hist), hist, hist + 1, sink, recent,
                                        keep_self)
    got_i, got_v = fi.cpu().numpy(), fv.cpu().numpy()
    assert np.array_equal(got_v, want_v)
    assert np.array_equal(got_i[got_v], want_i[want_v])   # invalid entries' indices are not read
    assert np.array_equal(ids.cpu().numpy(), np.where(got_v, got_i, -1))


def _qabs_case(b, hist, pattern, seed):
    # (q, K) whose partial scores follow `pattern` (K[t] = c_t * a fixed
    # vector: the scores are c_t times the row's sum over its dims)
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((b, 32, 128), generator=gen).to(torch.bfloat16)
    if pattern == "normal":
        k = torch.randn((b, 8, hist + 1, 128), generator=gen)
    else:
        if pattern == "equal":     # the whole row in one bin: the list selected from memory
            c = torch.ones(hist + 1)
        elif pattern == "narrow":  # 128 values in [1, 2): a few thousand scores in the boundary bin
            c = 1.0 + torch.randint(0, 256, (hist + 1,), generator=gen).float() / 256.0
        elif pattern == "coarse":  # 16 values in one bin: ties at the threshold
            c = 1.0 + torch.randint(0, 16, (hist + 1,), generator=gen).float() / 128.0
        else:
            raise ValueError(pattern)
        k = c.view(1, 1, hist + 1, 1).expand(b, 8, hist + 1, 128).clone()
    return q.to(DEV), k.to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("b,hist,pattern,frac,sink,recent,keep_self,append", [
    (1, 32768, "normal", 0.03, 10, 10, 1, 0),    # the timed mode's shape: 5 slices per row
    (1, 32768, "normal", 0.05, 4, 16, 1, 1),     # appendattn: protected picks stay valid
    (1, 20000, "equal", 0.03, 0, 0, 0, 0),       # every score equal: the lowest positions
    (1, 20000, "narrow", 0.1, 10, 10, 1, 0),
    (1, 30011, "coarse", 0.03, 10, 10, 1, 0),    # equal scores at the threshold, lowest positions first
    (3, 777, "narrow", 1.0, 2, 2, 1, 0),         # every position kept
    (2, 40960, "normal", 0.02, 10, 10, 1, 0),    # the longest one-workgroup row, 64 rows
])
def test_qabs_candidates_equal_two_calls(b, hist, pattern, frac, sink, recent, keep_self, append):
    # qkv_qabs_candidates (partial scores with first-digit counts, the selection
    # across workgroups) against qkv_reuse_partial_scores + qkv_qabs_candidate_select
    from kv_cache_amd import _lib

    lib = _lib.load()
    q, k = _qabs_case(b, hist, pattern, hist + b)
    rows, dims, key_count = b * 32, 8, hist + 1
    kdm = torch.zeros((b, 8, 128, hist + 8), dtype=torch.bfloat16, device=DEV)
    RU.dim_major_append(k, kdm, 0, hist)
    want_p = RU.reuse_partial_scores(q, kdm, hist, dims)
    want = RU.qabs_candidate_select(want_p, key_count, frac, sink, recent, bool(keep_self), bool(append))
    n_out = want[0].size(1)
    got = (torch.full_like(want[0], -7), torch.zeros_like(want[1]), torch.full_like(want[2], -7),
           torch.zeros_like(want[3]))
    part = torch.zeros((rows, hist + 8), device=DEV)
    ws = torch.zeros((lib.qkv_qabs_candidates_workspace_bytes(rows, hist, frac) + 3) // 4, device=DEV)
    for _ in range(2):   # the second call on the workspace the first left
        _lib.check(lib.qkv_qabs_candidates(
            q.data_ptr(), kdm.data_ptr(), _lib.strides(*kdm.stride()), 0, b, 32, 8, key_count, 128, dims, frac, sink,
            recent, keep_self, append, part.data_ptr(), part.stride(0), ws.data_ptr(), ws.numel() * 4,
            got[0].data_ptr(), got[1].data_ptr(), got[2].data_ptr(), n_out, got[3].data_ptr(), got[3].stride(0),
            _lib.stream_of(q)))
        assert torch.equal(part[:, :hist], want_p[:, :hist])
        for g, w in zip(got, want):
            assert torch.equal(g, w)
        assert not ws[: rows * 4096].any()   # the first-digit counts are left zero
        state = ws[rows * 4096 : rows * 4096 + rows * 48].view(torch.int32).view(rows, 48)
        assert not state[:, 40].any()        # ... and the tickets
    if pattern == "equal":
        keep = want[0].size(1) - (sink + recent + keep_self)
        assert torch.equal(got[0][:, :keep].cpu(), torch.arange(keep).expand(rows, keep))
