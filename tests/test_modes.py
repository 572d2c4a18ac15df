"""Mode-string parsing and budget arithmetic of the path (host logic, CPU).

Pinned by known answers written from the reference's grammar (EV:748-754,
798-806) and by the closed forms of the budget (brute force over small
counts: the smallest integer at least fraction * history, clamped)."""

import math

import pytest
import torch

from kv_cache_amd import modes as M


@pytest.mark.parametrize("mode,want", [
    ("qabs32cand6p25attn", (32, 0.0625)),
    ("qabs8cand3reuse", (8, 0.03)),
    ("qabs16cand10rerank", (16, 0.10)),
    ("qabs64cand2p5reusefinalblk16", (64, 0.025)),
    ("lagtop2qabs32cand5", (32, 0.05)),
    ("qabs32cand6p25", (32, 0.0625)),
    ("qabs32cand6p25attnx", None),
    ("qboracle16q32s6p25cand2", None),
])
def test_parse_qabs(mode, want):
    got = M.parse_qabs_partial_rerank_params(mode)
    if want is None:
        assert got is None
    else:
        assert got[0] == want[0] and got[1] == pytest.approx(want[1], abs=0)


@pytest.mark.parametrize("mode,want", [
    ("qboracle16q32s6p25cand2", (16, 32, 0.0625, 0.02)),
    ("qboracle0q8s50cand1p5", (1, 8, 0.5, 0.015)),
    ("qboracle16q32s6p25", None),
])
def test_parse_qboracle(mode, want):
    assert M.parse_qboracle_params(mode) == want


def test_candidate_count_closed_form():
    for history in range(0, 300):
        for frac in (0.0, 0.001, 0.02, 0.0625, 0.5, 1.0, 1.7):
            got = M.candidate_count(frac, history)
            # smallest c >= frac*history, at least 1, at most history
            want = min(history, max(1, next(c for c in range(0, 10 ** 6) if c >= frac * history)))
            assert got == want


def test_scan_block_count_closed_form():
    for history in range(1, 200):
        for block in (1, 3, 16, 64):
            for scan in (0.01, 0.0625, 0.5, 1.0):
                nb = len(range(0, history, block))                      # blocks covering the history
                least = next(c for c in range(0, 10 ** 6) if c * block >= scan * history)
                assert M.scan_block_count(scan, history, block) == min(nb, max(1, least))


def test_decode_plan():
    p = M.decode_plan("qabs32cand6p25attn", 32769)
    assert (p.selected, p.block, p.topk, p.history) == (32, 1, 2048, 32768)
    p = M.decode_plan("qboracle16q32s6p25cand2", 32769)
    assert (p.selected, p.block, p.topk) == (32, 16, 128)          # cfg2's 128 blocks of 16
    assert p.tokens_kept == 2048
    p = M.decode_plan("qabs8cand3attn", 4097)
    assert p.selected == 16 and p.topk == math.ceil(0.03 * 4096)   # 8 channels round up to the 16-slab
    assert M.decode_plan("qabs8cand3reuse", 4097) is None          # not a mode of this path
    assert M.decode_plan("qabs32cand5attn", 1) is None             # no history yet
    assert M.selected_dims(500, 128) == 128 and M.selected_dims(0, 128) == 16


@pytest.mark.parametrize("mode,want", [
    ("qabs8cand5reuse", (8, 0.05, True, True, None)),
    ("qabs16cand10reusefinal", (16, 0.10, False, True, None)),
    ("qabs8cand3reuse2set", (8, 0.03, True, False, None)),
    ("qabs8cand6p25reuseblk16", (8, 0.0625, True, True, 16)),
    # EV:955-960 test the suffix: with a blk suffix both previous masks stay on
    ("qabs16cand10reusefinalblk8", (16, 0.10, True, True, 8)),
    ("qabs8cand3reuse2setblk32", (8, 0.03, True, True, 32)),
    ("qabs8cand5reuseblk0", (8, 0.05, True, True, 1)),     # max(1, bs) (EV:757-761)
])
def test_parse_reuse_mode(mode, want):
    from kv_cache_amd import reuse as RU

    dims, frac, use_pc, use_pf, block = RU.parse_reuse_mode(mode)
    assert (dims, use_pc, use_pf, block) == (want[0], want[2], want[3], want[4])
    assert math.isclose(frac, want[1])


@pytest.mark.parametrize("mode", ["qabs8cand5attn", "qabs8cand5reuseblk", "qabs8cand5reusefinal2set", "reuse"])
def test_parse_reuse_mode_rejects(mode):
    from kv_cache_amd import reuse as RU

    with pytest.raises(RuntimeError, match="is not a qabs"):
        RU.parse_reuse_mode(mode)


def test_sample_columns_host():
    from kv_cache_amd import reuse as RU

    assert RU.sample_columns(100, 256) is None and RU.sample_columns(100, 100) is None
    cols = RU.sample_columns(1000, 64)
    assert cols.dtype.is_floating_point is False and cols.numel() == 64
    assert int(cols[0]) == 0 and int(cols[-1]) == 999


def test_sample_column_table_rows_are_the_host_columns():
    # the device table a sample_quantile step reads: row h is sample_columns(h)
    # padded with its last column, count 0 where the sample covers the row;
    # rows are filled on first use only
    import time

    from kv_cache_amd import reuse as RU

    t0 = time.perf_counter()
    big = RU.SampleColumnTable(131072, 256, "cpu")
    assert time.perf_counter() - t0 < 1.0 and big.max_count == 256
    assert big.count(131071) == 256 and torch.equal(big.row(131071), RU.sample_columns(131071, 256))
    table = RU.SampleColumnTable(300, 40, "cpu")
    assert table.rows.shape == (300, 40) and table.rows.dtype == torch.int32 and table.max_count == 40
    for h in range(300):
        cols = RU.sample_columns(h, 40) if h else None
        n = table.count(h)
        if cols is None:
            assert n == 0
            continue
        row = table.row(h)
        assert n == cols.numel() and torch.equal(row[:n], cols)
        assert bool((row[n:] == cols[-1]).all())
    with pytest.raises(RuntimeError):
        table.count(300)
    # rows are filled in batches from the first missing history: any access
    # order gives every row its own columns
    shuffled = RU.SampleColumnTable(300, 40, "cpu")
    for h in torch.randperm(300, generator=torch.Generator().manual_seed(3)).tolist() + [299, 0, 65, 64]:
        cols = RU.sample_columns(h, 40) if h else None
        n = shuffled.count(h)
        assert n == (0 if cols is None else cols.numel())
        if n:
            assert torch.equal(shuffled.row(h)[:n], cols) and bool((shuffled.row(h)[n:] == cols[-1]).all())


@pytest.mark.parametrize("mode,want", [
    ("lagtop2qabs8cand5", ("lagtop2", None, 8, 0.05)),
    ("lagrefresh3qabs16cand6p25", ("lagrefresh", 3, 16, 0.0625)),
    ("lagrefresh0qabs8cand5", ("lagrefresh", 1, 8, 0.05)),          # max(1, N) (EV:924-928)
    ("qdriftqabs8cand5", ("qdrift", None, 8, 0.05)),
    ("qdriftcosheadqabs8cand10", ("qdriftcoshead", None, 8, 0.1)),
    ("pconf37p5qabs16cand10", ("pconf", 0.375, 16, 0.1)),            # T / 100, 'p' as the point (EV:918-922)
])
def test_parse_lagged_mode(mode, want):
    from kv_cache_amd import reuse as RU

    kind, param, dims, frac = RU.parse_lagged_mode(mode)
    assert (kind, dims) == (want[0], want[2]) and frac == pytest.approx(want[3])
    assert param == (pytest.approx(want[1]) if isinstance(want[1], float) else want[1])
    assert RU.is_lagged_mode(mode)


@pytest.mark.parametrize("mode", ["qabs8cand5reuse", "lagtop2qabs8cand5reuse", "qdriftfooqabs8cand5", "pconfqabs8cand5"])
def test_parse_lagged_mode_rejects(mode):
    from kv_cache_amd import reuse as RU

    assert not RU.is_lagged_mode(mode)
    with pytest.raises(RuntimeError, match="not a lagged reuse mode"):
        RU.parse_lagged_mode(mode)


@pytest.mark.parametrize("mode,want", [
    ("qabs8cand3attn", (8, 0.03, False, None)),
    ("qabs16cand6p25appendattn", (16, 0.0625, True, None)),
    ("qabs8cand5r4attn", (8, 0.05, False, 4)),
    ("qabs8cand5r0attn", (8, 0.05, False, 1)),                       # max(1, N) (EV:778-782)
])
def test_parse_qabs_attn_mode(mode, want):
    from kv_cache_amd import reuse as RU

    dims, frac, append, interval = RU.parse_qabs_attn_mode(mode)
    assert (dims, append, interval) == (want[0], want[2], want[3]) and frac == pytest.approx(want[1])


@pytest.mark.parametrize("mode", ["qabs8cand3", "qabs8cand3r4appendattn", "qabs8cand3sharedattn", "qabs8cand3reuse"])
def test_parse_qabs_attn_mode_rejects(mode):
    from kv_cache_amd import reuse as RU

    with pytest.raises(RuntimeError, match="is not a qabs"):
        RU.parse_qabs_attn_mode(mode)
