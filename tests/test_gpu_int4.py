"""GPU parity of the int4 path against the CPU oracle: bit-exact packing,
channel choice, slab, int32 scores, fp32 keys, block maxima and top-k
indices; attention within 1e-2 relative / 2e-2 absolute of fp64."""

import numpy as np
import pytest
import torch

from kv_cache_amd import int4 as K
from kv_cache_amd import prefill as P
from kv_cache_amd.workloads import CONFIGS, make_layer
from oracle import qkv_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2   # attention tolerance stated by the north star


def f32(t):
    return t.float().cpu().numpy()


def bits16(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def u64(t):
    return t.cpu().numpy().view(np.uint64)


def rand_k(b, h, t, d, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((b, h, t, d), generator=g) * scale
    k[..., 3] *= 8.0
    return k.to(torch.bfloat16)


# ---------------------------------------------------------------------------
# pack
# ---------------------------------------------------------------------------

def test_pack_known_answers():
    rows = torch.zeros((1, 1, 8, 128), dtype=torch.float32)
    kat = [[0, 0, 0, 0], [7, -7, 3.5, 0.5], [14, 1, -1, 2.5], [7, 2.5, -2.5, 1.5],
           [1.0e6, -1.0e6, 0, 1], [7 * 2.0 ** -20, 0, 0, 0], [2.0 ** -30, 0, 0, 0], [1, -0.5, 0.25, 0]]
    for t, vals in enumerate(kat):
        rows[0, 0, t, :4] = torch.tensor(vals)
    key = rows.to(torch.bfloat16).to(DEV)
    packed, scales = K.int4_pack_k(key, 32)
    torch.cuda.synchronize()
    want_p, want_s = O.int4_pack_k(f32(key), 32)
    assert np.array_equal(packed[..., :8, :].cpu().numpy(), want_p)
    assert np.array_equal(bits16(scales[..., :8, :]), want_s)
    assert bits16(scales)[0, 0, :8, 0].tolist() == [0, 0x3C00, 0x4000, 0x3C00, 0x7BFF, 0x0010, 0, 0x3092]


@pytest.mark.parametrize("group", [32, 64, 128])
def test_pack_matches_oracle(group):
    key = rand_k(2, 3, 300, 128, seed=group).to(DEV)
    packed, scales = K.int4_pack_k(key, group)
    want_p, want_s = O.int4_pack_k(f32(key), group)
    assert np.array_equal(packed[:, :, :300].cpu().numpy(), want_p)
    assert np.array_equal(bits16(scales[:, :, :300]), want_s)


def test_pack_strided_and_appended_range():
    # K as a slice of a larger-capacity buffer (non-contiguous token stride),
    # packed in two calls: tokens [0, 100) then the decode-style append [100, 101).
    big = rand_k(1, 2, 160, 128, seed=7).to(DEV)
    key = big[:, :, :101]
    packed = torch.zeros((1, 2, 128, 64), dtype=torch.uint8, device=DEV)
    scales = torch.zeros((1, 2, 128, 4), dtype=torch.float16, device=DEV)
    K.int4_pack_k(key, 32, packed=packed, scales=scales, t_end=100)
    K.int4_pack_k(key, 32, packed=packed, scales=scales, t_begin=100, t_end=101)
    want_p, want_s = O.int4_pack_k(f32(key), 32)
    assert np.array_equal(packed[:, :, :101].cpu().numpy(), want_p)
    assert np.array_equal(bits16(scales[:, :, :101]), want_s)
    assert int(packed[:, :, 101:].abs().sum()) == 0


# ---------------------------------------------------------------------------
# channel subset and slab
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("group,count", [(32, 32), (128, 64), (64, 16), (32, 128)])
def test_select_channels_matches_oracle(group, count):
    key = rand_k(2, 4, 777, 128, seed=count).to(DEV)
    packed, scales = K.int4_pack_k(key, group)
    chan, stats = K.select_channels(packed, scales, 777, group, count)
    want_p, want_s = O.int4_pack_k(f32(key), group)
    want_stats = O.channel_stats(want_p, want_s, group)
    assert np.array_equal(u64(stats).reshape(8, 128), want_stats.reshape(8, 128))
    assert np.array_equal(chan.cpu().numpy().reshape(8, count), O.select_channels(want_stats.reshape(8, 128), count))
    assert 3 in chan.cpu().numpy()[0, 0].tolist()   # the x8 outlier channel is always chosen


def test_select_channels_all_ties():
    key = torch.ones((1, 1, 64, 128), dtype=torch.bfloat16, device=DEV)
    packed, scales = K.int4_pack_k(key, 32)
    chan, _ = K.select_channels(packed, scales, 64, 32, 32)
    assert chan.cpu().numpy()[0, 0].tolist() == list(range(32))


@pytest.mark.parametrize("count", [16, 32, 64, 128])
def test_slab_matches_oracle(count):
    key = rand_k(1, 3, 513, 128, seed=100 + count).to(DEV)
    g = torch.Generator().manual_seed(count)
    chan = torch.stack([torch.randperm(128, generator=g)[:count].sort().values for _ in range(3)])
    chan = chan.view(1, 3, count).to(torch.int32).to(DEV)
    cap = K.round_capacity(513)
    slab = torch.zeros((1, 3, cap, count // 2), dtype=torch.uint8, device=DEV)
    ss = torch.zeros((1, 3, cap), dtype=torch.float16, device=DEV)
    K.build_slab(key, chan, slab=slab, slab_scales=ss)
    want, want_s = O.build_slab(f32(key).reshape(3, 513, 128), chan.cpu().numpy().reshape(3, count))
    stored = slab.cpu().numpy().reshape(3, -1)
    assert np.array_equal(O.unswizzle_slab(stored, count, 513), want)
    # the stored bytes are exactly the oracle's swizzled slab (padding untouched)
    assert np.array_equal(stored, O.swizzle_slab(want, slab.size(2)))
    assert np.array_equal(bits16(ss[:, :, :513]).reshape(3, 513), want_s)


# ---------------------------------------------------------------------------
# decode scoring + block max
# ---------------------------------------------------------------------------

def _score_case(b, hq, hkv, t, count, block, seed):
    g = torch.Generator().manual_seed(seed)
    key = rand_k(b, hkv, t, 128, seed=seed).to(DEV)
    q = torch.randn((b, hq, 128), generator=g).to(torch.bfloat16).to(DEV)
    cache = K.Int4KCache.from_prefill(key, 32 if count <= 32 else 128, count)
    bmax, isum, keys, qs = K.decode_scores(q, cache.chan_idx, cache.slab, cache.slab_scales, t, block, debug=True)
    bmax_only = K.decode_scores(q, cache.chan_idx, cache.slab, cache.slab_scales, t, block)
    rows = b * hkv
    chan = cache.chan_idx.cpu().numpy().reshape(rows, count)
    slab = O.unswizzle_slab(cache.slab.cpu().numpy().reshape(rows, -1), count, t)
    sbits = bits16(cache.slab_scales[:, :, :t]).reshape(rows, t)
    q8, want_qs = O.quantize_query_group(f32(q), chan, hkv)
    want_i = O.partial_scores_i32(q8, slab)
    want_k = O.ranking_keys(want_i, sbits)
    want_b = O.block_max(want_k, block)
    assert np.array_equal(qs.cpu().numpy().reshape(rows), want_qs)
    assert np.array_equal(isum.cpu().numpy().reshape(rows, t), want_i)
    assert np.array_equal(keys.cpu().numpy().reshape(rows, t).view(np.uint32), want_k.view(np.uint32))
    assert np.array_equal(bmax.cpu().numpy().reshape(rows, -1), want_b)
    assert np.array_equal(bmax_only.cpu().numpy().reshape(rows, -1), want_b)
    return want_b


@pytest.mark.parametrize("count", [16, 32, 64, 128])
def test_query_words_match_oracle(count):
    g = torch.Generator().manual_seed(count)
    b, hq, hkv = 2, 16, 4
    q = torch.randn((b, hq, 128), generator=g).to(torch.bfloat16)
    chan = torch.stack([torch.randperm(128, generator=g)[:count].sort().values for _ in range(b * hkv)])
    chan = chan.view(b, hkv, count).to(torch.int32)
    words, qs = K.query_words(q.to(DEV), chan.to(DEV), qscale=torch.empty((b, hkv), device=DEV))
    q8, want_qs = O.quantize_query_group(f32(q), chan.numpy().reshape(b * hkv, count), hkv)
    got = words.cpu().numpy().reshape(b * hkv, count // 4).view(np.uint32)
    assert np.array_equal(got, O.pack_query_words(q8))
    assert np.array_equal(qs.cpu().numpy().reshape(-1), want_qs)


@pytest.mark.parametrize("count", [16, 32, 64, 128])
@pytest.mark.parametrize("block", [1, 16, 64])
def test_decode_scores_matches_oracle(count, block):
    _score_case(2, 8, 4, 1000, count, block, seed=count * 7 + block)


@pytest.mark.parametrize("b,hq,hkv,t", [(1, 8, 8, 64), (1, 16, 8, 4096), (3, 32, 8, 5003), (1, 64, 8, 2500)])
def test_decode_scores_shapes(b, hq, hkv, t):
    _score_case(b, hq, hkv, t, 32, 16, seed=t)


def test_decode_scores_many_chunks():
    # enough tokens that one row spans several workgroups
    _score_case(1, 2, 1, 70000, 32, 16, seed=11)


# ---------------------------------------------------------------------------
# top-k
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,k", [(5, 2), (100, 1), (100, 100), (2048, 128), (2048, 256), (4096, 256),
                                 (5000, 999), (12288, 64), (20000, 1024), (131072, 1024),
                                 (4097, 1), (4097, 1024), (8192, 1024), (300000, 1000), (20000, 1025)])
def test_topk_matches_oracle(n, k):
    g = torch.Generator().manual_seed(n + k)
    vals = torch.randint(-50, 50, (6, n), generator=g).float()   # heavy ties
    vals[0] = torch.randn(n, generator=g)
    vals[1, ::3] = -0.0
    vals[1, 1::3] = 0.0
    vals[2, : n // 2] = -float("inf")
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))


def test_topk_staged_equals_single_workgroup():
    # Rows longer than 4096 keys go through the staged reduction; qkv_topk
    # (one workgroup per row) must give the same indices.
    from kv_cache_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(77)
    vals = torch.randint(-1000, 1000, (5, 70000), generator=g).float().to(DEV)
    vals[1, 10000:] = -float("inf")
    for k in (1, 64, 1024):
        want = torch.empty((5, k), dtype=torch.int32, device=DEV)
        _lib.check(lib.qkv_topk(vals.data_ptr(), 5, 70000, 70000, k, want.data_ptr(), _lib.stream_of(vals)))
        assert lib.qkv_topk_workspace_bytes(5, 70000, k) > 0
        got = K.block_topk(vals, k)
        assert torch.equal(got, want)


def _adversarial_rows(n, seed):
    """Rows that stress the selection's lower bound (thread t of a 256-thread
    row holds keys t + 256i, so key x sits in wave (x % 256) // 64)."""
    g = torch.Generator().manual_seed(seed)
    rows = [torch.randn(n, generator=g) for _ in range(7)]
    wave = (torch.arange(n) % 256) // 64
    rows[0][wave == 0] += 50.0                               # every large key in one wave
    rows[1] = torch.where(wave == 3, rows[1] + 50.0, rows[1])  # ... in the last wave
    rows[2] = torch.full((n,), 2.5)                          # all equal
    rows[3] = (torch.arange(n) % 5).float()                  # 5 values, heavy ties at the boundary
    rows[4][(torch.arange(n) % 64) != 7] = -float("inf")     # one lane per wave holds finite keys
    rows[5] = torch.where(torch.arange(n) % 256 < 3, rows[5] + 9.0, -rows[5].abs() - 20.0)
    rows[6] = torch.ldexp(torch.ones(n), torch.randint(-30, 30, (n,), generator=g))   # wide exponent range
    return torch.stack(rows)


@pytest.mark.parametrize("n,k", [(2048, 128), (2048, 1), (2048, 7), (2048, 256), (2048, 300), (1000, 64),
                                 (4096, 255), (4096, 129), (2049, 128)])
def test_topk_adversarial_layouts(n, k):
    vals = _adversarial_rows(n, n + k)
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))
    got = P.block_topk(vals.to(DEV), k).cpu().numpy()    # -inf keys not selectable, -1 padding
    assert np.array_equal(got, O.prefill_block_topk(vals.numpy(), k))


@pytest.mark.parametrize("n,k", [(131072, 1024), (70000, 64), (8193, 1000), (40000, 1), (16384, 513)])
def test_topk_long_rows_adversarial(n, k):
    # long rows (the bound-and-filter path: per-chunk bounds, filtered
    # per-chunk lists, one WideSelect per row): all-equal rows and heavy ties
    # pass more than k keys per chunk, one-lane rows leave most chunks empty,
    # a partial last chunk adds no bound
    vals = _adversarial_rows(n, n + k)
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))


def test_topk_long_rows_one_chunk_over_k():
    # one chunk holds far more than k keys above the floor, the others a few
    n, k = 65536, 256
    g = torch.Generator().manual_seed(5)
    vals = torch.randn((3, n), generator=g)
    vals[0, 8192:12288] += 10.0                 # chunk 2: 4096 keys above every other chunk's
    vals[1, 5::4096] = 100.0                   # one huge key per chunk
    vals[2, 4096 * 15:] = -float("inf")        # the last chunk -inf only
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))


def test_topk_long_rows_three_launch_grid():
    # rows * chunks above 256: histogram, filter and final selection as three
    # launches (the one-launch form needs every workgroup resident)
    n, k = 131072, 1024
    vals = torch.cat([_adversarial_rows(n, 11), _adversarial_rows(n, 12)[:2]])   # 9 rows x 32 chunks
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))


def test_topk_one_launch_workspace_reuse():
    # the one-launch path's row tickets return to zero: one workspace serves
    # calls of different shapes in a row, and every call is exact
    g = torch.Generator().manual_seed(21)
    ws = K.topk_workspace(8, 131072, 1024, DEV)
    for rows, n, k in [(8, 131072, 1024), (3, 131072, 1024), (8, 131072, 1024), (5, 70000, 64),
                       (8, 131072, 1)]:
        vals = torch.randn((rows, n), generator=g)
        vals[rows // 2, ::2] = 7.0   # ties across every chunk
        got = K.block_topk(vals.to(DEV), k, workspace=ws).cpu().numpy()
        assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k)), (rows, n, k)


def test_topk_one_launch_ticket_pool_wraps():
    # more one-launch calls than the library's ticket slots (4096): every
    # completed call leaves its words zero, so a reused slot counts from zero
    g = torch.Generator().manual_seed(23)
    xs = [torch.randn((2, 9000), generator=g) for _ in range(3)]
    xs[1][0, ::3] = 0.5   # ties
    want = [O.topk_lowest_index(x.numpy(), 64) for x in xs]
    dev = [x.to(DEV) for x in xs]
    out = torch.empty((2, 64), dtype=torch.int32, device=DEV)
    ws = K.topk_workspace(2, 9000, 64, DEV)
    for i in range(4200):
        K.block_topk(dev[i % 3], 64, out=out, workspace=ws)
        if i % 700 == 0 or i >= 4197:
            assert np.array_equal(out.cpu().numpy(), want[i % 3]), i


def test_topk_one_launch_graph_replays():
    # the one-launch path captured in a graph: replays with new inputs between
    # them, each checked
    n, k, rows = 131072, 1024, 8
    g = torch.Generator().manual_seed(31)
    x = torch.empty((rows, n), device=DEV)
    out = torch.empty((rows, k), dtype=torch.int32, device=DEV)
    ws = K.topk_workspace(rows, n, k, DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.block_topk(x.normal_(), k, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.block_topk(x, k, out=out, workspace=ws)
    for rep in range(4):
        host = torch.randn((rows, n), generator=g)
        if rep == 2:
            host[3] = 1.0
        x.copy_(host)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), O.topk_lowest_index(host.numpy(), k)), rep


def test_topk_one_launch_wait_limit_zero():
    # a chunk that stops waiting for its row keeps its exact top-k instead of
    # filtering by the row's floor (forced here from the host with a zero
    # wait): the lists then exceed what the final step gathers into LDS, and
    # the result is still exact
    from kv_cache_amd import _lib
    lib = _lib.load()
    n, k = 131072, 1024
    vals = _adversarial_rows(n, 41)
    _lib.check(lib.qkv_topk_set_wait_limit(0))
    try:
        got = K.block_topk(vals.to(DEV), k).cpu().numpy()
        got2 = K.block_topk(vals.to(DEV), 3).cpu().numpy()
    finally:
        _lib.check(lib.qkv_topk_set_wait_limit(-1))
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))
    assert np.array_equal(got2, O.topk_lowest_index(vals.numpy(), 3))
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()   # default wait again
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))


@pytest.mark.parametrize("n,k", [(1, 1), (7, 3), (64, 64), (200, 17), (255, 128), (256, 1), (256, 255), (257, 100)])
def test_topk_small_rows(n, k):
    # rows of at most 256 keys rank every key against the row (one key per
    # thread): ties, signed zeros, -inf (selectable for qkv_topk, not for the
    # prefill selection, which pads with -1), an all -inf row
    g = torch.Generator().manual_seed(n * 31 + k)
    vals = torch.randint(-5, 5, (6, n), generator=g).float()
    vals[0] = torch.randn(n, generator=g)
    vals[1, ::2] = -0.0
    vals[1, 1::2] = 0.0
    vals[2, : n // 2] = -float("inf")
    vals[3] = -float("inf")
    vals[4] = 3.0
    got = K.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))
    got = P.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.prefill_block_topk(vals.numpy(), k))


@pytest.mark.parametrize("n,k,ld", [(1024, 64, 1024), (1024, 1, 1025), (1000, 100, 1000), (200, 64, 203),
                                    (513, 7, 513)])
def test_topk_many_short_rows(n, k, ld):
    # >= 1024 rows of <= 1024 keys take the one-wave-per-row kernel (16-byte
    # loads only for full, aligned rows); ties, signed zeros and -inf rows.
    rows = 1100
    g = torch.Generator().manual_seed(n * 7 + k)
    base = torch.randn((rows, ld), generator=g)
    base[::3] = torch.randint(-4, 4, (len(range(0, rows, 3)), ld), generator=g).float()   # heavy ties
    base[1::7, : n // 2] = -float("inf")
    base[2::11] = 0.0
    base[2::22] = -0.0
    vals = base[:, :n]
    dev = base.to(DEV)[:, :n]   # rows ld apart on the device too
    got = K.block_topk(dev, k).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(vals.numpy(), k))
    got = P.block_topk(dev, k).cpu().numpy()   # -inf keys not selectable, -1 padding
    assert np.array_equal(got, O.prefill_block_topk(vals.numpy(), k))


def test_topk_strided_rows():
    g = torch.Generator().manual_seed(3)
    base = torch.randint(0, 4, (4, 300), generator=g).float().to(DEV)
    view = base[:, :256]
    got = K.block_topk(view, 17).cpu().numpy()
    assert np.array_equal(got, O.topk_lowest_index(view.cpu().numpy(), 17))


# ---------------------------------------------------------------------------
# sparse attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("g_size", [1, 2, 4, 8])
@pytest.mark.parametrize("block,nsel", [(1, 256), (1, 300), (16, 128), (64, 7)])
def test_sparse_attention_matches_fp64(g_size, block, nsel):
    b, hkv, t = 2, 2, 3000
    hq = hkv * g_size
    gen = torch.Generator().manual_seed(g_size * 1000 + block)
    q = torch.randn((b, hq, 128), generator=gen).to(torch.bfloat16)
    k = (torch.randn((b, hkv, t, 128), generator=gen) * 2).to(torch.bfloat16)
    v = torch.randn((b, hkv, t, 128), generator=gen).to(torch.bfloat16)
    nb = -(-t // block)
    sel = torch.stack([torch.randperm(nb, generator=gen)[:nsel].sort().values for _ in range(b * hkv)])
    sel = sel.view(b, hkv, nsel).to(torch.int32)
    sel[0, 0, 0] = -1                  # invalid ids are skipped
    sel[0, 1, -1] = nb - 1             # the partial last block
    out = K.sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV), block, t, 128 ** -0.5)
    want = O.sparse_attention(f32(q), f32(k), f32(v), sel.numpy(), block, t, 128 ** -0.5)
    assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("g_size,batch,t,block,nsel", [
    (2, 8, 20000, 16, 1024),    # 64 rows x 16384 slots: 16 chunks per wave, 8 splits
    (2, 1, 9000, 16, 512),      # 8 rows x 8192 slots: 2 chunks per wave
    (4, 1, 9000, 16, 512),      # G = 4 (4-token steps): 4 chunks per wave
    (4, 16, 9000, 16, 300),     # G = 4, 128 rows x 4800 slots: 32 chunks per wave, partial last split
    (8, 4, 20000, 1, 4000),     # G = 8, block 1: 8 chunks per wave, slots not a multiple of a chunk
    (1, 8, 20000, 64, 300),     # G = 1: 16 chunks per wave, partial last split
])
def test_sparse_attention_long_selections(g_size, batch, t, block, nsel):
    # Long selections take several chunks per wave and few splits per row;
    # sampled rows are checked against fp64 (rows are independent).
    hkv = 8
    hq = hkv * g_size
    gen = torch.Generator().manual_seed(g_size * 31 + nsel)
    q = torch.randn((batch, hq, 128), generator=gen).to(torch.bfloat16).to(DEV)
    k = (torch.randn((batch, hkv, t, 128), generator=gen) * 2).to(torch.bfloat16).to(DEV)
    v = torch.randn((batch, hkv, t, 128), generator=gen).to(torch.bfloat16).to(DEV)
    nb = -(-t // block)
    rows = batch * hkv
    sel = torch.stack([torch.randperm(nb, generator=gen)[:nsel].sort().values for _ in range(rows)])
    sel = sel.view(batch, hkv, nsel).to(torch.int32)
    sel[0, 0, :5] = -1                  # invalid ids are skipped
    sel[0, 0, 7] = nb + 3               # ids past the last block too
    sel[-1, -1, -1] = nb - 1            # the partial last block
    out = K.sparse_attention(q, k, v, sel.to(DEV), block, t, 128 ** -0.5)
    got = f32(out)
    for r in (0, rows // 2, rows - 1):
        bi, j = divmod(r, hkv)
        want = O.sparse_attention(f32(q[bi:bi + 1, j * g_size:(j + 1) * g_size]), f32(k[bi:bi + 1, j:j + 1]),
                                  f32(v[bi:bi + 1, j:j + 1]), sel[bi:bi + 1, j:j + 1].numpy(), block, t,
                                  128 ** -0.5)
        np.testing.assert_allclose(got[bi, j * g_size:(j + 1) * g_size], want[0], rtol=RTOL, atol=ATOL)


def test_sparse_attention_workspace_reuse():
    # One zero-filled workspace serves successive calls with different split
    # counts: the row tickets return to zero after every call.
    gen = torch.Generator().manual_seed(9)
    b, hkv, g_size, t = 2, 4, 2, 5000
    q = torch.randn((b, hkv * g_size, 128), generator=gen).to(torch.bfloat16)
    k = torch.randn((b, hkv, t, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((b, hkv, t, 128), generator=gen).to(torch.bfloat16)
    ws = K.attention_workspace(b, hkv * g_size, hkv, 128, 313, 16, DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    for nsel, block in [(313, 16), (40, 16), (200, 1), (313, 16), (700, 1), (16, 16), (99, 16)]:
        nb = -(-t // block)
        sel = torch.stack([torch.randperm(nb, generator=gen)[:nsel].sort().values for _ in range(b * hkv)])
        sel = sel.view(b, hkv, nsel).to(torch.int32)
        out = K.sparse_attention(qd, kd, vd, sel.to(DEV), block, t, 0.088, workspace=ws)
        want = O.sparse_attention(f32(q), f32(k), f32(v), sel.numpy(), block, t, 0.088)
        assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL), (nsel, block)
    tickets = ws[:65536].view(torch.int32).cpu()
    assert int(tickets.abs().sum()) == 0


@pytest.mark.parametrize("g_size,batch,t,block,nsel", [
    (4, 8, 32768, 16, 128),     # cfg2's shape: 2048 blocks, 128 kept
    (2, 2, 65536, 16, 256),     # 4096 blocks: the largest row that selects in the kernel
    (4, 1, 4096, 1, 4096),      # every block kept
    (1, 3, 3000, 64, 7),        # partial last block, G = 1
    (8, 2, 700, 16, 44),        # G = 8
    (4, 1, 10, 16, 1),          # one block
])
def test_sparse_attention_select_equals_unfused(g_size, batch, t, block, nsel):
    # The fused selection equals block_topk on the same maxima (bit-exact,
    # lowest index wins ties) and the attention equals the unfused call's.
    hkv = 8 if batch > 1 else 4
    hq = hkv * g_size
    nb = -(-t // block)
    gen = torch.Generator().manual_seed(t + nsel)
    q = torch.randn((batch, hq, 128), generator=gen).to(torch.bfloat16).to(DEV)
    k = torch.randn((batch, hkv, t, 128), generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn((batch, hkv, t, 128), generator=gen).to(torch.bfloat16).to(DEV)
    bmax = torch.randint(-40, 40, (batch, hkv, nb), generator=gen).float()   # heavy ties
    bmax[0, 0] = torch.randn(nb, generator=gen)
    bmax[-1, -1, : nb // 2] = -float("inf")
    bmax = bmax.to(DEV)
    sel = torch.empty((batch, hkv, nsel), dtype=torch.int32, device=DEV)
    out = K.sparse_attention_select(q, k, v, bmax, nsel, block, t, 0.088, sel_out=sel)
    want_sel = K.block_topk(bmax, nsel)
    assert torch.equal(sel, want_sel)
    assert np.array_equal(sel.cpu().numpy().reshape(-1, nsel),
                          O.topk_lowest_index(bmax.cpu().numpy().reshape(-1, nb), nsel))
    want = K.sparse_attention(q, k, v, want_sel, block, t, 0.088)
    assert torch.equal(out, want)


def test_sparse_attention_select_wide_rows_and_reuse():
    # bmax rows wider than the block count (a capacity-sized buffer): values
    # past the last block are never selected; one workspace serves calls of
    # different sizes, with and without sel_out.
    gen = torch.Generator().manual_seed(12)
    b, hkv, g_size, cap = 2, 4, 4, 9000
    q = torch.randn((b, hkv * g_size, 128), generator=gen).to(torch.bfloat16).to(DEV)
    kc = torch.randn((b, hkv, cap, 128), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((b, hkv, cap, 128), generator=gen).to(torch.bfloat16).to(DEV)
    ws = K.attention_workspace(b, hkv * g_size, hkv, 128, 512, 16, DEV)
    for t, nsel in [(8000, 300), (1000, 17), (8999, 512), (33, 2)]:
        nb = -(-t // 16)
        wide = torch.randn((b, hkv, 600), generator=gen).to(DEV)
        wide[..., nb:] = 1e30
        k, v = kc[:, :, :t], vc[:, :, :t]
        sel = torch.empty((b, hkv, nsel), dtype=torch.int32, device=DEV)
        out = K.sparse_attention_select(q, k, v, wide, nsel, 16, t, 0.09, workspace=ws, sel_out=sel)
        out2 = K.sparse_attention_select(q, k, v, wide, nsel, 16, t, 0.09, workspace=ws)
        want_sel = K.block_topk(wide[..., :nb].contiguous(), nsel)
        assert torch.equal(sel, want_sel), t
        assert torch.equal(out, out2)
        want = O.sparse_attention(f32(q), f32(k), f32(v), want_sel.cpu().numpy(), 16, t, 0.09)
        assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL), t
    assert int(ws[:65536].view(torch.int32).abs().sum()) == 0


def test_sparse_attention_select_rejects_long_rows():
    q = torch.randn((1, 8, 128)).to(torch.bfloat16).to(DEV)
    k = torch.randn((1, 2, 4097, 128)).to(torch.bfloat16).to(DEV)
    bmax = torch.randn((1, 2, 4097), device=DEV)
    with pytest.raises(RuntimeError, match="at most 4096 blocks"):
        K.sparse_attention_select(q, k, k, bmax, 16, 1, 4097, 0.1)
    with pytest.raises(RuntimeError, match="n_sel <= blocks"):
        K.sparse_attention_select(q, k[:, :, :64], k[:, :, :64], bmax, 65, 1, 64, 0.1)


def test_sparse_attention_no_valid_block_gives_zero():
    q = torch.randn((1, 2, 128)).to(torch.bfloat16).to(DEV)
    k = torch.randn((1, 1, 64, 128)).to(torch.bfloat16).to(DEV)
    sel = torch.tensor([[[-1, 5, 100]]], dtype=torch.int32, device=DEV)
    out = K.sparse_attention(q, k, k, sel, 16, 64, 0.1)
    assert torch.count_nonzero(out.float()) == 0


def test_sparse_attention_strided_cache():
    # K/V live in a larger-capacity cache; only the first `t` tokens exist.
    gen = torch.Generator().manual_seed(5)
    kc = torch.randn((1, 2, 512, 128), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((1, 2, 512, 128), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((1, 4, 128), generator=gen).to(torch.bfloat16).to(DEV)
    t = 300
    k, v = kc[:, :, :t], vc[:, :, :t]
    sel = torch.tensor([[[0, 3, 18], [1, 2, 17]]], dtype=torch.int32, device=DEV)   # 18*16 > t: partial
    out = K.sparse_attention(q, k, v, sel, 16, t, 0.09)
    want = O.sparse_attention(f32(q), f32(k), f32(v), sel.cpu().numpy(), 16, t, 0.09)
    assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL)


# ---------------------------------------------------------------------------
# config 1 end to end (full size)
# ---------------------------------------------------------------------------

def test_config1_end_to_end():
    cfg = CONFIGS["cfg1"]
    q, k, v, _ = make_layer(cfg, 0)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    cache = K.Int4KCache.from_prefill(kd, cfg.group, cfg.selected)
    step = K.SparseDecodeStep(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.tokens, cfg.block,
                              cfg.topk, DEV)
    out = step(qd, cache, kd, vd, cfg.scaling)
    torch.cuda.synchronize()
    rows = cfg.rows
    kn = f32(k).reshape(rows, cfg.tokens, 128)
    want_p, want_s = O.int4_pack_k(kn, cfg.group)
    assert np.array_equal(cache.packed[:, :, : cfg.tokens].cpu().numpy().reshape(want_p.shape), want_p)
    chan = O.select_channels(O.channel_stats(want_p, want_s, cfg.group), cfg.selected)
    assert np.array_equal(cache.chan_idx.cpu().numpy().reshape(rows, -1), chan)
    slab, sbits = O.build_slab(kn, chan)
    _, _, bmax, sel = O.decode_select(f32(q), slab, sbits, chan, cfg.kv_heads, cfg.block, cfg.topk)
    assert np.array_equal(step.bmax.cpu().numpy().reshape(rows, -1), bmax)
    assert np.array_equal(step.sel.cpu().numpy().reshape(rows, -1), sel)
    want = O.sparse_attention(f32(q), f32(k), f32(v), sel.reshape(cfg.batch, cfg.kv_heads, -1), cfg.block,
                              cfg.tokens, cfg.scaling)
    assert np.allclose(f32(out), want, rtol=RTOL, atol=ATOL)


def _protected_case(g_size, batch, t, block, n_sel, sink, recent, keep_self, mode=None):
    """A decode step with the reference's protected tokens against the oracle:
    the top-k over the history's block maxima bit-exact, the attention over
    the kept blocks plus the sink / recent / current tokens within tolerance."""
    hkv = 8 if g_size < 8 else 4
    hq = hkv * g_size
    g = torch.Generator().manual_seed(t + (n_sel or 0))
    k = rand_k(batch, hkv, t, 128, t)
    v = torch.randn((batch, hkv, t, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((batch, hq, 128), generator=g).to(torch.bfloat16)
    if mode is None:
        step = K.SparseDecodeStep(batch, hq, hkv, 128, t, block, n_sel, DEV, protect_sink=sink,
                                  protect_recent=recent, keep_self=keep_self)
    else:
        step = K.SparseDecodeStep.for_mode(mode, batch, hq, hkv, 128, t, DEV, protect_sink=sink,
                                           protect_recent=recent, keep_self=keep_self)
    channels = step.plan.selected if mode else 32
    cache = K.Int4KCache.from_prefill(k.to(DEV), 32, channels)
    out = step(q.to(DEV), cache, k.to(DEV), v.to(DEV), 128 ** -0.5)
    history = t - 1
    rows = batch * hkv
    kn = f32(k).reshape(rows, t, 128)
    packed, scales = O.int4_pack_k(kn, 32)
    chan = O.select_channels(O.channel_stats(packed, scales, 32), channels)   # chosen over the whole cache
    slab, sbits = O.build_slab(kn[:, :history], chan)                     # the history is what is scored
    _, _, bmax, sel = O.decode_select(f32(q), slab, sbits, chan, hkv, step.block, step.topk)
    assert np.array_equal(step.sel.cpu().numpy().reshape(rows, -1), sel)
    want = O.sparse_attention_protected(f32(q), f32(k), f32(v), sel.reshape(batch, hkv, -1), step.block, history,
                                        128 ** -0.5, sink, recent, keep_self)
    np.testing.assert_allclose(f32(out), want, rtol=RTOL, atol=ATOL)
    return step


@pytest.mark.parametrize("g_size,batch,t,block,n_sel,sink,recent,keep_self", [
    (2, 2, 4097, 16, 64, 4, 8, True),       # fused selection, every kind of protected token
    (4, 1, 2001, 16, 32, 0, 0, True),       # keep the current token only; partial last block
    (1, 1, 1025, 1, 256, 10, 10, True),     # one-token blocks
    (8, 1, 3000, 16, 16, 100, 0, False),    # a long sink that overlaps selected blocks
    (4, 1, 1500, 64, 4, 0, 700, True),      # a recent range over many selected blocks
    (2, 1, 70001, 16, 128, 4, 16, True),    # 4375 blocks: top-k launch, then attention
])
def test_decode_step_protected(g_size, batch, t, block, n_sel, sink, recent, keep_self):
    _protected_case(g_size, batch, t, block, n_sel, sink, recent, keep_self)


def test_decode_step_current_token_only_through_keep_self():
    # the current token is never a candidate (the selection ranks the history,
    # EV:4414-4415) and is attended only with keep_self (EV:2978): give it the
    # highest score and a value of 50, so whether it is attended shows
    batch, hkv, hq, t = 1, 8, 16, 2049
    g = torch.Generator().manual_seed(3)
    k = rand_k(batch, hkv, t, 128, 5)
    v = torch.randn((batch, hkv, t, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((batch, hq, 128), generator=g).to(torch.bfloat16)
    qs = q.float().view(batch, hkv, 2, 128).sum(2)
    k[:, :, t - 1] = (4.0 * qs).to(torch.bfloat16)
    v[:, :, t - 1] = 50.0
    for keep_self in (True, False):
        step = K.SparseDecodeStep(batch, hq, hkv, 128, t, 16, 8, DEV, keep_self=keep_self, history_only=True)
        cache = K.Int4KCache.from_prefill(k.to(DEV), 32, 32)
        out = step(q.to(DEV), cache, k.to(DEV), v.to(DEV), 128 ** -0.5)
        assert (step.sel.cpu() < (t - 1) // 16).all()          # blocks of the history only
        w = O.sparse_attention_protected(f32(q), f32(k), f32(v), step.sel.cpu().numpy(), 16, t - 1, 128 ** -0.5,
                                         0, 0, keep_self)
        np.testing.assert_allclose(f32(out), w, rtol=RTOL, atol=ATOL)
        assert (f32(out).mean() > 40) == keep_self


def test_step_for_reference_mode():
    # qboracle16q32s6p25cand2 at 4097 keys: 4096 history keys, 32 channels,
    # blocks of 16, ceil(6.25% * 4096 / 16) = 16 blocks kept, plus the
    # current token (the reference's default --always_keep_self)
    from kv_cache_amd import modes as M
    mode, t = "qboracle16q32s6p25cand2", 4097
    step = _protected_case(2, 1, t, 16, None, 0, 0, True, mode=mode)
    assert (step.plan.selected, step.block, step.topk, step.scored) == (32, 16, 16, 4096)
    # qabs8cand3attn at 4097 keys: one-token blocks, ceil(3% * 4096) = 123 tokens
    step = _protected_case(2, 1, t, 1, None, 2, 4, True, mode="qabs8cand3attn")
    assert (step.block, step.topk) == (1, 123)
    with pytest.raises(RuntimeError, match="not a decode mode"):
        K.SparseDecodeStep.for_mode("qabs8cand3reuse", 1, 16, 8, 128, t, DEV)
    assert M.decode_plan(mode, t).tokens_kept == 256


def _prefill_rows(n, seed):
    """Rows for the prefill top-k's candidate lists (many rows of 513-1024
    block maxima, k <= 64): i.i.d. rows plus one row of each case the
    selection branches on."""
    g = torch.Generator().manual_seed(seed)
    rows = torch.randn((2048, n), generator=g)
    j = torch.arange(n)
    rows[0] = 2.5                                             # all equal: the list overflows, full-row path
    rows[1] = -float("inf")                                   # nothing selectable
    rows[2] = torch.where(j % 97 == 3, (j % 11).float(), -float("inf"))    # fewer than k finite keys
    rows[3] = torch.where(j < 40 * 16, torch.randn(n, generator=g), -float("inf"))  # < 64 lanes hold keys
    rows[4] = (j % 5).float()                                 # ties at the k-th key
    rows[5] = -1.0 - ((j * 37) % 1000).float()                # negative keys
    rows[6] = torch.where(j % 3 == 0, -0.0, torch.where(j % 3 == 1, 0.0, -1.0))   # -0 and +0 tie
    rows[7] = ((j * 7919) % 300).float() * 0.25               # duplicated values across lanes
    rows[8] = torch.where(j % 16 == 0, 1.0 + j.float(), -float("inf"))   # one key per lane
    rows[9, n - 5:] = -float("inf")                           # a causal tail
    rows[10] = torch.ldexp(torch.ones(n), torch.randint(-30, 30, (n,), generator=g))   # wide exponents
    rows[11] = torch.randint(-3, 3, (n,), generator=g).float()   # 6 values: hundreds of candidates per bin
    return rows


@pytest.mark.parametrize("n", [1024, 1000, 600])
@pytest.mark.parametrize("k", [64, 1, 17])
def test_prefill_topk_candidate_lists(n, k):
    # 2048 rows take the one-wave-per-row kernels; rows of 513-1024 keys with
    # k <= 64 filter each row by its lane-maxima bound into a candidate list
    vals = _prefill_rows(n, n * 7 + k)
    got = P.block_topk(vals.to(DEV), k).cpu().numpy()
    assert np.array_equal(got, O.prefill_block_topk(vals.numpy(), k))
