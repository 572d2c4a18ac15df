"""Pins the int4-path oracle (oracle/qkv_oracle.py) with hand-derived known
answers, closed forms, invariants and brute force on tiny inputs.  The
reference has no int4 code or test vectors, so these checks -- not the
reference -- are what fix the oracle's arithmetic."""

import itertools

import numpy as np
import pytest

from oracle import qkv_oracle as O

# ---------------------------------------------------------------------------
# fp16 scale arithmetic
# ---------------------------------------------------------------------------


def test_fp16_known_bits():
    # 1/7 = 1.001001001001..b x 2^-3; 10 mantissa bits 0010010010, next bit 0
    # -> round down: exponent 12, mantissa 0x092.
    assert O.fp16_bits_rne_sat(np.float32(1.0) / np.float32(7.0)) == 0x3092
    assert O.fp16_bits_rne_sat(np.float32(1.0)) == 0x3C00
    assert O.fp16_bits_rne_sat(np.float32(2.0)) == 0x4000
    # 2^-20 is the fp16 subnormal 16 * 2^-24
    assert O.fp16_bits_rne_sat(np.float32(2.0 ** -20)) == 0x0010
    # below half the smallest subnormal -> 0
    assert O.fp16_bits_rne_sat(np.float32(2.0 ** -26)) == 0
    # overflow saturates to 65504 instead of +inf
    assert O.fp16_bits_rne_sat(np.float32(1.0e6)) == 0x7BFF
    assert O.fp16_bits_rne_sat(np.float32(65504.0)) == 0x7BFF
    # ties to even: 1 + 2^-11 is halfway between 1 and 1 + 2^-10 -> 1
    assert O.fp16_bits_rne_sat(np.float32(1.0 + 2.0 ** -11)) == 0x3C00
    assert O.fp16_bits_rne_sat(np.float32(1.0 + 3 * 2.0 ** -11)) == 0x3C02


def test_fp16_fixed24_closed_form():
    assert O.fp16_fixed24(np.uint16(0x0001)) == 1                    # 2^-24
    assert O.fp16_fixed24(np.uint16(0x3C00)) == 1 << 24              # 1.0
    assert O.fp16_fixed24(np.uint16(0x7BFF)) == 65504 * (1 << 24)    # max finite
    assert O.fp16_fixed24(np.uint16(0x3092)) == 1170 * (1 << 11)     # 1170 * 2^-13 * 2^24


# ---------------------------------------------------------------------------
# int4 quantization and packing
# ---------------------------------------------------------------------------


def test_quantize_known_answers():
    x = np.array([
        [0.0, 0.0, 0.0, 0.0],          # all zero -> scale 0, codes 0
        [7.0, -7.0, 3.5, 0.5],         # scale 1: 3.5 -> 4 (ties to even), 0.5 -> 0
        [14.0, 1.0, -1.0, 2.5],        # scale 2: 0.5 -> 0, -0.5 -> 0, 1.25 -> 1
        [7.0, 2.5, -2.5, 1.5],         # scale 1: 2.5 -> 2, -2.5 -> -2, 1.5 -> 2
        [1.0e6, -1.0e6, 0.0, 1.0],     # scale saturates at 65504: clamp to [-8, 7]
        [7 * 2.0 ** -20, 0, 0, 0],     # subnormal fp16 scale 2^-20
        [2.0 ** -30, 0, 0, 0],         # scale underflows to 0 -> codes 0
    ], dtype=np.float32)
    codes, scale = O.quantize_int4(x, 4)
    assert scale[:, 0].tolist() == [0, 0x3C00, 0x4000, 0x3C00, 0x7BFF, 0x0010, 0]
    assert codes.tolist() == [
        [0, 0, 0, 0],
        [7, -7, 4, 0],
        [7, 0, 0, 1],
        [7, 2, -2, 2],
        [7, -8, 0, 0],
        [7, 0, 0, 0],
        [0, 0, 0, 0],
    ]


def test_quantize_scale_not_power_of_two():
    # amax 1 -> scale fp16(1/7) = 0.142822265625; 1/scale = 7.0017 -> 7;
    # -0.5/scale = -3.5009 -> -4 (not a tie)
    codes, scale = O.quantize_int4(np.array([[1.0, -0.5, 0.25, 0.0]], np.float32), 4)
    assert scale[0, 0] == 0x3092
    assert codes[0].tolist() == [7, -4, 2, 0]


def test_quantize_symmetric_range_and_error_bound():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((64, 128)) * rng.choice([1e-3, 1, 8], size=(64, 1))).astype(np.float32)
    x = x.astype(np.float32)
    codes, scale = O.quantize_int4(x, 32)
    assert codes.min() >= -7 and codes.max() <= 7      # symmetric: -8 never produced
    deq = O.dequantize_int4(O.pack_int4(codes), scale, 32)
    s = np.repeat(O.fp16_bits_to_f32(scale), 32, axis=-1)
    # |x - s*code| <= s/2 up to the relative rounding of the fp16 scale
    assert np.all(np.abs(x - deq) <= 0.5 * s * (1 + 2 ** -9) + 1e-30)
    # the group maximum always maps to +-7
    grp = np.abs(codes.reshape(64, 4, 32)).max(axis=-1)
    assert np.all(grp == 7)


def test_pack_nibble_layout():
    packed = O.pack_int4(np.array([1, -1, 7, -8], np.int8))
    assert packed.tolist() == [0xF1, 0x87]


def test_pack_unpack_exhaustive():
    allbytes = np.arange(256, dtype=np.uint8)
    codes = O.unpack_int4(allbytes)
    for byte in range(256):
        lo, hi = byte & 0xF, byte >> 4
        assert codes[2 * byte] == (lo - 16 if lo >= 8 else lo)
        assert codes[2 * byte + 1] == (hi - 16 if hi >= 8 else hi)
    assert np.array_equal(O.pack_int4(codes), allbytes)


# ---------------------------------------------------------------------------
# Channel statistic and subset
# ---------------------------------------------------------------------------


def test_channel_stats_closed_form():
    k = np.array([[[7.0, 0.0, 0.0, -7.0],       # scale 1 -> codes 7,0,0,-7
                   [0.0, 14.0, -14.0, 0.0]]],   # scale 2 -> codes 0,7,-7,0
                 dtype=np.float32)
    packed, scale = O.int4_pack_k(k, 4)
    stats = O.channel_stats(packed, scale, 4)
    one = 1 << 24
    assert stats.tolist() == [[7 * one, 14 * one, 14 * one, 7 * one]]


def test_channel_stats_matches_python_bigint_sum():
    rng = np.random.default_rng(1)
    k = (rng.standard_normal((3, 37, 64)) * 3).astype(np.float32)
    packed, scale = O.int4_pack_k(k, 32)
    stats = O.channel_stats(packed, scale, 32)
    codes = O.unpack_int4(packed)
    for r in range(3):
        for c in range(64):
            want = 0
            for t in range(37):
                sv = float(np.uint16(scale[r, t, c // 32]).view(np.float16))
                want += abs(int(codes[r, t, c])) * int(round(sv * 2 ** 24))
            assert int(stats[r, c]) == want
    # token order does not matter
    perm = rng.permutation(37)
    assert np.array_equal(O.channel_stats(packed[:, perm], scale[:, perm], 32), stats)


def test_select_channels_ties_and_order():
    st = np.array([[5, 9, 9, 1, 9]], dtype=np.uint64)
    assert O.select_channels(st, 1).tolist() == [[1]]
    assert O.select_channels(st, 2).tolist() == [[1, 2]]
    assert O.select_channels(st, 3).tolist() == [[1, 2, 4]]
    assert O.select_channels(st, 4).tolist() == [[0, 1, 2, 4]]
    big = np.array([[2 ** 63 + 5, 2 ** 63 + 5, 7]], dtype=np.uint64)   # uint64 past int64 range
    assert O.select_channels(big, 1).tolist() == [[0]]


def test_select_channels_brute_force():
    rng = np.random.default_rng(2)
    st = rng.integers(0, 6, size=(20, 32)).astype(np.uint64)
    for s in (1, 5, 16, 32):
        got = O.select_channels(st, s)
        for r in range(20):
            want = sorted(sorted(range(32), key=lambda c: (-int(st[r, c]), c))[:s])
            assert got[r].tolist() == want


def test_build_slab_is_requantized_gather():
    rng = np.random.default_rng(3)
    k = rng.standard_normal((2, 9, 16)).astype(np.float32)
    idx = np.array([[0, 3, 4, 9], [1, 2, 14, 15]], dtype=np.int32)
    slab, sscale = O.build_slab(k, idx)
    want_codes, want_scale = O.quantize_int4(np.take_along_axis(k, idx[:, None, :].astype(np.int64), -1), 4)
    assert np.array_equal(O.unpack_int4(slab), want_codes)
    assert np.array_equal(sscale, want_scale[..., 0])
    # one hand row: channels (0,3,4,9) of [7,..] with amax 7 -> scale 1.0
    k2 = np.zeros((1, 1, 16), np.float32)
    k2[0, 0, [0, 3, 4, 9]] = [7.0, -1.0, 2.5, 0.0]
    k2[0, 0, 5] = 100.0   # not selected: does not enter the slab scale
    slab2, s2 = O.build_slab(k2, idx[:1])
    assert s2.tolist() == [[0x3C00]]
    assert O.unpack_int4(slab2).tolist() == [[[7, -1, 2, 0]]]


# ---------------------------------------------------------------------------
# Query quantization, int32 scores, ranking keys
# ---------------------------------------------------------------------------


def test_query_group_known_answer():
    q = np.array([[[0.0, 1.0, 0.0, 2.0],     # head 0 -> kv head 0
                   [0.0, 3.0, 0.0, -2.0],    # head 1 -> kv head 0
                   [1.0, 0.0, -5.0, 0.0],    # head 2 -> kv head 1
                   [1.0, 0.0, 5.0, 0.0]]], np.float32)
    idx = np.array([[1, 3], [0, 2]], np.int32)
    q8, qs = O.quantize_query_group(q, idx, kv_heads=2)
    # kv0: qg = [4, 0] -> [127, 0];  kv1: qg = [2, 0] -> [127, 0]
    assert q8.tolist() == [[127, 0], [127, 0]]
    assert qs.tolist() == [np.float32(4.0) / np.float32(127.0), np.float32(2.0) / np.float32(127.0)]
    zero, zs = O.quantize_query_group(np.zeros((1, 2, 4), np.float32), idx[:1], kv_heads=1)
    assert zero.tolist() == [[0, 0]] and zs.tolist() == [0.0]


def test_query_group_sum_matches_per_head_sum():
    # The group-summed query equals the sum of the per-head queries, so the
    # dequantized score approximates sum_h q_h . k (the GQA-summed score).
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 8, 64)).astype(np.float32)
    k = rng.standard_normal((2 * 2, 50, 64)).astype(np.float32)
    idx = np.sort(rng.permutation(64)[:32])[None].repeat(4, 0).astype(np.int32)
    q8, qs = O.quantize_query_group(q, idx, kv_heads=2)
    slab, ss = O.build_slab(k, idx)
    approx = O.partial_scores_i32(q8, slab) * qs[:, None] * O.fp16_bits_to_f32(ss)
    exact = np.einsum("bjgs,bjts->bjt", np.take_along_axis(q.reshape(2, 2, 4, 64), idx.reshape(2, 2, 1, 32).astype(np.int64), -1),
                      np.take_along_axis(k.reshape(2, 2, 50, 64), idx.reshape(2, 2, 1, 32).astype(np.int64), -1)).reshape(4, 50)
    assert np.corrcoef(approx.ravel(), exact.ravel())[0, 1] > 0.99


def test_scores_brute_force_and_key():
    rng = np.random.default_rng(5)
    q8 = rng.integers(-127, 128, size=(3, 16)).astype(np.int8)
    codes = rng.integers(-8, 8, size=(3, 11, 16)).astype(np.int8)
    slab = O.pack_int4(codes)
    got = O.partial_scores_i32(q8, slab)
    for r, t in itertools.product(range(3), range(11)):
        assert got[r, t] == sum(int(q8[r, s]) * int(codes[r, t, s]) for s in range(16))
    # known answer: q8 [127, 0] . [7, -8] = 889
    assert O.partial_scores_i32(np.array([[127, 0]], np.int8), O.pack_int4(np.array([[[7, -8]]], np.int8))).tolist() == [[889]]
    key = O.ranking_keys(np.array([[-889, 0, 3]], np.int32), np.array([[0x4000, 0x0000, 0x3092]], np.uint16))
    assert key[0, 0] == np.float32(-1778.0)
    assert key[0, 1] == 0.0 and not np.signbit(key[0, 1])
    assert key[0, 2] == np.float32(np.float32(0.142822265625) * np.float32(3.0))


def test_zero_scale_key_is_positive_zero():
    key = O.ranking_keys(np.array([[-5]], np.int32), np.array([[0]], np.uint16))
    assert key[0, 0] == 0.0 and not np.signbit(key[0, 0])


# ---------------------------------------------------------------------------
# Block max, top-k
# ---------------------------------------------------------------------------


def test_block_max_known_answer():
    v = np.array([[1, 5, 2, 7, 3]], np.float32)
    assert O.block_max(v, 2).tolist() == [[5, 7, 3]]
    assert O.block_max(v, 1).tolist() == v.tolist()
    assert O.block_max(v, 8).tolist() == [[7]]


def test_topk_ties_lowest_index_ascending():
    v = np.array([[3, 5, 5, 1, 5]], np.float32)
    assert O.topk_lowest_index(v, 1).tolist() == [[1]]
    assert O.topk_lowest_index(v, 2).tolist() == [[1, 2]]
    assert O.topk_lowest_index(v, 3).tolist() == [[1, 2, 4]]
    assert O.topk_lowest_index(v, 4).tolist() == [[0, 1, 2, 4]]
    assert O.topk_lowest_index(v, 5).tolist() == [[0, 1, 2, 3, 4]]
    z = np.array([[0.0, -0.0, 0.0, -1.0]], np.float32)   # -0 == +0
    assert O.topk_lowest_index(z, 2).tolist() == [[0, 1]]
    ninf = np.array([[-np.inf, -np.inf, -5.0]], np.float32)
    assert O.topk_lowest_index(ninf, 2).tolist() == [[0, 2]]


def test_topk_brute_force():
    rng = np.random.default_rng(6)
    v = rng.integers(-4, 4, size=(30, 40)).astype(np.float32)
    for k in (1, 7, 20, 40):
        got = O.topk_lowest_index(v, k)
        for r in range(30):
            want = sorted(sorted(range(40), key=lambda i: (-v[r, i], i))[:k])
            assert got[r].tolist() == want


def test_expand_blocks():
    toks = O.expand_blocks(np.array([[0, 2, -1, 9]]), 4, 10)
    assert toks[0].tolist() == [0, 1, 2, 3, 8, 9]


# ---------------------------------------------------------------------------
# Sparse attention
# ---------------------------------------------------------------------------


def test_attention_closed_forms():
    rng = np.random.default_rng(7)
    k = rng.standard_normal((1, 1, 8, 4))
    v = rng.standard_normal((1, 1, 8, 4))
    q = rng.standard_normal((1, 2, 4))
    # one token: output is that token's value row, for every head
    out = O.sparse_attention(q, k, v, np.array([[[5]]]), 1, 8, 0.5)
    assert np.allclose(out[0], v[0, 0, 5])
    # zero query: uniform weights -> mean of the selected values
    out = O.sparse_attention(np.zeros((1, 2, 4)), k, v, np.array([[[0, 3]]]), 2, 8, 1.0)
    assert np.allclose(out[0, 0], v[0, 0, [0, 1, 6, 7]].mean(0))
    # no valid block -> zeros
    out = O.sparse_attention(q, k, v, np.array([[[-1, 99]]]), 2, 8, 1.0)
    assert np.all(out == 0)
    # partial tail block: tokens past T are not attended
    out = O.sparse_attention(np.zeros((1, 2, 4)), k, v, np.array([[[1]]]), 4, 6, 1.0)
    assert np.allclose(out[0, 1], v[0, 0, [4, 5]].mean(0))


def test_attention_matches_dense_softmax():
    rng = np.random.default_rng(8)
    b, hq, hkv, t, d = 2, 4, 2, 20, 8
    q = rng.standard_normal((b, hq, d))
    k = rng.standard_normal((b, hkv, t, d))
    v = rng.standard_normal((b, hkv, t, d))
    sel = np.tile(np.arange(5), (b, hkv, 1))    # all tokens, block 4
    out = O.sparse_attention(q, k, v, sel, 4, t, 0.3)
    for bi, h in itertools.product(range(b), range(hq)):
        s = k[bi, h // 2] @ q[bi, h] * 0.3
        w = np.exp(s - s.max())
        w /= w.sum()
        assert np.allclose(out[bi, h], w @ v[bi, h // 2])


def test_protected_tokens_known_answers():
    # history 10: sink 2 -> 0, 1; recent 3 -> 7, 8, 9; self -> 10
    assert O.protected_tokens(10, 2, 3, True).tolist() == [0, 1, 7, 8, 9, 10]
    # a recent range reaching into the sink keeps each token once
    assert O.protected_tokens(4, 3, 3, False).tolist() == [0, 1, 2, 3]
    assert O.protected_tokens(5, 0, 0, True).tolist() == [5]
    assert O.protected_tokens(5, 9, 0, False).tolist() == [0, 1, 2, 3, 4]
    assert O.protected_tokens(5, 0, 0, False).size == 0


def test_protected_tokens_match_reference_index_build():
    # the valid entries of the reference's own final index build
    # (ref_semantics.final_indices_from_selected, EV:2938-2982, pinned by the
    # reference's qabs-attn vectors) are the selection plus protected_tokens
    import torch

    from oracle import ref_semantics as R

    rng = np.random.default_rng(11)
    for history, sink, recent, keep_self in [(40, 4, 6, True), (40, 0, 0, True), (12, 8, 8, False),
                                             (25, 0, 5, True), (25, 3, 0, False)]:
        sel = np.sort(rng.choice(history, size=7, replace=False))
        idx, valid = R.final_indices_from_selected(torch.from_numpy(sel).view(1, 1, -1),
                                                   torch.ones((1, 1, 7), dtype=torch.bool), history, history + 1,
                                                   sink, recent, keep_self)
        got = idx[valid].numpy()
        assert got.size == np.unique(got).size                       # every token once
        assert np.array_equal(np.sort(got), np.union1d(sel, O.protected_tokens(history, sink, recent, keep_self)))


def test_protected_attention_closed_forms():
    rng = np.random.default_rng(12)
    b, hq, hkv, t, d = 1, 4, 2, 33, 8                  # history 32 + the current token
    q = rng.standard_normal((b, hq, d))
    k = rng.standard_normal((b, hkv, t, d))
    v = rng.standard_normal((b, hkv, t, d))
    # every history block selected + protected ranges + self == dense softmax
    # over all 33 tokens (a protected token counted twice would not be)
    all_blocks = np.tile(np.arange(8), (b, hkv, 1))
    out = O.sparse_attention_protected(q, k, v, all_blocks, 4, 32, 0.3, sink=3, recent=5, keep_self=True)
    for h in range(hq):
        s = k[0, h // 2] @ q[0, h] * 0.3
        w = np.exp(s - s.max())
        assert np.allclose(out[0, h], (w / w.sum()) @ v[0, h // 2])
    # nothing selected, no sink / recent, keep_self: the current token's value
    out = O.sparse_attention_protected(q, k, v, np.full((b, hkv, 1), -1), 4, 32, 0.3, keep_self=True)
    assert np.allclose(out[0], v[0, np.arange(hq) // 2, 32])
    # one selected block overlapping the sink: tokens 0..3 with sink 2 -> {0, 1, 2, 3} once
    out = O.sparse_attention_protected(np.zeros((b, hq, d)), k, v, np.zeros((b, hkv, 1), int), 4, 32, 1.0, sink=2)
    assert np.allclose(out[0, 0], v[0, 0, :4].mean(0))


# ---------------------------------------------------------------------------
# Prefill scoring
# ---------------------------------------------------------------------------


def test_prefill_scores_brute_force():
    rng = np.random.default_rng(9)
    b, hq, hkv, nq, t, d, bs = 1, 4, 2, 5, 24, 16, 4
    q8 = rng.integers(-127, 128, size=(b, hq, nq, d)).astype(np.int8)
    codes = rng.integers(-7, 8, size=(b, hkv, t, d)).astype(np.int8)
    kp = O.pack_int4(codes)
    ks = O.fp16_bits_rne_sat(rng.uniform(0.01, 2, size=(b, hkv, t)).astype(np.float32))
    pos0 = t - nq
    got = O.prefill_block_scores(q8, kp, ks, bs, pos0)
    for h, i in itertools.product(range(hq), range(nq)):
        p = pos0 + i
        for j in range(t // bs):
            vals = []
            for tt in range(j * bs, (j + 1) * bs):
                if tt <= p:
                    isum = sum(int(q8[0, h, i, c]) * int(codes[0, h // 2, tt, c]) for c in range(d))
                    vals.append(np.float32(O.fp16_bits_to_f32(ks[0, h // 2, tt])) * np.float32(isum))
            want = max(vals) if vals else -np.inf
            assert got[0, h, i, j] == np.float32(want)


def test_prefill_topk_pads_invisible_blocks():
    bmax = np.array([[3.0, -np.inf, -np.inf], [1.0, 2.0, -np.inf]], np.float32)
    assert O.prefill_block_topk(bmax, 2).tolist() == [[0, -1], [0, 1]]


def test_query_rows_quantization():
    q8, qs = O.quantize_query_rows(np.array([[1.0, -2.0, 0.5, 0.0]], np.float32))
    assert q8.tolist() == [[64, -127, 32, 0]]   # 1/(2/127) = 63.5 -> 64 (ties to even), 0.5 -> 31.75 -> 32
    assert qs.tolist() == [np.float32(2.0) / np.float32(127.0)]


def test_recall_at():
    assert O.recall_at([np.array([1, 5]), np.array([2])], np.array([5, 3])) == 0.5


@pytest.mark.parametrize("group", [32, 64, 128])
def test_pack_roundtrip_groups(group):
    rng = np.random.default_rng(group)
    k = rng.standard_normal((2, 3, 128)).astype(np.float32)
    packed, scale = O.int4_pack_k(k, group)
    assert packed.shape == (2, 3, 64) and scale.shape == (2, 3, 128 // group)
    deq = O.dequantize_int4(packed, scale, group)
    s = np.repeat(O.fp16_bits_to_f32(scale), group, axis=-1)
    assert np.all(np.abs(deq - k) <= 0.5 * s * (1 + 2 ** -9))


# ---------------------------------------------------------------------------
# slab storage swizzle
# ---------------------------------------------------------------------------

def test_slab_swizzle_known_positions():
    # S = 32: 4 keys of 16 bytes per lane; lane l owns keys 4l..4l+3
    off = lambda t, x: int(O.slab_storage_offset(t, x, 32))  # noqa: E731
    assert [off(0, x) for x in (0, 15)] == [0, 15]
    assert off(1, 0) == 1024          # key 1 = lane 0's second 16-byte chunk
    assert off(4, 3) == 16 + 3        # key 4 = lane 1's first chunk
    assert off(255, 15) == (64 * 3 + 63) * 16 + 15
    assert off(256, 0) == 4096        # next tile
    # S = 128: one key of 64 bytes per lane
    assert int(O.slab_storage_offset(5, 17, 128)) == (64 * 1 + 5) * 16 + 1
    # S = 16: 8 keys of 8 bytes per lane
    assert int(O.slab_storage_offset(9, 2, 16)) == (64 * 0 + 1) * 16 + 8 + 2


@pytest.mark.parametrize("sel", [16, 32, 64, 128])
def test_slab_swizzle_is_a_permutation_per_tile(sel):
    cap = O.slab_tile_keys(sel) * 2
    t, x = np.meshgrid(np.arange(cap), np.arange(sel // 2), indexing="ij")
    off = O.slab_storage_offset(t, x, sel).reshape(-1)
    assert np.array_equal(np.sort(off), np.arange(cap * sel // 2))
    # each lane's four loads of one tile are 16-byte chunks 64j + l
    k = np.arange(O.slab_tile_keys(sel))
    first = O.slab_storage_offset(k, 0, sel) // 16
    assert np.array_equal(np.unique(first % 64), np.arange(64))


@pytest.mark.parametrize("sel", [16, 32, 64, 128])
def test_slab_swizzle_round_trip(sel):
    rng = np.random.default_rng(sel)
    t = 777
    cap = -(-t // 512) * 512
    slab = rng.integers(0, 256, size=(3, t, sel // 2), dtype=np.uint8)
    stored = O.swizzle_slab(slab, cap)
    assert stored.shape == (3, cap * sel // 2)
    assert np.array_equal(O.unswizzle_slab(stored, sel, t), slab)
    assert int(stored.astype(np.int64).sum()) == int(slab.astype(np.int64).sum())


def test_pack_query_words_layout():
    q8 = np.arange(-8, 8, dtype=np.int8).reshape(1, 16)        # channel c holds c - 8
    w = O.pack_query_words(q8)
    assert w.shape == (1, 4) and w.dtype == np.uint32
    b = w.view(np.uint8).view(np.int8).reshape(-1).tolist()
    # word 0: even channels 0,2,4,6; word 1: odd channels 1,3,5,7; then 8..15
    assert b == [-8, -6, -4, -2, -7, -5, -3, -1, 0, 2, 4, 6, 1, 3, 5, 7]


def test_prefill_query_slot_layout():
    slot = O.prefill_query_slot(np.arange(128))
    assert np.array_equal(np.sort(slot), np.arange(128))            # a permutation
    # channels 0..15 (group 0, half 0): even channels of 0..7, odd of 0..7, then 8..15
    assert slot[:16].tolist() == [0, 4, 1, 5, 2, 6, 3, 7, 8, 12, 9, 13, 10, 14, 11, 15]
    assert slot[16] == 16 and slot[32] == 32 and slot[127] == 127
    q = np.arange(-64, 64, dtype=np.int8)
    perm = O.permute_prefill_query(q)
    assert perm[slot[5]] == q[5] and perm[1] == q[2]
