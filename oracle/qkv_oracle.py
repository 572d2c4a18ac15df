"""CPU oracle for the int4 sparse-attention KV-retrieval path (numpy).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product path (``kv_cache_amd``) never calls it and fails loudly
when its HIP library is missing.

The reference (littlexi001/kv_cache) has no int4, int32, static-channel,
GQA-grouped or prefill-scoring code: its partial scores are fp32 over
GQA-expanded bf16 K (ymluo/projects/qwen3_top2_head_limit3_ppl/src/
qabs_cuda_kernels.py:63-158, evaluate_qwen3_top2_head_limit3_ppl.py:2563-2570).
The functions below are therefore the written specification of those parts,
restated as the simplest numpy expressions.  Each is pinned in
``tests/test_oracle_*.py`` by hand-derived known answers, closed forms,
invariants and brute force on tiny inputs.  Citations of the nearest
reference code are given per function ("EV" = evaluate_qwen3_top2_head_limit3
_ppl.py, "QK" = qabs_cuda_kernels.py, both under
ymluo/projects/qwen3_top2_head_limit3_ppl/src/).

Conventions: bf16 tensors are passed as float32 arrays holding bf16-exact
values; fp16 scales are passed as their uint16 bit patterns; rows are
(batch, kv_head) pairs flattened as ``r = b * Hkv + j``; query head ``h``
belongs to KV head ``h // G`` (the ``repeat_interleave`` grouping of
EV:6248-6251).
"""

from __future__ import annotations

import numpy as np

FP16_MAX_BITS = np.uint16(0x7BFF)  # 65504.0, the largest finite fp16
INT4_MIN, INT4_MAX = -8, 7
Q8_MAX = 127
# T limit for the exact uint64 channel statistic: |code| <= 8, F(scale) < 2**40.
CHANNEL_STAT_MAX_TOKENS = 1 << 20


def _f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


# ---------------------------------------------------------------------------
# fp16 helpers
# ---------------------------------------------------------------------------

def fp16_bits_rne_sat(x) -> np.ndarray:
    """fp32 -> fp16 bit pattern, round-to-nearest-even, +inf saturated to 65504.

    Inputs are non-negative magnitudes (a group max divided by 7), so only the
    positive overflow needs saturating.
    """
    with np.errstate(over="ignore"):
        h = _f32(x).astype(np.float16)
    bits = np.array(h.view(np.uint16), copy=True)
    bits[np.isposinf(h)] = FP16_MAX_BITS
    return bits


def fp16_bits_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def fp16_fixed24(bits) -> np.ndarray:
    """Exact integer value of an fp16 times 2**24 (every finite fp16 is a
    multiple of 2**-24), as uint64.  Used by the order-free channel statistic."""
    v = np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)
    return (v * float(1 << 24)).astype(np.uint64)


# ---------------------------------------------------------------------------
# int4 quantize / pack  (no reference code; nearest layout precedent is the
# auxiliary dim-major K copy, EV:2018-2042)
# ---------------------------------------------------------------------------

def quantize_int4(x, group: int) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int4 quantization of the last axis in groups of ``group``.

    Per group: ``amax = max|x|`` (fp32, exact); ``scale = fp16_rne(amax / 7)``
    with an IEEE fp32 division, saturated at 65504; ``code = clamp(rint_even(
    x / float(scale)), -8, 7)`` with an IEEE fp32 division; ``scale == 0`` gives
    code 0.  Returns (codes int8 [..., C], scale bits uint16 [..., C // group]).
    """
    x = _f32(x)
    c = x.shape[-1]
    if c % group:
        raise ValueError("channel count must be a multiple of the group size")
    xg = x.reshape(*x.shape[:-1], c // group, group)
    amax = np.abs(xg).max(axis=-1)
    scale_bits = fp16_bits_rne_sat(amax / np.float32(7.0))
    scale = fp16_bits_to_f32(scale_bits)
    safe = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    code = np.rint(xg / safe[..., None])
    code = np.clip(code, INT4_MIN, INT4_MAX)
    code = np.where(scale[..., None] == 0, np.float32(0.0), code)
    return code.astype(np.int8).reshape(x.shape), scale_bits


def pack_int4(codes) -> np.ndarray:
    """Two's-complement nibbles; byte i holds channel 2i (low) and 2i+1 (high)."""
    c = np.asarray(codes).astype(np.int16) & 0xF
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8).astype(np.int16)
    lo = p & 0xF
    hi = (p >> 4) & 0xF
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty((*p.shape[:-1], p.shape[-1] * 2), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def int4_pack_k(k, group: int) -> tuple[np.ndarray, np.ndarray]:
    """K [..., T, D] -> (packed uint8 [..., T, D/2], scale bits uint16 [..., T, D/group])."""
    codes, scale_bits = quantize_int4(k, group)
    return pack_int4(codes), scale_bits


def dequantize_int4(packed, scale_bits, group: int) -> np.ndarray:
    codes = unpack_int4(packed).astype(np.float32)
    scale = np.repeat(fp16_bits_to_f32(scale_bits), group, axis=-1)
    return codes * scale


# ---------------------------------------------------------------------------
# Static channel subset per KV head  (reference: dynamic top-|q| per query
# head, EV:4428 / QK:123-145; the configs ask for the S channels with the
# largest mean |K| per KV head, which has no reference code)
# ---------------------------------------------------------------------------

def channel_stats(packed, scale_bits, group: int) -> np.ndarray:
    """stat[r, c] = sum_t |code[r, t, c]| * F(scale[r, t, c // group]), uint64, exact.

    F(s) = s * 2**24 is an integer for every fp16 s, so the sum is an exact,
    order-free integer: proportional to the mean |dequantized K| of channel c.
    packed: uint8 [R, T, D/2]; scale_bits: uint16 [R, T, D/group].
    """
    codes = unpack_int4(packed)
    t = codes.shape[-2]
    if t > CHANNEL_STAT_MAX_TOKENS:
        raise ValueError("channel statistic is exact only up to 2**20 tokens")
    fixed = np.repeat(fp16_fixed24(scale_bits), group, axis=-1)
    mag = np.abs(codes.astype(np.int16)).astype(np.uint64)
    return (mag * fixed).sum(axis=-2, dtype=np.uint64)


def select_channels(stats, count: int) -> np.ndarray:
    """The ``count`` channels with the largest statistic, ties to the lower
    channel, returned in ascending channel order (int32 [..., count])."""
    stats = np.asarray(stats, dtype=np.uint64)
    order = np.argsort(~stats, axis=-1, kind="stable")  # ~x reverses uint64 order
    return np.sort(order[..., :count], axis=-1).astype(np.int32)


def build_slab(k, chan_idx) -> tuple[np.ndarray, np.ndarray]:
    """Subset slab: the selected channels of every token re-quantized as one
    int4 group of S channels.

    k: [R, T, D] (bf16-exact f32); chan_idx: int32 [R, S] ascending.
    Returns (slab uint8 [R, T, S/2], slab scale bits uint16 [R, T]) in logical
    key order; the device stores the codes swizzled (``swizzle_slab``) and the
    scales in key order.  The reference keeps a transposed bf16 copy of K for
    its scoring kernel (EV:2018-2042); this is the int4 analogue with the
    channel gather folded in.
    """
    k = _f32(k)
    idx = np.asarray(chan_idx, dtype=np.int64)
    gathered = np.take_along_axis(k, idx[:, None, :], axis=-1)  # [R, T, S]
    s = gathered.shape[-1]
    codes, scale_bits = quantize_int4(gathered, s)
    return pack_int4(codes), scale_bits[..., 0]


def slab_tile_keys(selected: int) -> int:
    """Keys per 4096-byte slab tile: 64 lanes x 64 bytes of S/2-byte codes."""
    return 8192 // selected


def slab_storage_offset(t, x, selected: int):
    """Storage byte offset, within a row's slab, of logical code byte ``x`` of
    key ``t`` (the swizzle that lets a 64-lane wave read whole keys per lane
    with coalesced 16-byte loads).

    Tile = t // (8192/S); lane = (t % (8192/S)) // (128/S) owns 128/S
    consecutive keys = 64 logical bytes; its logical byte b = (t % (128/S)) *
    S/2 + x is stored at tile * 4096 + (64 * (b // 16) + lane) * 16 + b % 16.
    """
    t = np.asarray(t, dtype=np.int64)
    x = np.asarray(x, dtype=np.int64)
    kpln = 128 // selected
    tk = slab_tile_keys(selected)
    tile, k = np.divmod(t, tk)
    lane, e = np.divmod(k, kpln)
    b = e * (selected // 2) + x
    return tile * 4096 + (64 * (b // 16) + lane) * 16 + b % 16


def swizzle_slab(slab, capacity: int) -> np.ndarray:
    """Logical slab uint8 [R, T, S/2] -> stored bytes uint8 [R, capacity * S/2]
    (positions past T stay zero); capacity is a multiple of the tile."""
    slab = np.asarray(slab, dtype=np.uint8)
    r, t, half = slab.shape
    sel = 2 * half
    if capacity % slab_tile_keys(sel) or capacity < t:
        raise ValueError("capacity must be a multiple of the slab tile and hold every key")
    out = np.zeros((r, capacity * half), dtype=np.uint8)
    tt, xx = np.meshgrid(np.arange(t), np.arange(half), indexing="ij")
    off = slab_storage_offset(tt, xx, sel)
    out[:, off.reshape(-1)] = slab.reshape(r, -1)
    return out


def unswizzle_slab(stored, selected: int, tokens: int) -> np.ndarray:
    """Inverse of ``swizzle_slab``: stored bytes [R, >= cap * S/2] -> [R, T, S/2]."""
    stored = np.asarray(stored, dtype=np.uint8)
    r = stored.shape[0]
    flat = stored.reshape(r, -1)
    half = selected // 2
    tt, xx = np.meshgrid(np.arange(tokens), np.arange(half), indexing="ij")
    off = slab_storage_offset(tt, xx, selected)
    return flat[:, off.reshape(-1)].reshape(r, tokens, half)


# ---------------------------------------------------------------------------
# Decode-step query quantization and int32 scoring
# (reference fp32 scoring: QK:63-96 dim-major, QK:98-158 token-major,
#  fallback EV:4443-4446)
# ---------------------------------------------------------------------------

def quantize_query_group(q, chan_idx, kv_heads: int) -> tuple[np.ndarray, np.ndarray]:
    """GQA-grouped int8 query over the KV head's channel subset.

    q: [B, Hq, D] (bf16-exact f32); chan_idx: int32 [B*Hkv, S].
    qg[s] = sum over the G query heads of the group of q[h, idx[s]], summed in
    fp32 in head order; ``qscale = amax(|qg|) / 127`` (IEEE fp32 division);
    ``q8 = clamp(rint_even(qg / qscale), -127, 127)``, zero when qscale == 0.
    Returns (q8 int8 [B*Hkv, S], qscale f32 [B*Hkv]).
    """
    q = _f32(q)
    b, hq, d = q.shape
    g = hq // kv_heads
    idx = np.asarray(chan_idx, dtype=np.int64).reshape(b, kv_heads, -1)
    qh = q.reshape(b, kv_heads, g, d)
    acc = np.zeros(idx.shape, dtype=np.float32)
    for i in range(g):
        acc = (acc + np.take_along_axis(qh[:, :, i, :], idx, axis=-1)).astype(np.float32)
    amax = np.abs(acc).max(axis=-1)
    qscale = (amax / np.float32(Q8_MAX)).astype(np.float32)
    safe = np.where(qscale == 0, np.float32(1.0), qscale).astype(np.float32)
    q8 = np.clip(np.rint(acc / safe[..., None]), -Q8_MAX, Q8_MAX)
    q8 = np.where(qscale[..., None] == 0, np.float32(0.0), q8)
    return q8.astype(np.int8).reshape(b * kv_heads, -1), qscale.reshape(-1)


def pack_query_words(q8) -> np.ndarray:
    """int8 query [R, S] -> uint32 words [R, S/4] in the order the int4 code
    dwords pair with: word 2d holds channels 8d, 8d+2, 8d+4, 8d+6 (bytes 0..3),
    word 2d+1 channels 8d+1, 8d+3, 8d+5, 8d+7."""
    q = np.asarray(q8, dtype=np.int8).view(np.uint8)
    r, s = q.shape
    g = q.reshape(r, s // 8, 4, 2)                            # [R, d, pair, parity]
    ordered = np.ascontiguousarray(g.transpose(0, 1, 3, 2))   # [R, d, parity, pair]
    return ordered.reshape(r, s).view("<u4").reshape(r, s // 4)


def partial_scores_i32(q8, slab) -> np.ndarray:
    """I[r, t] = sum_s q8[r, s] * code[r, t, s]  (exact int32)."""
    codes = unpack_int4(slab).astype(np.int64)
    q = np.asarray(q8, dtype=np.int64)
    return np.einsum("rts,rs->rt", codes, q).astype(np.int32)


def ranking_keys(scores_i32, slab_scale_bits) -> np.ndarray:
    """key = fp32(scale) * fp32(I): one IEEE fp32 multiply, -0 folded to +0.

    |I| <= 127 * 8 * 128 < 2**24 so fp32(I) is exact; the query scale is a
    common positive factor of a row and is left out of the ranking key.
    """
    scale = fp16_bits_to_f32(slab_scale_bits)
    key = (scale * np.asarray(scores_i32).astype(np.float32)).astype(np.float32)
    return np.where(key == 0, np.float32(0.0), key).astype(np.float32)


def block_max(keys, block: int) -> np.ndarray:
    """bmax[r, j] = max over tokens [j*block, min(T, (j+1)*block)) -- the
    reference pads with -inf and takes ``amax`` (EV:5038-5044)."""
    keys = _f32(keys)
    t = keys.shape[-1]
    nb = -(-t // block)
    pad = nb * block - t
    if pad:
        fill = np.full((*keys.shape[:-1], pad), -np.inf, dtype=np.float32)
        keys = np.concatenate([keys, fill], axis=-1)
    return keys.reshape(*keys.shape[:-1], nb, block).max(axis=-1)


def topk_lowest_index(values, k: int) -> np.ndarray:
    """Indices of the k largest values of each row, ties to the lower index,
    returned in ascending index order (int32 [R, k]).

    The reference uses ``torch.topk`` (EV:4448, 5046), whose tie order is
    unspecified; this build fixes the lowest-index rule.
    """
    values = _f32(values)
    rows = values.reshape(-1, values.shape[-1])
    n = rows.shape[-1]
    if not 1 <= k <= n:
        raise ValueError("k must be in [1, n]")
    pos = np.arange(n)
    out = np.empty((rows.shape[0], k), dtype=np.int32)
    for r in range(rows.shape[0]):
        order = np.lexsort((pos, -rows[r]))
        out[r] = np.sort(order[:k])
    return out.reshape(*values.shape[:-1], k)


def expand_blocks(block_ids, block: int, tokens: int) -> list[np.ndarray]:
    """Token ids covered by each row's selected blocks (ascending); ids < 0 or
    past the last block are skipped.  Reference block expansion: EV:2914-2922."""
    ids = np.asarray(block_ids).reshape(-1, np.asarray(block_ids).shape[-1])
    nb = -(-tokens // block)
    out = []
    for row in ids:
        toks = [np.arange(j * block, min(tokens, (j + 1) * block)) for j in row if 0 <= j < nb]
        out.append(np.concatenate(toks) if toks else np.zeros(0, dtype=np.int64))
    return out


# ---------------------------------------------------------------------------
# Sparse gather attention, GQA-native  (reference kernel QK:335-419,
# fallback EV:4612-4647)
# ---------------------------------------------------------------------------

def sparse_attention(q, k, v, block_ids, block: int, tokens: int, scaling: float) -> np.ndarray:
    """fp64 softmax attention of every query head over the union of its KV
    head's selected blocks.

    q: [B, Hq, D]; k, v: [B, Hkv, Tcap, D]; block_ids: [B, Hkv, n] (invalid ids
    skipped); only tokens < ``tokens`` exist.  A row with no valid token
    outputs zeros (QK:388, 404).  Returns float64 [B, Hq, D].
    """
    return _attend(q, k, v, expand_blocks(block_ids, block, tokens), scaling)


def protected_tokens(history: int, sink: int, recent: int, keep_self: bool) -> np.ndarray:
    """The tokens every reference selection adds (EV:2938-2982): the sink
    range [0, min(sink, history)), the recent range [max(0, history - recent),
    history) without the sink's tokens, and the current token ``history``."""
    sink_end = min(sink, history) if sink > 0 else 0
    recent_start = max(0, history - recent) if recent > 0 else history
    parts = [np.arange(sink_end), np.arange(max(recent_start, sink_end), history)]
    if keep_self:
        parts.append(np.array([history]))
    return np.concatenate(parts).astype(np.int64)


def sparse_attention_protected(q, k, v, block_ids, block: int, history: int, scaling: float, sink: int = 0,
                               recent: int = 0, keep_self: bool = False) -> np.ndarray:
    """``sparse_attention`` over the selected blocks of the history [0,
    history) together with the protected tokens, every token once (the
    reference masks selected tokens that fall in the protected ranges,
    EV:2946-2953).  Returns float64 [B, Hq, D]."""
    prot = protected_tokens(history, sink, recent, keep_self)
    toks = [np.union1d(t, prot) for t in expand_blocks(block_ids, block, history)]
    return _attend(q, k, v, toks, scaling)


def _attend(q, k, v, toks, scaling: float) -> np.ndarray:
    """fp64 softmax attention of each row's G query heads over its token list."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros((b, hq, d), dtype=np.float64)
    for bi in range(b):
        for j in range(hkv):
            t = toks[bi * hkv + j]
            if t.size == 0:
                continue
            kk = k[bi, j, t]
            vv = v[bi, j, t]
            for i in range(g):
                h = j * g + i
                s = kk @ q[bi, h] * scaling
                p = np.exp(s - s.max())
                out[bi, h] = (p / p.sum()) @ vv
    return out


# ---------------------------------------------------------------------------
# Chunked-prefill scoring as a dense contraction (no reference code; prefill
# is dense HF attention, EV:7079-7111, dense QK EV:6602-6604)
# ---------------------------------------------------------------------------

def quantize_query_rows(q) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8 over all D channels: q [..., D] -> (q8, qscale)."""
    q = _f32(q)
    amax = np.abs(q).max(axis=-1)
    qscale = (amax / np.float32(Q8_MAX)).astype(np.float32)
    safe = np.where(qscale == 0, np.float32(1.0), qscale).astype(np.float32)
    q8 = np.clip(np.rint(q / safe[..., None]), -Q8_MAX, Q8_MAX)
    q8 = np.where(qscale[..., None] == 0, np.float32(0.0), q8)
    return q8.astype(np.int8), qscale


def prefill_query_slot(c):
    """Byte position of channel c in a permuted 128-channel prefill query row:
    32*(c/32) + 16*((c/16)%2) + 8*((c%16)/8) + 4*(c%2) + (c%8)/2 (the order in
    which the MFMA scoring kernel's unpacked K bytes list channels)."""
    c = np.asarray(c, dtype=np.int64)
    c16 = c % 16
    return 32 * (c // 32) + 16 * ((c // 16) % 2) + 8 * (c16 // 8) + 4 * (c16 % 2) + (c16 % 8) // 2


def permute_prefill_query(q8) -> np.ndarray:
    """int8 [..., 128] logical channel order -> the device's permuted order."""
    q8 = np.asarray(q8, dtype=np.int8)
    out = np.empty_like(q8)
    out[..., prefill_query_slot(np.arange(128))] = q8
    return out


def prefill_block_scores(q8, kpacked, kscale_bits, block: int, q_pos0: int) -> np.ndarray:
    """Block-max ranking keys of a query chunk against the whole packed K.

    q8: int8 [B, Hq, Nq, D]; kpacked: uint8 [B, Hkv, T, D/2] (one scale per
    token, i.e. packed with group D); kscale_bits: uint16 [B, Hkv, T].
    Query i sits at absolute position q_pos0 + i and sees keys t <= that
    position (causal).  key = fp32(kscale) * fp32(I) with I the exact int32
    dot over D; invisible keys are -inf; returns bmax f32 [B, Hq, Nq, nb].
    """
    q8 = np.asarray(q8, dtype=np.int64)
    b, hq, nq, d = q8.shape
    hkv = kpacked.shape[1]
    g = hq // hkv
    t = kpacked.shape[2]
    codes = unpack_int4(kpacked).astype(np.int64)          # [B, Hkv, T, D]
    codes_q = np.repeat(codes, g, axis=1)                  # [B, Hq, T, D]
    isum = np.einsum("bhid,bhtd->bhit", q8, codes_q)
    scale = np.repeat(fp16_bits_to_f32(kscale_bits), g, axis=1)[:, :, None, :]
    key = (scale * isum.astype(np.float32)).astype(np.float32)
    key = np.where(key == 0, np.float32(0.0), key)
    pos = q_pos0 + np.arange(nq)
    visible = np.arange(t)[None, :] <= pos[:, None]        # [Nq, T]
    key = np.where(visible[None, None], key, np.float32(-np.inf))
    return block_max(key, block)


def prefill_block_topk(bmax, k: int) -> np.ndarray:
    """Top-k blocks per query row (ties to the lower block), ascending; when a
    row has fewer than k visible blocks the tail is padded with -1."""
    sel = topk_lowest_index(bmax, k)
    vals = np.take_along_axis(np.asarray(bmax, dtype=np.float32), sel.astype(np.int64), axis=-1)
    valid = np.isfinite(vals)
    out = np.full(sel.shape, -1, dtype=np.int32)
    flat_sel = sel.reshape(-1, k)
    flat_valid = valid.reshape(-1, k)
    flat_out = out.reshape(-1, k)
    for r in range(flat_sel.shape[0]):
        keep = flat_sel[r][flat_valid[r]]
        flat_out[r, : keep.size] = keep
    return out


# ---------------------------------------------------------------------------
# Whole decode step for one layer, as the oracle composes it
# ---------------------------------------------------------------------------

def decode_select(q, slab, slab_scale_bits, chan_idx, kv_heads: int, block: int, topk: int):
    """Scores, block maxima and selected blocks of one decode step.
    Returns (I int32 [R, T], keys f32 [R, T], bmax f32 [R, nb], sel int32 [R, k])."""
    q8, _ = quantize_query_group(q, chan_idx, kv_heads)
    isum = partial_scores_i32(q8, slab)
    keys = ranking_keys(isum, slab_scale_bits)
    bmax = block_max(keys, block)
    sel = topk_lowest_index(bmax, topk)
    return isum, keys, bmax, sel


def recall_at(selected_tokens: list[np.ndarray], planted: np.ndarray) -> float:
    """Fraction of rows whose planted key position is among the selected
    tokens (hits / true count, OV:260-322 restated for one planted key)."""
    hits = sum(int(p in set(sel.tolist())) for sel, p in zip(selected_tokens, planted))
    return hits / max(1, len(planted))
