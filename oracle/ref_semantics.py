"""CPU restatement of the reference's fp32 QABS kernels and host op sequence.

TEST INFRASTRUCTURE ONLY (see ``oracle/qkv_oracle.py``): imported by tests,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``.

"QK" = ymluo/projects/qwen3_top2_head_limit3_ppl/src/qabs_cuda_kernels.py,
"EV" = ymluo/projects/qwen3_top2_head_limit3_ppl/src/
evaluate_qwen3_top2_head_limit3_ppl.py.

Two kinds of function live here:

* numpy restatements of the four kernels behind the reference's Python API
  (``partial_scores``, ``partial_scores_dim_major``, ``candidate_full_scores``,
  ``final_attention``).  The fp32 loops accumulate in the same order as the
  reference kernels with separately rounded multiply and add, so a GPU kernel
  built without FMA contraction matches them bit for bit; each is also pinned
  against an fp64 brute force in the tests.
* ``qabs_candidate_attention_cpu``: the reference's PyTorch op sequence for
  one ``qabs{S}cand{pct}attn`` decode step (EV:4419-4502, index build
  EV:2938-2982), run on CPU tensors.  It is the CPU baseline that ``bench.py``
  times next to the GPU path.
"""

from __future__ import annotations

import math

import numpy as np

QABS_MAX_DIMS = 128  # QK:60


def select_dims_by_abs(q_row, dim_count: int) -> np.ndarray:
    """Top-|q| dimensions in the reference kernel's order (QK:120-145).

    The serial selector takes, for each slot, the unused dimension with the
    largest |q| scanning d upwards with a strict ``>``: equal magnitudes keep
    the lower index.  That is a stable sort by descending |q|.  The count is
    clamped to [1, min(D, 128)] (QK:120, 438).
    """
    q_row = np.asarray(q_row, dtype=np.float32)
    d = q_row.shape[-1]
    count = min(max(int(dim_count), 1), d, QABS_MAX_DIMS)
    return np.argsort(-np.abs(q_row), kind="stable")[:count]


def _seq_dot(q_vals, k_vals) -> np.ndarray:
    """sum_s q[s] * k[..., s] in fp32, s ascending, multiply and add rounded
    separately (the accumulation loops of QK:91-94, 154-156, 210-213)."""
    acc = np.zeros(k_vals.shape[:-1], dtype=np.float32)
    for s in range(k_vals.shape[-1]):
        acc = (acc + (np.float32(q_vals[s]) * k_vals[..., s]).astype(np.float32)).astype(np.float32)
    return acc


def partial_scores(query, key, dim_count: int) -> np.ndarray:
    """QK:98-158 / QK:654-656.  query [B,H,D], key [B,H,T,D] -> f32 [B,H,T]."""
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    b, h, _ = q.shape
    out = np.empty((b, h, k.shape[2]), dtype=np.float32)
    for bi in range(b):
        for hi in range(h):
            dims = select_dims_by_abs(q[bi, hi], dim_count)
            out[bi, hi] = _seq_dot(q[bi, hi, dims], k[bi, hi][:, dims])
    return out


def partial_scores_dim_major(query, key_dim_major, dim_indices) -> np.ndarray:
    """QK:63-96 / QK:659-665.  key_dim_major [B,H,D,T], dim_indices int64
    [B,H,S] (used in the given order) -> f32 [B,H,T]."""
    q = np.asarray(query, dtype=np.float32)
    kdm = np.asarray(key_dim_major, dtype=np.float32)
    idx = np.asarray(dim_indices, dtype=np.int64)
    b, h, _ = q.shape
    out = np.empty((b, h, kdm.shape[3]), dtype=np.float32)
    for bi in range(b):
        for hi in range(h):
            dims = idx[bi, hi]
            out[bi, hi] = _seq_dot(q[bi, hi, dims], kdm[bi, hi][dims, :].T)
    return out


def candidate_full_scores(query, key, current, previous, previous_final,
                          protect_sink: int, protect_recent: int, scaling: float) -> np.ndarray:
    """QK:160-216 / QK:668-691.  Masks are bool [B,H,T] (or None).  A token is
    scored when any mask is set or it lies in the first ``protect_sink`` or
    last ``protect_recent`` positions; scored tokens get the full-D fp32 dot
    times ``scaling``, the rest -inf."""
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    sel = np.asarray(current, dtype=bool).copy()
    if previous is not None:
        sel |= np.asarray(previous, dtype=bool)
    if previous_final is not None:
        sel |= np.asarray(previous_final, dtype=bool)
    t = k.shape[2]
    pos = np.arange(t)
    if protect_sink > 0:
        sel |= (pos < protect_sink)[None, None, :]
    if protect_recent > 0:
        sel |= (pos >= max(0, t - protect_recent))[None, None, :]
    b, h, d = q.shape
    out = np.full((b, h, t), -np.inf, dtype=np.float32)
    for bi in range(b):
        for hi in range(h):
            full = _seq_dot(q[bi, hi], k[bi, hi])
            scored = (full * np.float32(scaling)).astype(np.float32)
            out[bi, hi] = np.where(sel[bi, hi], scored, np.float32(-np.inf))
    return out


def final_attention(query, key, value, indices, valid, scaling: float) -> np.ndarray:
    """QK:335-419 / QK:694-705, in fp64.  query [B,H,D]; key/value [B,H,T,D];
    indices int64 [B,H,N]; valid bool/uint8 [B,H,N].  Entries that are invalid
    or out of [0, T) get weight 0; with no valid entry the max is taken as 0
    and the output is 0 (QK:388, 404).  Returns float64 [B, 1, H, D]."""
    q = np.asarray(query, dtype=np.float64)
    k = np.asarray(key, dtype=np.float64)
    v = np.asarray(value, dtype=np.float64)
    idx = np.asarray(indices, dtype=np.int64)
    ok = np.asarray(valid).astype(bool)
    b, h, d = q.shape
    t = k.shape[2]
    out = np.zeros((b, h, d), dtype=np.float64)
    for bi in range(b):
        for hi in range(h):
            m = ok[bi, hi] & (idx[bi, hi] >= 0) & (idx[bi, hi] < t)
            sel = idx[bi, hi][m]
            if sel.size == 0:
                continue
            s = k[bi, hi, sel] @ q[bi, hi] * scaling
            p = np.exp(s - s.max())
            out[bi, hi] = (p / max(p.sum(), 1e-20)) @ v[bi, hi, sel]
    return out[:, None, :, :]


# ---------------------------------------------------------------------------
# Reference op sequence on CPU tensors (the cpu_baseline)
# ---------------------------------------------------------------------------

def final_indices_from_selected(selected, selected_valid, history_count: int, key_count: int,
                                sink: int, recent: int, keep_self: bool):
    """EV:2938-2982 on torch tensors: selected history indices with the sink
    and recent ranges masked out, then the sink range, the recent range and
    the current token appended."""
    import torch

    b, h, _ = selected.shape
    valid = selected_valid.clone()
    sink_end = min(sink, history_count) if sink > 0 else 0
    recent_start = history_count
    if recent > 0:
        recent_start = max(0, history_count - recent)
        valid &= ~((selected >= recent_start) & (selected < history_count))
    if sink_end > 0:
        valid &= selected >= sink_end
    parts, vparts = [selected], [valid]
    if sink_end > 0:
        parts.append(torch.arange(sink_end, dtype=torch.long).view(1, 1, -1).expand(b, h, -1))
        vparts.append(torch.ones((b, h, sink_end), dtype=torch.bool))
    if recent > 0 and recent_start < history_count:
        start = max(recent_start, sink_end)
        if start < history_count:
            parts.append(torch.arange(start, history_count, dtype=torch.long).view(1, 1, -1).expand(b, h, -1))
            vparts.append(torch.ones((b, h, history_count - start), dtype=torch.bool))
    if keep_self:
        parts.append(torch.full((b, h, 1), key_count - 1, dtype=torch.long))
        vparts.append(torch.ones((b, h, 1), dtype=torch.bool))
    return torch.cat(parts, dim=-1), torch.cat(vparts, dim=-1)


def qabs_candidate_attention_cpu(query_states, key_states, value_states, dim_count: int,
                                 candidate_fraction: float, scaling: float,
                                 sink: int = 0, recent: int = 0, keep_self: bool = True):
    """One ``qabs{S}cand{pct}attn`` decode step in the reference's PyTorch ops
    (EV:4419-4502), on CPU tensors.

    query_states [B,Hq,1,D]; key/value_states [B,Hkv,T,D] are GQA-expanded
    first, as the attention hook does (EV:6248-6251).  Steps: top-|q| dims
    (EV:4428), gather + fp32 multiply-sum partial scores over the history
    (EV:4443-4446), ``torch.topk`` candidates (EV:4448), index build
    (EV:2938-2982), gather, matmul, softmax, weighted sum (EV:4490-4502).
    Returns [B, 1, Hq, D].
    """
    import torch
    import torch.nn.functional as F

    b, hq, _, d = query_states.shape
    if key_states.shape[1] != hq:
        rep = hq // key_states.shape[1]
        key_states = key_states.repeat_interleave(rep, dim=1)
        value_states = value_states.repeat_interleave(rep, dim=1)
    key_count = key_states.shape[-2]
    history = key_count - 1
    sdims = min(max(1, dim_count), d)
    requested = min(history, max(1, math.ceil(candidate_fraction * history)))
    q_raw = query_states[:, :, 0, :]
    k_hist = key_states[:, :, :history, :]
    qdims = torch.topk(q_raw.float().abs(), k=sdims, dim=-1, largest=True).indices
    q_sel = torch.gather(q_raw.float(), dim=-1, index=qdims)
    k_idx = qdims[:, :, None, :].expand(-1, -1, history, -1)
    k_sel = torch.gather(k_hist.float(), dim=-1, index=k_idx)
    partial = (k_sel * q_sel[:, :, None, :]).sum(dim=-1)
    _, cand = torch.topk(partial, k=requested, dim=-1, largest=True)
    cand_valid = torch.ones_like(cand, dtype=torch.bool)
    final_idx, final_valid = final_indices_from_selected(cand, cand_valid, history, key_count,
                                                         sink, recent, keep_self)
    gather = final_idx[:, :, :, None].expand(-1, -1, -1, d)
    sel_k = torch.gather(key_states, dim=2, index=gather)
    sel_v = torch.gather(value_states, dim=2, index=gather)
    scores = torch.matmul(query_states[:, :, 0:1, :], sel_k.transpose(2, 3)).squeeze(2) * scaling
    scores = scores.masked_fill(~final_valid, torch.finfo(scores.dtype).min)
    weights = F.softmax(scores, dim=-1, dtype=torch.float32).to(query_states.dtype)
    out = torch.sum(weights[:, :, :, None] * sel_v, dim=2)
    return out[:, None, :, :].contiguous()


def qabs_attn_step(query, key, value, dim_count: int, candidate_fraction: float, scaling: float,
                   sink: int = 0, recent: int = 0, keep_self: bool = True, append: bool = False):
    """One ``qabs{S}cand{pct}attn`` decode step (EV:4400-4502) in numpy with
    the kernels' arithmetic: per query head, the fp32 partial score of every
    history token on its top-|q| dims (selection order, QK:63-96), the
    ``min(history, max(1, ceil(pct * history)))`` best (ties to the lower
    index), plus the sink / recent ranges and the current token
    (EV:2938-2982), then softmax attention over that set (QK:335-419).
    With ``append`` (the ``appendattn`` modes, EV:4451-4458, 2985-3022) the
    selected copies of protected tokens stay in the list, so those tokens
    are attended twice.

    query [B,Hq,D]; key/value [B,Hkv,T,D] (head h reads KV head h // G).
    Returns (out float64 [B,1,Hq,D], final_keep bool [B,Hq,T])."""
    from .qkv_oracle import topk_lowest_index

    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, hq, d = q.shape
    g = hq // k.shape[1]
    kx, vx = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    key_count = k.shape[2]
    if key_count <= 1:
        return vx[:, :, -1:, :].transpose(0, 2, 1, 3).astype(np.float64), np.ones((b, hq, key_count), bool)
    history = key_count - 1
    requested = min(history, max(1, math.ceil(candidate_fraction * history)))
    part = partial_scores(q, kx[:, :, :history], dim_count)
    sel = topk_lowest_index(part.reshape(-1, history), requested).reshape(b, hq, requested)
    final_keep = np.zeros((b, hq, key_count), dtype=bool)
    np.put_along_axis(final_keep, sel.astype(np.int64), True, axis=-1)
    if sink > 0:
        final_keep[..., : min(sink, history)] = True
    if recent > 0:
        final_keep[..., max(0, history - recent):history] = True
    if keep_self:
        final_keep[..., history] = True
    if append:   # the selection as it is, then the protected tokens (EV:2992-3022)
        sink_end = min(sink, history) if sink > 0 else 0
        rec_begin = max(max(0, history - recent), sink_end) if recent > 0 else history
        tail = list(range(sink_end)) + list(range(rec_begin, history)) + ([history] if keep_self else [])
        idx = np.concatenate([sel.astype(np.int64), np.broadcast_to(np.array(tail, dtype=np.int64),
                                                                       (b, hq, len(tail)))], axis=-1)
        return final_attention(q, kx, vx, idx, np.ones(idx.shape, dtype=bool), scaling), final_keep
    idx = np.broadcast_to(np.arange(key_count), final_keep.shape)
    return final_attention(q, kx, vx, idx, final_keep, scaling), final_keep


def qabs_periodic_step(query, key, value, dim_count: int, candidate_fraction: float, interval: int,
                       scaling: float, sink: int = 0, recent: int = 0, keep_self: bool = True, previous=None):
    """One ``qabs{S}cand{pct}r{N}attn`` decode step (EV:4505-4609, the default
    path without QABS_PERIODIC_FUSED_REMOTE_RECENT): when the query token
    (= history) is not a multiple of ``interval`` and ``previous`` holds the
    last step's selected indices (the state keeps them for query token - 1
    only, EV:1702-1733), they are reused as they are; otherwise the
    ``min(history, max(1, ceil(pct * history)))`` best fp32 partial scores
    are selected (ties to the lower index).  The final list is
    ``final_indices_np`` of the selection at the current history
    (EV:2938-2982), then attention over it.

    Returns (out float64 [B,1,Hq,D], final_keep bool [B,Hq,T], the selection
    int64 [B,Hq,n] the next step may reuse)."""
    from .qkv_oracle import topk_lowest_index

    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, hq, _ = q.shape
    g = hq // k.shape[1]
    kx, vx = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    key_count = k.shape[2]
    history = key_count - 1
    if previous is not None and history % max(1, int(interval)) != 0:
        sel = np.asarray(previous, dtype=np.int64)
    else:
        requested = min(history, max(1, math.ceil(candidate_fraction * history)))
        part = partial_scores(q, kx[:, :, :history], dim_count)
        sel = np.sort(topk_lowest_index(part.reshape(-1, history), requested), axis=-1)
        sel = sel.reshape(b, hq, requested).astype(np.int64)
    valid = (sel >= 0) & (sel < history)
    fi, fv = final_indices_np(np.maximum(sel, 0), valid, history, key_count, sink, recent, keep_self)
    keep = np.zeros((b, hq, key_count), dtype=bool)
    for lead in np.ndindex(b, hq):
        keep[lead][fi[lead][fv[lead]]] = True
    return final_attention(q, kx, vx, fi, fv, scaling), keep, sel


# ---------------------------------------------------------------------------
# Candidate reuse and exact rerank (qabs{S}cand{pct}reuse[final|2set])
# ---------------------------------------------------------------------------

def budget_count(history: int, fraction: float) -> int:
    """``min(history, max(1, ceil(fraction * history)))`` (EV:4132, 4270)."""
    return min(int(history), max(1, math.ceil(float(fraction) * int(history))))


def threshold_mask(partial, requested: int) -> np.ndarray:
    """EV:3988-3989: every value >= the row's ``requested``-th largest (ties
    at the threshold are all kept, so a row may hold more than requested)."""
    p = np.asarray(partial, dtype=np.float32)
    thr = -np.sort(-p, axis=-1)[..., requested - 1:requested]
    return p >= thr


def sample_columns(history: int, sample_size: int):
    """The sampled positions of the ``sample_quantile`` candidate selection
    (EV:3973-3981): ``linspace(0, history - 1, steps=min(history,
    max(1, sample_size)))`` in float32, rounded half to even, deduplicated;
    None when the sample covers the row.  The float32 linspace is torch's
    own (its CPU kernel fills vector lanes from a running base, which a
    closed form does not reproduce at .5 ties), so this calls it."""
    import torch

    count = min(int(history), max(1, int(sample_size)))
    if count >= history:
        return None
    cols = torch.linspace(0, history - 1, steps=count, dtype=torch.float32).round().long().unique()
    return cols.numpy()


def candidate_mask(partial, requested: int, fraction: float, selection: str = "topk", previous_thresholds=None,
                   sample_size: int = 256):
    """``_select_qabs_candidate_from_partial_scores`` (EV:3958-3989):
    (mask, thresholds [..., 1] float32, selection used).  ``topk``: every
    value >= the ``requested``-th largest; ``sample_quantile``: the
    threshold is the ``min(n, max(1, ceil(fraction * n)))``-th largest of
    the n sampled columns (the whole row when the sample covers it);
    ``previous_threshold``: the given per-row thresholds, falling back to
    ``topk`` when there are none."""
    p = np.asarray(partial, dtype=np.float32)
    history = p.shape[-1]
    if selection == "previous_threshold" and previous_thresholds is not None:
        thr = np.asarray(previous_thresholds, dtype=np.float32).reshape(*p.shape[:-1], 1)
        return p >= thr, thr, "previous_threshold"
    if selection == "sample_quantile" and history > 0:
        cols = sample_columns(history, sample_size)
        sampled = p if cols is None else p[..., cols]
        k = min(sampled.shape[-1], max(1, math.ceil(fraction * sampled.shape[-1])))
        thr = -np.sort(-sampled, axis=-1)[..., k - 1:k]
        return p >= thr, thr, "sample_quantile"
    thr = -np.sort(-p, axis=-1)[..., requested - 1:requested]
    return p >= thr, thr, "topk"


def final_indices_np(selected, selected_valid, history: int, key_count: int, sink: int, recent: int,
                     keep_self: bool):
    """EV:2938-2982 in numpy: the selected history indices with the sink and
    recent ranges masked invalid, then the sink range, the recent range (not
    overlapping the sink) and the current token appended."""
    sel = np.asarray(selected, dtype=np.int64)
    valid = np.asarray(selected_valid, dtype=bool).copy()
    lead = sel.shape[:-1]
    sink_end = min(sink, history) if sink > 0 else 0
    recent_start = history
    if recent > 0:
        recent_start = max(0, history - recent)
        valid &= ~((sel >= recent_start) & (sel < history))
    if sink_end > 0:
        valid &= sel >= sink_end
    parts, vparts = [sel], [valid]
    if sink_end > 0:
        parts.append(np.broadcast_to(np.arange(sink_end), (*lead, sink_end)))
        vparts.append(np.ones((*lead, sink_end), dtype=bool))
    if recent > 0 and recent_start < history:
        start = max(recent_start, sink_end)
        if start < history:
            parts.append(np.broadcast_to(np.arange(start, history), (*lead, history - start)))
            vparts.append(np.ones((*lead, history - start), dtype=bool))
    if keep_self:
        parts.append(np.full((*lead, 1), key_count - 1, dtype=np.int64))
        vparts.append(np.ones((*lead, 1), dtype=bool))
    return np.concatenate(parts, axis=-1).astype(np.int64), np.concatenate(vparts, axis=-1)


def expand_to_blocks(keep, block):
    """EV:2914-2922: every aligned block of ``block`` history positions
    (block j = positions [j*block, (j+1)*block), the last one cut at the
    history) that holds a set flag becomes wholly set.  Unchanged for
    ``block`` None or <= 1, or a history of at most one position."""
    m = np.asarray(keep, dtype=bool)
    history = m.shape[-1]
    if block is None or block <= 1 or history <= 1:
        return m.copy()
    blocks = -(-history // block)
    padded = np.zeros((*m.shape[:-1], blocks * block), dtype=bool)
    padded[..., :history] = m
    hit = padded.reshape(*m.shape[:-1], blocks, block).any(axis=-1)
    return np.repeat(hit, block, axis=-1)[..., :history]


def indices_from_keep_mask(keep):
    """EV:2896-2911: the set positions of each row in descending order,
    padded to the largest count over the rows with (0, invalid)."""
    m = np.asarray(keep, dtype=bool)
    width = int(m.sum(axis=-1).max()) if m.size else 0
    idx = np.zeros((*m.shape[:-1], width), dtype=np.int64)
    valid = np.zeros((*m.shape[:-1], width), dtype=bool)
    for lead in np.ndindex(*m.shape[:-1]):
        pos = np.flatnonzero(m[lead])[::-1]
        idx[lead][: len(pos)] = pos
        valid[lead][: len(pos)] = True
    return idx, valid


def reuse_select(query, key_states, current, previous, previous_final, sink: int, recent: int,
                 top_fraction: float, keep_self: bool, scaling: float, block: int | None = None):
    """The selection the reference asks of its absent ``reuse_select`` kernel
    (called at EV:3901-3914 with the signature of EV:3881-3892), restated from
    the fallback that runs when the kernel is missing (EV:4257-4365, no
    block or evidence-span option):

    * scores: full-D fp32 dot * scaling on the union current | previous |
      previous_final, -inf elsewhere (candidate_full_scores with no sink or
      recent protection, EV:4257-4267: the non-lagged modes pass 0 there);
    * the ``budget_count(history, top_fraction)`` largest scores (EV:4270-4274;
      ``torch.topk``, ties here to the lower index), valid where finite;
    * history_final: the valid selections, then the sink and recent ranges
      set (EV:4301-4307);
    * with ``block`` (the ``reuse…blk{block}`` modes, EV:4022, 4314-4316):
      history_final expanded to whole aligned blocks (``expand_to_blocks``)
      and the selection re-read from it (``indices_from_keep_mask``);
    * final indices and validity by ``final_indices_np`` (EV:4365, 2938-2982).

    query [B,H,D]; key_states [B,H,K,D] with K = history + 1; masks bool
    [B,H,history] (previous ones may be None).  Without ``block`` the
    selected indices come in ascending order (the reference's come in
    descending score order; only the set and its validity carry meaning).
    Returns (final_indices int64, final_valid bool, history_final bool
    [B,H,history]).
    """
    from .qkv_oracle import topk_lowest_index

    cur = np.asarray(current, dtype=bool)
    b, h, history = cur.shape
    key = np.asarray(key_states, dtype=np.float32)
    key_count = key.shape[2]
    scores = candidate_full_scores(query, key[:, :, :history], cur, previous, previous_final, 0, 0,
                                   scaling)
    keep = budget_count(history, top_fraction)
    sel = topk_lowest_index(scores.reshape(-1, history), keep).reshape(b, h, keep).astype(np.int64)
    valid = np.isfinite(np.take_along_axis(scores, sel, axis=-1))
    hist_final = np.zeros((b, h, history), dtype=bool)
    for bi in range(b):
        for hi in range(h):
            hist_final[bi, hi, sel[bi, hi][valid[bi, hi]]] = True
    if sink > 0:
        hist_final[..., : min(sink, history)] = True
    if recent > 0:
        hist_final[..., max(0, history - recent):] = True
    if block is not None:
        hist_final = expand_to_blocks(hist_final, block)
        sel, valid = indices_from_keep_mask(hist_final)
    fi, fv = final_indices_np(sel, valid, history, key_count, sink, recent, keep_self)
    return fi, fv, hist_final


def reuse_decode_step(query, key, value, dim_count: int, candidate_fraction: float, top_fraction: float,
                      sink: int, recent: int, keep_self: bool, scaling: float,
                      previous_candidate=None, previous_final=None, block: int | None = None, *,
                      selection: str = "topk", sample_size: int = 256, previous_thresholds=None,
                      thresholds_out: list | None = None):
    """One decode step of ``_qabs_reuse_fast_attention_forward`` (EV:3991-4397)
    for the default candidate selection (``topk``), block-expanded when
    ``block`` is given (``reuse…blk{block}``, EV:757-761, 4314-4316).

    query [B,Hq,D]; key/value [B,Hkv,T,D] (query head h reads KV head
    h // (Hq/Hkv), the grouping of EV:6248-6251).  previous_* are the masks
    the previous step left (bool [B,Hq,>= T-2]; pass None when there is no
    previous step, or to leave one out as the ``reusefinal`` / ``reuse2set``
    modes do, EV:955-960).  They are cut or padded with False to the history
    length, as ``ReuseCandidateState.previous_layer_masks`` does (EV:1645-1662).

    Steps: top-|q| dims and fp32 partial scores (EV:4068, 4123-4135), the
    candidate mask under ``selection`` (``candidate_mask``, EV:4136-4144;
    ``previous_thresholds`` are the thresholds the previous step left, the
    step's own are appended to ``thresholds_out`` when given; the
    reference keeps them in its state, EV:1686-1694, 1744-1745),
    ``reuse_select``, and the attention over the final indices (QK:335-419,
    fp64 here).  A cache of at most one key returns the last value
    (EV:4012-4014).

    Returns (out float64 [B,1,Hq,D], current bool [B,Hq,history],
    history_final bool [B,Hq,history]); the last two are the state the next
    step reads (EV:4384-4393).
    """
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, hq, d = q.shape
    g = hq // k.shape[1]
    kx, vx = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    key_count = k.shape[2]
    if key_count <= 1:
        return vx[:, :, -1:, :].transpose(0, 2, 1, 3).astype(np.float64), None, None
    history = key_count - 1
    partial = partial_scores(q, kx[:, :, :history], dim_count)
    current, thr, _ = candidate_mask(partial, budget_count(history, candidate_fraction), candidate_fraction,
                                     selection, previous_thresholds, sample_size)
    if thresholds_out is not None:
        thresholds_out.append(thr)

    def fit(m):
        if m is None:
            return None
        m = np.asarray(m, dtype=bool)[..., :history]
        pad = history - m.shape[-1]
        return np.concatenate([m, np.zeros((*m.shape[:-1], pad), dtype=bool)], axis=-1) if pad else m

    fi, fv, hist_final = reuse_select(q, kx, current, fit(previous_candidate), fit(previous_final), sink, recent,
                                      top_fraction, keep_self, scaling, block)
    out = final_attention(q, kx, vx, fi, fv, scaling)
    return out, current, hist_final


# The lagged reuse family (EV:473-476, 918-955): kind -> the mode prefix.
LAGGED_KINDS = ("lagtop2", "lagrefresh", "qdrift", "qdriftmaj", "qdrifthead", "qdriftshare", "qdriftcos",
                "qdriftcoshead", "pconf")
_PER_HEAD_KINDS = ("qdrifthead", "qdriftcoshead", "qdriftshare", "pconf")   # EV:4089


def _bf16_round(x):
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


def previous_final_ess_fraction(query, key, previous_final, scaling: float, bf16_scores: bool = False):
    """The pconf test's statistic (EV:4071-4085): per row, the softmax weights
    of q over the tokens of the previous final mask (full-D dot * scaling;
    with ``bf16_scores`` the dot and the scaled score rounded to bf16, as a
    bf16 matmul and multiply leave them), the effective sample size
    1 / max(sum w^2, 1e-12), divided by max(count, 1), every step in float32
    as the reference's fp32 softmax and the ops after it (EV:4079-4083).  A
    row with no token has all weights 0, hence 1e12.  query [B,H,D]; key
    [B,H,>=hist,D]; previous_final bool [B,H,hist].  Returns float32 [B,H]."""
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    m = np.asarray(previous_final, dtype=bool)
    b, h, _ = q.shape
    out = np.empty((b, h), dtype=np.float32)
    f32 = np.float32
    for bi in range(b):
        for hi in range(h):
            pos = np.flatnonzero(m[bi, hi])
            if pos.size == 0:
                out[bi, hi] = f32(1.0) / f32(1e-12)
                continue
            sc = (k[bi, hi, pos].astype(np.float64) @ q[bi, hi].astype(np.float64)).astype(np.float32)
            if bf16_scores:
                sc = _bf16_round(_bf16_round(sc) * f32(scaling))
            else:
                sc = sc * f32(scaling)
            e = np.exp(sc - sc.max(), dtype=np.float32)
            w = e / e.sum(dtype=np.float32)
            sw2 = (w * w).sum(dtype=np.float32)
            out[bi, hi] = (f32(1.0) / max(sw2, f32(1e-12))) / f32(pos.size)
    return out


def lagged_reuse_decode_step(query, key, value, kind: str, param, dim_count: int, candidate_fraction: float,
                             top_fraction: float, sink: int, recent: int, keep_self: bool, scaling: float,
                             previous=None, bf16_scores: bool = False, *, selection: str = "topk",
                             sample_size: int = 256):
    """One decode step of the lagged reuse modes (``lagtop2``, ``lagrefresh{N}``,
    ``qdrift[maj|head|share|cos|coshead]`` and ``pconf{T}`` before
    ``qabs{S}cand{pct}``), ``_qabs_reuse_fast_attention_forward`` EV:4020-4198,
    then the rerank of EV:4257-4365.  The candidate ``selection`` (``topk``,
    ``sample_quantile``, ``previous_threshold``; ``candidate_mask``) applies
    where every head thresholds its partial scores (EV:4116-4145); the per-head
    refresh scores flagged heads by ``topk`` (EV:4089-4106).

    ``param`` is N for lagrefresh and T (a fraction) for pconf.  ``previous``
    is None or the previous step's state: dict(final=bool [B,Hq,>= hist-1],
    dims=int [B,Hq,S], values=float [B,Hq,S], and thresholds [B,Hq,1] when
    that step thresholded every head) (EV:1645-1694, 1733-1745, present only
    when the previous step was query token - 1).

    * refresh test: lagrefresh refreshes when history % N == 0 (EV:4024); the
      qdrift kinds flag a head whose current top-S dims share fewer than
      max(1, ceil(S/2)) with the previous ones, or (cos kinds) whose q on the
      previous dims has cosine < 0.5 with the previous values (EV:4045-4066);
      the step refreshes if any head is flagged (a majority for qdriftmaj);
      pconf flags heads whose ``previous_final_ess_fraction`` > T (EV:4068-4087);
    * candidates: with a previous final mask, the per-head kinds (head,
      coshead, share, pconf) score only flagged heads, others keep an empty
      candidate set (EV:4089-4109); the other kinds reuse the previous final
      mask alone unless the step refreshes (EV:4110-4115); otherwise every head
      thresholds its partial scores (EV:4116-4145);
    * union = candidates | previous final (| for share, the OR over the
      batch's heads) | the sink and recent ranges (EV:4147-4175); the rerank
      and final selection of ``reuse_select`` on it.

    Returns (out float64 [B,1,Hq,D], current bool [B,Hq,hist], history_final
    bool [B,Hq,hist], state dict for the next step, flagged bool [B,Hq] or
    None)."""
    if kind not in LAGGED_KINDS:
        raise ValueError(f"unknown lagged kind {kind!r}")
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, hq, d = q.shape
    g = hq // k.shape[1]
    kx, vx = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    history = k.shape[2] - 1
    s_count = min(max(1, int(dim_count)), d)
    dims = np.stack([np.stack([select_dims_by_abs(q[bi, hi], s_count) for hi in range(hq)]) for bi in range(b)])
    values = np.take_along_axis(q, dims, axis=-1)
    refresh = kind == "lagrefresh" and history % int(param) == 0
    prev_final = None
    if previous is not None:
        m = np.asarray(previous["final"], dtype=bool)[..., :history]
        pad = history - m.shape[-1]
        prev_final = np.concatenate([m, np.zeros((*m.shape[:-1], pad), dtype=bool)], axis=-1) if pad else m
    flagged = None
    if kind.startswith("qdrift"):
        refresh = True
        if previous is not None:
            pd = np.asarray(previous["dims"])
            overlap = (dims[..., :, None] == pd[..., None, :]).any(axis=-1).sum(axis=-1)
            flagged = overlap < max(1, math.ceil(s_count / 2))
            if kind in ("qdriftcos", "qdriftcoshead"):
                on_prev = np.take_along_axis(q, pd, axis=-1).astype(np.float64)
                pv = np.asarray(previous["values"], dtype=np.float64)
                den = np.linalg.norm(on_prev, axis=-1) * np.linalg.norm(pv, axis=-1)
                flagged = flagged | ((on_prev * pv).sum(axis=-1) / np.maximum(den, 1e-6) < 0.5)
            refresh = bool(flagged.mean() > 0.5) if kind == "qdriftmaj" else bool(flagged.any())
    if kind == "pconf":
        refresh = True
        if prev_final is not None:
            flagged = previous_final_ess_fraction(q, kx, prev_final, scaling, bf16_scores) > float(param)
            refresh = bool(flagged.any())
    requested = budget_count(history, candidate_fraction)
    thr = None
    if kind in _PER_HEAD_KINDS and prev_final is not None and flagged is not None:
        partial = partial_scores(q, kx[:, :, :history], dim_count)
        current = threshold_mask(partial, requested) & flagged[..., None]
        union = prev_final | current
        if kind == "qdriftshare":
            union = union | current.any(axis=1, keepdims=True)
    elif prev_final is not None and not refresh:
        current = np.zeros((b, hq, history), dtype=bool)
        union = prev_final.copy()
    else:
        prev_thr = previous.get("thresholds") if previous is not None else None
        current, thr, _ = candidate_mask(partial_scores(q, kx[:, :, :history], dim_count), requested,
                                         candidate_fraction, selection, prev_thr, sample_size)
        union = current | prev_final if prev_final is not None else current.copy()
    if sink > 0:
        union[..., : min(sink, history)] = True
    if recent > 0:
        union[..., max(0, history - recent):] = True
    fi, fv, hist_final = reuse_select(q, kx, union, None, None, sink, recent, top_fraction, keep_self, scaling)
    out = final_attention(q, kx, vx, fi, fv, scaling)
    state = {"final": hist_final, "dims": dims, "values": values}
    if thr is not None:   # recorded only by a step that thresholded every head (EV:1744-1745)
        state["thresholds"] = thr
    return out, current, hist_final, state, flagged


def qabs_reuse_step_cpu(query_states, key_states, value_states, dim_count: int, candidate_fraction: float,
                        top_fraction: float, scaling: float, sink: int = 0, recent: int = 0, keep_self: bool = True,
                        previous_candidate=None, previous_final=None, block: int | None = None, *,
                      selection: str = "topk", sample_size: int = 256, previous_thresholds=None,
                      thresholds_out: list | None = None):
    """One ``qabs{S}cand{pct}reuse`` decode step in the reference's PyTorch
    ops on CPU tensors: the path ``_qabs_reuse_fast_attention_forward`` takes
    when no CUDA kernel is available (EV:3991-4397 with the dense-mask
    fallbacks of EV:4161-4167, 4276-4303 and the gather attention of
    EV:4365-4374), block-expanded when ``block`` is given (EV:4314-4316).
    It is the CPU baseline that ``bench.py`` times next to the GPU reuse
    step.

    query_states [B,Hq,1,D]; key/value_states [B,Hkv,T,D] (GQA-expanded
    first, EV:6248-6251); previous_* bool [B,Hq,T-1] or None.  Returns
    (out [B,1,Hq,D], current, history_final)."""
    import torch
    import torch.nn.functional as F

    b, hq, _, d = query_states.shape
    if key_states.shape[1] != hq:
        rep = hq // key_states.shape[1]
        key_states = key_states.repeat_interleave(rep, dim=1)
        value_states = value_states.repeat_interleave(rep, dim=1)
    key_count = key_states.shape[-2]
    history = key_count - 1
    q_raw = query_states[:, :, 0, :]
    k_hist = key_states[:, :, :history, :]
    sdims = min(max(1, dim_count), d)
    qdims = torch.topk(q_raw.float().abs(), k=sdims, dim=-1, largest=True).indices               # EV:4068
    q_sel = torch.gather(q_raw.float(), dim=-1, index=qdims)
    k_sel = torch.gather(k_hist.float(), dim=-1, index=qdims[:, :, None, :].expand(-1, -1, history, -1))
    partial = (k_sel * q_sel[:, :, None, :]).sum(dim=-1)                                          # EV:4130-4135
    requested = budget_count(history, candidate_fraction)
    thr = torch.topk(partial, k=requested, dim=-1, largest=True).values[:, :, -1:]
    current = partial >= thr                                                                      # EV:3988-3989
    union = current.clone()                                                                       # EV:4161-4167
    if previous_candidate is not None:
        union |= previous_candidate
    if previous_final is not None:
        union |= previous_final
    # _indices_from_keep_mask (EV:2896-2911): descending positions of the mask
    counts = union.sum(dim=-1)
    width = max(1, int(counts.max().item()))
    pos = torch.arange(history).view(1, 1, -1).expand_as(union)
    cand_idx = torch.topk(torch.where(union, pos, torch.full_like(pos, -1)), k=width, dim=-1, largest=True).values
    cand_valid = cand_idx >= 0
    cand_idx = cand_idx.clamp_min(0)
    keys = torch.gather(k_hist, dim=2, index=cand_idx[:, :, :, None].expand(-1, -1, -1, d))       # EV:4290-4296
    scores = torch.matmul(query_states[:, :, 0:1, :], keys.transpose(2, 3)).squeeze(2) * scaling
    scores = scores.masked_fill(~cand_valid, torch.finfo(scores.dtype).min)
    keep = min(budget_count(history, top_fraction), scores.shape[-1])
    _, sel_pos = torch.topk(scores, k=keep, dim=-1, largest=True)                                # EV:4298-4303
    selected = torch.gather(cand_idx, dim=-1, index=sel_pos)
    selected_valid = torch.gather(cand_valid, dim=-1, index=sel_pos)
    history_final = torch.zeros_like(current)                                                     # EV:4305-4312
    history_final.scatter_(dim=-1, index=selected, src=selected_valid)
    if sink > 0:
        history_final[:, :, : min(sink, history)] = True
    if recent > 0:
        history_final[:, :, max(0, history - recent):history] = True
    if block is not None and block > 1 and history > 1:                                           # EV:2914-2922
        blocks = -(-history // block)
        padded = F.pad(history_final, (0, blocks * block - history), value=False)
        hit = padded.view(b, hq, blocks, block).any(dim=-1, keepdim=True)
        history_final = hit.expand(-1, -1, -1, block).reshape(b, hq, blocks * block)[..., :history]
    if block is not None:                                                                         # EV:4316
        width = int(history_final.sum(dim=-1).max().item())
        pos = torch.arange(history).view(1, 1, -1).expand_as(history_final)
        selected = torch.topk(torch.where(history_final, pos, torch.full_like(pos, -1)), k=width, dim=-1,
                              largest=True).values
        selected_valid = selected >= 0
        selected = selected.clamp_min(0)
    final_idx, final_valid = final_indices_from_selected(selected, selected_valid, history, key_count, sink,
                                                         recent, keep_self)                     # EV:4365
    gather = final_idx[:, :, :, None].expand(-1, -1, -1, d)                                       # EV:4366-4374
    sel_k = torch.gather(key_states, dim=2, index=gather)
    sel_v = torch.gather(value_states, dim=2, index=gather)
    att = torch.matmul(query_states[:, :, 0:1, :], sel_k.transpose(2, 3)).squeeze(2) * scaling
    att = att.masked_fill(~final_valid, torch.finfo(att.dtype).min)
    weights = F.softmax(att, dim=-1, dtype=torch.float32).to(query_states.dtype)
    out = torch.sum(weights[:, :, :, None] * sel_v, dim=2)
    return out[:, None, :, :].contiguous(), current, history_final


# ---------------------------------------------------------------------------
# Block-metadata selectors: Quest-style channel bounds (qbb) and block
# representatives (brep)
# ---------------------------------------------------------------------------

def block_minmax(key, block: int):
    """Per block of ``block`` tokens and per channel, the min and max of K
    over the block's tokens (the last block may be partial; EV:5536-5553).
    key [..., T, D] -> (kmin, kmax) [..., ceil(T/block), D] float32."""
    k = np.asarray(key, dtype=np.float32)
    t = k.shape[-2]
    nb = -(-t // block)
    pad = nb * block - t
    hi = np.concatenate([k, np.full((*k.shape[:-2], pad, k.shape[-1]), -np.inf, np.float32)], axis=-2)
    lo = np.concatenate([k, np.full((*k.shape[:-2], pad, k.shape[-1]), np.inf, np.float32)], axis=-2)
    shape = (*k.shape[:-2], nb, block, k.shape[-1])
    return lo.reshape(shape).min(axis=-2), hi.reshape(shape).max(axis=-2)


def qbb_block_bounds(query, kmin, kmax, dim_count: int) -> np.ndarray:
    """Quest-style upper bound of q.k over a block on the row's top-|q| dims
    (EV:5554): sum over dims d_s, in selection order, of q_s * max_d when
    q_s >= 0 else q_s * min_d, fp32 with separately rounded products and
    sums.  query [B,H,D]; kmin/kmax [B,H,nb,D] -> f32 [B,H,nb]."""
    q = np.asarray(query, dtype=np.float32)
    b, h, _ = q.shape
    out = np.zeros((b, h, kmin.shape[2]), dtype=np.float32)
    for bi in range(b):
        for hi in range(h):
            dims = select_dims_by_abs(q[bi, hi], dim_count)
            acc = np.zeros(kmin.shape[2], dtype=np.float32)
            for d in dims:
                qs = np.float32(q[bi, hi, d])
                ext = kmax[bi, hi, :, d] if qs >= 0 else kmin[bi, hi, :, d]
                acc = (acc + (qs * ext).astype(np.float32)).astype(np.float32)
            out[bi, hi] = acc
    return out


def block_representatives(key, block: int, reps: int):
    """Per block, the ``reps`` tokens of largest squared norm (fp32 sum of
    squares in channel order), ties to the lower position, in descending
    norm order (BlockRepState.representatives, EV:1857-1918).
    key [..., T, D] -> (indices int64 [..., nb, R], valid bool [..., nb, R]);
    a partial last block with fewer tokens pads with index 0, invalid."""
    k = np.asarray(key, dtype=np.float32)
    t, d = k.shape[-2], k.shape[-1]
    nb = -(-t // block)
    r = max(1, min(reps, block))
    lead = k.shape[:-2]
    norms = np.zeros((*lead, t), dtype=np.float32)
    for c in range(d):
        norms = (norms + (k[..., c] * k[..., c]).astype(np.float32)).astype(np.float32)
    idx = np.zeros((*lead, nb, r), dtype=np.int64)
    valid = np.zeros((*lead, nb, r), dtype=bool)
    flat_n = norms.reshape(-1, t)
    fi, fv = idx.reshape(-1, nb, r), valid.reshape(-1, nb, r)
    for row in range(flat_n.shape[0]):
        for j in range(nb):
            s, e = j * block, min(t, (j + 1) * block)
            order = np.lexsort((np.arange(s, e), -flat_n[row, s:e]))[: min(r, e - s)]
            fi[row, j, : order.size] = s + order
            fv[row, j, : order.size] = True
    return idx, valid


def brep_block_scores(query, key, rep_idx, rep_valid, dim_count: int) -> np.ndarray:
    """Block score = max over the block's valid representatives of the fp32
    partial score on the row's top-|q| dims (EV:5431-5435); a block with no
    valid representative scores finfo(float32).min.  query [B,H,D]; key
    [B,H,T,D]; rep_* [B,H,nb,R] -> f32 [B,H,nb]."""
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    b, h, _ = q.shape
    nb = rep_idx.shape[2]
    lowest = np.finfo(np.float32).min
    out = np.full((b, h, nb), lowest, dtype=np.float32)
    for bi in range(b):
        for hi in range(h):
            dims = select_dims_by_abs(q[bi, hi], dim_count)
            sc = _seq_dot(q[bi, hi, dims], k[bi, hi][rep_idx[bi, hi]][..., dims])   # [nb, R]
            sc = np.where(rep_valid[bi, hi], sc, lowest)
            out[bi, hi] = sc.max(axis=-1)
    return out


def brep_partial_scores(query, key, rep_idx, rep_valid, block: int, dim_count: int, scan_fraction: float):
    """The absent ``brep_partial_scores`` kernel (wrapper EV:3847-3877, call
    EV:5419-5431): the partial scores of the tokens of the
    ``min(blocks, max(1, ceil(scan * T / block)))`` blocks with the best
    representative score (``brep_block_scores``, ties to the lower block),
    -inf elsewhere, so the caller's ``topk`` + ``isfinite`` (EV:5426-5428)
    draws candidates from the scanned blocks as its fallback does
    (EV:5442-5470).  query [B,H,D]; key [B,H,T,D]; rep_* [B,H,nb,R] ->
    f32 [B,H,T]."""
    from .qkv_oracle import topk_lowest_index

    k = np.asarray(key, dtype=np.float32)
    b, h, t, _ = k.shape
    nb = -(-t // block)
    bscore = brep_block_scores(query, k, rep_idx, rep_valid, dim_count)
    n_scan = min(nb, max(1, math.ceil(scan_fraction * t / block)))
    blocks = topk_lowest_index(bscore.reshape(-1, nb), n_scan).reshape(b, h, n_scan)
    keep = np.zeros((b, h, nb), dtype=bool)
    np.put_along_axis(keep, blocks.astype(np.int64), True, axis=-1)
    tok_keep = np.repeat(keep, block, axis=-1)[..., :t]
    return np.where(tok_keep, partial_scores(query, k, dim_count), np.float32(-np.inf)).astype(np.float32)


def brep_caller_final_mask(partial, query, key_history, key_count: int, candidate_fraction: float,
                           top_fraction: float, scaling: float, sink: int, recent: int, keep_self: bool):
    """What the reference's brep step does with ``brep_partial_scores``'
    output on one (b, h) row (EV:5426-5428, 5470-5491), ties to the lower
    index: the ``ceil(cand * history)`` best finite partial scores, their
    full-D scores * scaling, the ``ceil(top * history)`` best of those, then
    the final mask with the sink / recent ranges and the current token.
    partial [history]; query [D]; key_history [history, D] -> bool [key_count]."""
    from .qkv_oracle import topk_lowest_index

    partial = np.asarray(partial, dtype=np.float32)
    history = key_count - 1
    requested = min(history, max(1, math.ceil(candidate_fraction * history)))
    order = topk_lowest_index(partial[None], requested)[0]
    cidx = order[np.isfinite(partial[order])]
    final = np.zeros(key_count, dtype=bool)
    if cidx.size:
        q = np.asarray(query, dtype=np.float32)
        full = (_seq_dot(q, np.asarray(key_history, dtype=np.float32)[cidx]) * np.float32(scaling)).astype(np.float32)
        keep_count = min(cidx.size, requested, max(1, math.ceil(top_fraction * history)))
        final[cidx[topk_lowest_index(full[None], keep_count)[0]]] = True
    if sink > 0:
        final[: min(sink, history)] = True
    if recent > 0:
        final[max(0, history - recent):history] = True
    if keep_self:
        final[history] = True
    return final


def block_select_step(query, key, value, kind: str, block: int, dim_count: int, scan_fraction: float,
                      candidate_fraction: float, top_fraction: float, scaling: float, sink: int = 0,
                      recent: int = 0, keep_self: bool = True, reps: int = 1):
    """One decode step of the qbb (EV:5508-5617), brep (EV:5361-5505) or
    qboracle (block max of the partial scores, EV:5008-5097) selector:
    block scores -> the ``ceil(scan * history / block)`` best blocks
    -> partial scores of their tokens on the top-|q| dims -> the
    ``ceil(cand * history)`` best tokens -> full-D fp32 scores * scaling ->
    the ``ceil(top * history)`` best -> final mask with the sink / recent
    ranges and the current token -> attention over the mask.

    query [B,Hq,D]; key/value [B,Hkv,T,D] (head h reads KV head h // G).
    Ties go to the lower block / token index at every selection (the
    reference's ``torch.topk`` leaves them unspecified).  Returns (out
    float64 [B,1,Hq,D], final_keep bool [B,Hq,T])."""
    from .qkv_oracle import topk_lowest_index

    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    b, hq, d = q.shape
    g = hq // k.shape[1]
    kx, vx = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    key_count = k.shape[2]
    if key_count <= 1:
        return vx[:, :, -1:, :].transpose(0, 2, 1, 3).astype(np.float64), np.ones((b, hq, key_count), bool)
    history = key_count - 1
    kh = kx[:, :, :history]
    nb = -(-history // block)
    part_all = None
    if kind == "qbb":
        kmin, kmax = block_minmax(kh, block)
        bscore = qbb_block_bounds(q, kmin, kmax, dim_count)
    elif kind == "brep":
        ridx, rvalid = block_representatives(kh, block, reps)
        bscore = brep_block_scores(q, kh, ridx, rvalid, dim_count)
    elif kind == "qboracle":
        from .qkv_oracle import block_max

        part_all = partial_scores(q, kh, dim_count)
        bscore = block_max(part_all, block)
    else:
        raise ValueError(kind)
    n_scan = min(nb, max(1, math.ceil(scan_fraction * history / block)))
    blocks = topk_lowest_index(bscore.reshape(-1, nb), n_scan).reshape(b, hq, n_scan)
    final_keep = np.zeros((b, hq, key_count), dtype=bool)
    n_req = max(1, math.ceil(candidate_fraction * history))
    n_keep = max(1, math.ceil(top_fraction * history))
    lowest = np.float32(np.finfo(np.float32).min)
    for bi in range(b):
        for hi in range(hq):
            toks = np.concatenate([np.arange(j * block, min(history, (j + 1) * block)) for j in blocks[bi, hi]])
            toks.sort()
            if part_all is not None:
                # qboracle ranks every history token, the unscanned ones at
                # finfo(float32).min -- finite, so still valid candidates once
                # the scanned ones run out (EV:5055-5058)
                scores = np.full(history, lowest, dtype=np.float32)
                scores[toks] = part_all[bi, hi, toks]
                cand = np.sort(topk_lowest_index(scores[None], min(history, n_req))[0])
                full = (_seq_dot(q[bi, hi], kh[bi, hi][cand]) * np.float32(scaling)).astype(np.float32)
                keep = cand[topk_lowest_index(full[None], min(cand.size, n_keep))[0]]
                final_keep[bi, hi, keep] = True
                continue
            dims = select_dims_by_abs(q[bi, hi], dim_count)
            part = _seq_dot(q[bi, hi, dims], kh[bi, hi][toks][:, dims])
            cand = toks[np.sort(topk_lowest_index(part[None], min(toks.size, n_req))[0])]
            full = (_seq_dot(q[bi, hi], kh[bi, hi][cand]) * np.float32(scaling)).astype(np.float32)
            keep = cand[topk_lowest_index(full[None], min(cand.size, n_keep))[0]]
            final_keep[bi, hi, keep] = True
    if sink > 0:
        final_keep[..., : min(sink, history)] = True
    if recent > 0:
        final_keep[..., max(0, history - recent):history] = True
    if keep_self:
        final_keep[..., history] = True
    idx = np.broadcast_to(np.arange(key_count), final_keep.shape)
    out = final_attention(q, kx, vx, idx, final_keep, scaling)
    return out, final_keep


def block_select_step_cpu(query_states, key_states, value_states, kind: str, block: int, dim_count: int,
                          scan_fraction: float, candidate_fraction: float, top_fraction: float, scaling: float,
                          sink: int = 0, recent: int = 0, keep_self: bool = True, reps: int = 1):
    """One qbb (EV:5516-5617), brep (EV:5369-5505, representatives as
    BlockRepState computes them, EV:1899-1913) or qboracle (EV:5008-5097)
    decode step in the reference's PyTorch ops on CPU tensors: the CPU baseline ``bench.py``
    times next to the GPU block selectors.  query_states [B,Hq,1,D];
    key/value_states [B,Hkv,T,D] (GQA-expanded first, EV:6248-6251).
    Returns (out [B,1,Hq,D], final_keep bool [B,Hq,T])."""
    import torch
    import torch.nn.functional as F

    b, hq, _, d = query_states.shape
    if key_states.shape[1] != hq:
        rep = hq // key_states.shape[1]
        key_states = key_states.repeat_interleave(rep, dim=1)
        value_states = value_states.repeat_interleave(rep, dim=1)
    key_count = key_states.shape[-2]
    history = key_count - 1
    sdims = min(max(1, dim_count), d)
    q = query_states[:, :, 0, :].float()
    qdims = torch.topk(q.abs(), k=sdims, dim=-1, largest=True).indices
    q_sel = torch.gather(q, dim=-1, index=qdims)
    k_hist = key_states[:, :, :history, :]
    nb = math.ceil(history / block)
    padded = nb * block
    k_blocks = F.pad(k_hist.float(), (0, 0, 0, padded - history), value=0.0) if padded != history else k_hist.float()
    valid_b = torch.zeros((b, hq, padded), dtype=torch.bool)
    valid_b[:, :, :history] = True
    block_k = k_blocks.view(b, hq, nb, block, d)
    block_valid = valid_b.view(b, hq, nb, block)
    if kind == "qboracle":
        # partial scores of every history token, -inf padding, block max (EV:5030-5044)
        kall = torch.gather(k_hist.float(), dim=-1, index=qdims[:, :, None, :].expand(-1, -1, history, -1))
        part_all = (kall * q_sel[:, :, None, :]).sum(dim=-1)
        pscores = F.pad(part_all, (0, padded - history), value=-torch.inf) if padded != history else part_all
        bscore = pscores.view(b, hq, nb, block).amax(dim=-1)
    elif kind == "qbb":
        gidx = qdims[:, :, None, None, :].expand(-1, -1, nb, block, -1)
        sel = torch.gather(block_k, dim=-1, index=gidx)
        smax = sel.masked_fill(~block_valid[..., None], -torch.inf).amax(dim=3)
        smin = sel.masked_fill(~block_valid[..., None], torch.inf).amin(dim=3)
        qb = q_sel[:, :, None, :]
        bscore = torch.where(qb >= 0, qb * smax, qb * smin).sum(dim=-1)
    else:
        r = min(reps, block)
        norms = block_k.square().sum(dim=-1).masked_fill(~block_valid, -torch.inf)
        _, rpos = torch.topk(norms, k=r, dim=-1, largest=True)
        rkeys = torch.gather(block_k, dim=3, index=rpos[..., None].expand(-1, -1, -1, -1, d))
        rvalid = torch.gather(block_valid, dim=3, index=rpos)
        rsel = torch.gather(rkeys, dim=-1, index=qdims[:, :, None, None, :].expand(-1, -1, nb, r, -1))
        rsc = (rsel * q_sel[:, :, None, None, :]).sum(dim=-1).masked_fill(~rvalid, torch.finfo(torch.float32).min)
        bscore = rsc.amax(dim=-1)
    n_scan = min(nb, max(1, math.ceil(scan_fraction * history / block)))
    _, blocks = torch.topk(bscore, k=n_scan, dim=-1, largest=True)
    if kind == "qboracle":
        # candidates over the whole history, unscanned tokens at finfo.min,
        # which isfinite() keeps valid (EV:5048-5058)
        scan_blocks = torch.zeros((b, hq, nb), dtype=torch.bool).scatter_(-1, blocks, True)
        scan_keep = scan_blocks.repeat_interleave(block, dim=-1)[..., :history]
        cpart = part_all.masked_fill(~scan_keep, torch.finfo(part_all.dtype).min)
        req = min(history, max(1, math.ceil(candidate_fraction * history)))
        cps, ctok = torch.topk(cpart, k=req, dim=-1, largest=True)
        cvalid = torch.isfinite(cps)
    else:
        tok = (blocks[..., None] * block + torch.arange(block)).reshape(b, hq, -1)
        tvalid = tok < history
        tok = tok.clamp_max(history - 1)
        skeys = torch.gather(k_hist, dim=2, index=tok[..., None].expand(-1, -1, -1, d))
        ssel = torch.gather(skeys.float(), dim=-1, index=qdims[:, :, None, :].expand(-1, -1, tok.shape[-1], -1))
        part = (ssel * q_sel[:, :, None, :]).sum(dim=-1).masked_fill(~tvalid, torch.finfo(torch.float32).min)
        req = min(tok.shape[-1], max(1, math.ceil(candidate_fraction * history)))
        _, cpos = torch.topk(part, k=req, dim=-1, largest=True)
        ctok = torch.gather(tok, dim=-1, index=cpos)
        cvalid = torch.gather(tvalid, dim=-1, index=cpos)
    ckeys = torch.gather(k_hist, dim=2, index=ctok[..., None].expand(-1, -1, -1, d))
    cs = torch.matmul(query_states[:, :, 0:1, :], ckeys.transpose(2, 3)).squeeze(2) * scaling
    cs = cs.masked_fill(~cvalid, torch.finfo(cs.dtype).min)
    keep_n = min(cs.shape[-1], max(1, math.ceil(top_fraction * history)))
    _, kpos = torch.topk(cs, k=keep_n, dim=-1, largest=True)
    final_keep = torch.zeros((b, hq, key_count), dtype=torch.bool)
    final_keep[:, :, :history].scatter_(dim=-1, index=torch.gather(ctok, -1, kpos), src=torch.gather(cvalid, -1, kpos))
    if sink > 0:
        final_keep[:, :, : min(sink, history)] = True
    if recent > 0:
        final_keep[:, :, max(0, history - recent):history] = True
    if keep_self:
        final_keep[:, :, history] = True
    # gather attention over the mask (EV:5607-5617, via _indices_from_keep_mask)
    width = int(final_keep.sum(dim=-1).max().item())
    pos = torch.arange(key_count).view(1, 1, -1).expand_as(final_keep)
    fidx = torch.topk(torch.where(final_keep, pos, torch.full_like(pos, -1)), k=width, dim=-1).values
    fvalid = fidx >= 0
    fidx = fidx.clamp_min(0)
    g = fidx[..., None].expand(-1, -1, -1, d)
    sk, sv = torch.gather(key_states, 2, g), torch.gather(value_states, 2, g)
    att = torch.matmul(query_states[:, :, 0:1, :], sk.transpose(2, 3)).squeeze(2) * scaling
    att = att.masked_fill(~fvalid, torch.finfo(att.dtype).min)
    w = F.softmax(att, dim=-1, dtype=torch.float32).to(query_states.dtype)
    out = torch.sum(w[:, :, :, None] * sv, dim=2)
    return out[:, None, :, :].contiguous(), final_keep
