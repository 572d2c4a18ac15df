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
