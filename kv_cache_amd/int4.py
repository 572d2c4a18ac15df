"""Host API of the int4 sparse-attention KV-retrieval path on MI355X.

The path (no int4 counterpart in the reference; its fp32 equivalent is the
``qabs{S}cand{pct}attn`` / ``qboracle`` decode of evaluate_qwen3_top2_head_
limit3_ppl.py:4400-4502 and 5008-5097):

1. ``int4_pack_k``      -- K (bf16 or fp16) -> symmetric int4, fp16 scale per group.
2. ``select_channels``  -- per KV head, the S channels of largest mean |K|.
3. ``build_slab``       -- those S channels re-quantized as one int4 group:
                           the S/2 + 2 bytes per token that decode scoring streams
                           (codes swizzled in 4 KiB tiles, scales in key order).
4. ``decode_scores``    -- GQA-summed int8 query . int4 slab -> int32, ranking
                           key fp32(scale) * I, max-pooled per block
                           (``query_words`` exposes the int8 query alone).
5. ``block_topk``       -- top-k blocks, lowest index wins ties, ascending.
6. ``sparse_attention`` -- every query head of a KV head attends over the
                           selected blocks of K/V.

All tensors live on the GPU; every function launches on the current stream
and raises ``RuntimeError`` on bad input or a missing library (there is no
CPU fallback).  Layouts: K/V [B, Hkv, T, D] with contiguous channels, in
bf16 or fp16 (the query, K, V and the attention output share one dtype);
packed/slab tensors [B, Hkv, capacity, ...] with capacity a multiple of 512
(the slab's [B, Hkv, capacity, S/2] bytes hold the swizzled tile layout, so
the per-key view of it is not meaningful without un-swizzling).
"""

from __future__ import annotations

import math

import torch

from . import _lib

# Token capacity of packed K / slab buffers: a multiple of the largest slab
# tile (8192/S keys at S = 16), so one capacity serves every channel count.
CAPACITY_MULTIPLE = 512


def round_capacity(tokens: int) -> int:
    return max(CAPACITY_MULTIPLE, -(-int(tokens) // CAPACITY_MULTIPLE) * CAPACITY_MULTIPLE)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_kv(name: str, t: torch.Tensor) -> int:
    """Checks a K/V tensor; returns its dtype code."""
    _require(t.is_cuda, f"{name} must be CUDA")
    code = _lib.half_code(name, t)
    _require(t.dim() == 4, f"{name} must have shape [batch, kv_heads, tokens, dim]")
    _require(t.stride(3) == 1, f"{name} channels must be contiguous")
    return code


def _check_query(query: torch.Tensor) -> int:
    _require(query.is_cuda and query.dim() == 3, "query must be CUDA [B,Hq,D]")
    return _lib.half_code("query", query)


def _check_qkv(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> int:
    code = _check_kv("key", key)
    _check_kv("value", value)
    _check_query(query)
    _require(query.dtype == key.dtype == value.dtype,
             f"query, key and value must share one dtype (got {query.dtype}, {key.dtype}, {value.dtype})")
    _require(key.stride() == value.stride() and key.shape == value.shape, "key/value layout mismatch")
    return code


def int4_pack_k(key: torch.Tensor, group: int, *, capacity: int | None = None,
                packed: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                t_begin: int = 0, t_end: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize tokens [t_begin, t_end) of K into (packed uint8 [B,Hkv,cap,D/2],
    scales fp16 [B,Hkv,cap,D/group]); existing outputs are written in place."""
    lib = _lib.load()
    code = _check_kv("key", key)
    b, h, t, d = key.shape
    t_end = t if t_end is None else int(t_end)
    if packed is None or scales is None:
        cap = round_capacity(t) if capacity is None else int(capacity)
        packed = torch.empty((b, h, cap, d // 2), dtype=torch.uint8, device=key.device)
        scales = torch.empty((b, h, cap, d // group), dtype=torch.float16, device=key.device)
    cap = packed.size(2)
    _require(packed.is_contiguous() and scales.is_contiguous(), "packed/scales must be contiguous")
    _require(tuple(packed.shape) == (b, h, cap, d // 2), "packed shape mismatch")
    _require(tuple(scales.shape) == (b, h, cap, d // group), "scales shape mismatch")
    with _lib.on_device(key.device):
        _lib.check(lib.qkv_int4_pack_k(key.data_ptr(), _lib.strides(*key.stride()[:3]), b, h, int(t_begin),
                                       t_end, d, int(group), packed.data_ptr(), scales.data_ptr(), cap, code,
                                       _lib.stream_of(key)))
    return packed, scales


def select_channels(packed: torch.Tensor, scales: torch.Tensor, tokens: int, group: int,
                    count: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per (b, kv head): the ``count`` channels of largest exact mean
    |dequantized K| over tokens [0, tokens), ties to the lower channel, in
    ascending order.  Returns (chan_idx int32 [B,Hkv,count], stats int64
    [B,Hkv,D] holding the uint64 statistic)."""
    lib = _lib.load()
    _require(packed.is_cuda and packed.dtype == torch.uint8 and packed.is_contiguous(), "bad packed K")
    b, h, cap, half = packed.shape
    d = half * 2
    stats = torch.empty((b, h, d), dtype=torch.int64, device=packed.device)
    chan = torch.empty((b, h, int(count)), dtype=torch.int32, device=packed.device)
    with _lib.on_device(packed.device):
        _lib.check(lib.qkv_int4_select_channels(packed.data_ptr(), scales.data_ptr(), b * h, int(tokens), cap,
                                                d, int(group), int(count), stats.data_ptr(), chan.data_ptr(),
                                                _lib.stream_of(packed)))
    return chan, stats


def build_slab(key: torch.Tensor, chan_idx: torch.Tensor, *, capacity: int | None = None,
               slab: torch.Tensor | None = None, slab_scales: torch.Tensor | None = None,
               t_begin: int = 0, t_end: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Subset slab of tokens [t_begin, t_end): (slab uint8 [B,Hkv,cap,S/2],
    slab_scales fp16 [B,Hkv,cap])."""
    lib = _lib.load()
    code = _check_kv("key", key)
    b, h, t, d = key.shape
    _require(chan_idx.dtype == torch.int32 and chan_idx.is_contiguous(), "chan_idx must be contiguous int32")
    s = chan_idx.size(-1)
    t_end = t if t_end is None else int(t_end)
    if slab is None or slab_scales is None:
        cap = round_capacity(t) if capacity is None else int(capacity)
        slab = torch.empty((b, h, cap, s // 2), dtype=torch.uint8, device=key.device)
        slab_scales = torch.empty((b, h, cap), dtype=torch.float16, device=key.device)
    cap = slab.size(2)
    with _lib.on_device(key.device):
        _lib.check(lib.qkv_int4_build_slab(key.data_ptr(), _lib.strides(*key.stride()[:3]), b, h, int(t_begin),
                                           t_end, d, chan_idx.data_ptr(), s, slab.data_ptr(),
                                           slab_scales.data_ptr(), cap, code, _lib.stream_of(key)))
    return slab, slab_scales


def query_words(query: torch.Tensor, chan_idx: torch.Tensor, *, qwords: torch.Tensor | None = None,
                qscale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Per-row int8 query of decode scoring: (qwords int32 [B,Hkv,S/4] holding
    the packed uint32 words, qscale f32 [B,Hkv] or None)."""
    lib = _lib.load()
    code = _check_query(query)
    q = query.contiguous()
    b, hq, d = q.shape
    _require(chan_idx.dtype == torch.int32 and chan_idx.is_contiguous() and chan_idx.dim() == 3,
             "chan_idx must be contiguous int32 [B,Hkv,S]")
    hkv, s = chan_idx.size(1), chan_idx.size(2)
    _require(chan_idx.size(0) == b, "chan_idx batch mismatch")
    if qwords is None:
        qwords = torch.empty((b, hkv, s // 4), dtype=torch.int32, device=q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_int4_query_words(q.data_ptr(), b, hq, hkv, d, chan_idx.data_ptr(), s,
                                            qwords.data_ptr(), _lib.ptr(qscale), code, _lib.stream_of(q)))
    return qwords, qscale


def decode_scores(query: torch.Tensor, chan_idx: torch.Tensor, slab: torch.Tensor,
                  slab_scales: torch.Tensor, tokens: int, block: int, *,
                  bmax: torch.Tensor | None = None, debug: bool = False):
    """Fused int4 scoring + block max over tokens [0, tokens).

    query bf16 or fp16 [B, Hq, D].  Returns bmax f32 [B, Hkv, ceil(tokens/block)];
    with ``debug=True`` returns (bmax, isum int32 [B,Hkv,T], keys f32
    [B,Hkv,T], qscale f32 [B,Hkv])."""
    lib = _lib.load()
    code = _check_query(query)
    _require(slab.is_cuda and slab.dtype == torch.uint8 and slab.is_contiguous(), "slab must be contiguous CUDA uint8")
    q = query.contiguous()
    b, hq, d = q.shape
    _, hkv, cap, half = slab.shape
    s = half * 2
    _require(tuple(chan_idx.shape) == (b, hkv, s) and chan_idx.dtype == torch.int32 and chan_idx.is_contiguous(),
             "chan_idx must be contiguous int32 [B,Hkv,S]")
    nb = -(-int(tokens) // int(block))
    if bmax is None:
        bmax = torch.empty((b, hkv, nb), dtype=torch.float32, device=q.device)
    isum = keys = qscale = None
    if debug:
        isum = torch.empty((b, hkv, int(tokens)), dtype=torch.int32, device=q.device)
        keys = torch.empty((b, hkv, int(tokens)), dtype=torch.float32, device=q.device)
        qscale = torch.empty((b, hkv), dtype=torch.float32, device=q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_int4_decode_scores(q.data_ptr(), b, hq, hkv, d, chan_idx.data_ptr(), s, slab.data_ptr(),
                                              slab_scales.data_ptr(), cap, int(tokens), int(block),
                                              bmax.data_ptr(), _lib.ptr(isum), _lib.ptr(keys),
                                              _lib.ptr(qscale), code, _lib.stream_of(q)))
    if debug:
        return bmax, isum, keys, qscale
    return bmax


def decode_topk(query: torch.Tensor, chan_idx: torch.Tensor, slab: torch.Tensor, slab_scales: torch.Tensor,
                tokens: int, k: int, *, scores: torch.Tensor | None = None, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``decode_scores`` with block 1 then ``block_topk`` in one call
    (qkv_int4_decode_topk): the top-k token indices int32 [B, Hkv, k],
    ascending, lowest index first among equal scores; the token scores go to
    ``scores`` f32 [B, Hkv, tokens].  Long rows build the top-k's chunk
    histograms while they score."""
    lib = _lib.load()
    code = _check_query(query)
    _require(slab.is_cuda and slab.dtype == torch.uint8 and slab.is_contiguous(), "slab must be contiguous CUDA uint8")
    q = query.contiguous()
    b, hq, d = q.shape
    _, hkv, cap, half = slab.shape
    s = half * 2
    _require(tuple(chan_idx.shape) == (b, hkv, s) and chan_idx.dtype == torch.int32 and chan_idx.is_contiguous(),
             "chan_idx must be contiguous int32 [B,Hkv,S]")
    t = int(tokens)
    if scores is None:
        scores = torch.empty((b, hkv, t), dtype=torch.float32, device=q.device)
    _require(scores.dtype == torch.float32 and scores.is_contiguous() and scores.numel() >= b * hkv * t
             and scores.size(-1) == t, "scores must be contiguous float32 [B,Hkv,tokens]")
    if out is None:
        out = torch.empty((b, hkv, int(k)), dtype=torch.int32, device=q.device)
    need = lib.qkv_topk_workspace_bytes(b * hkv, t, int(k))
    _require(need >= 0, f"bad top-k sizes tokens={t} k={k}")
    if need > 0 and (workspace is None or workspace.numel() * 4 < need):
        workspace = topk_workspace(b * hkv, t, k, q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_int4_decode_topk(q.data_ptr(), b, hq, hkv, d, chan_idx.data_ptr(), s, slab.data_ptr(),
                                            slab_scales.data_ptr(), cap, t, int(k), scores.data_ptr(), out.data_ptr(),
                                            _lib.ptr(workspace), 0 if workspace is None else workspace.numel() * 4,
                                            code, _lib.stream_of(q)))
    return out


def topk_workspace(rows: int, n: int, k: int, device) -> torch.Tensor | None:
    """Workspace for ``block_topk`` on rows of n values (None when not needed)."""
    need = _lib.load().qkv_topk_workspace_bytes(int(rows), int(n), int(k))
    _require(need >= 0, f"bad top-k sizes rows={rows} n={n} k={k}")
    return torch.empty((need + 3) // 4, dtype=torch.float32, device=device) if need else None


def block_topk(values: torch.Tensor, k: int, *, out: torch.Tensor | None = None,
               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Top-k indices along the last axis, lowest index wins ties, ascending order (int32).
    Rows longer than 4096 values use a staged selection with a workspace
    (allocated here unless one from ``topk_workspace`` is passed)."""
    lib = _lib.load()
    _require(values.is_cuda and values.dtype == torch.float32, "values must be CUDA float32")
    n = values.size(-1)
    v2 = values.reshape(-1, n)
    _require(v2.stride(1) == 1, "values must be contiguous along the last axis")
    rows = v2.size(0)
    if out is None:
        out = torch.empty((*values.shape[:-1], int(k)), dtype=torch.int32, device=values.device)
    need = lib.qkv_topk_workspace_bytes(rows, n, int(k))
    with _lib.on_device(values.device):
        if need > 0:
            if workspace is None or workspace.numel() * 4 < need:
                workspace = topk_workspace(rows, n, k, values.device)
            _lib.check(lib.qkv_topk_ws(v2.data_ptr(), rows, n, v2.stride(0), int(k), out.data_ptr(),
                                       workspace.data_ptr(), workspace.numel() * 4, _lib.stream_of(values)))
        else:
            _lib.check(lib.qkv_topk(v2.data_ptr(), rows, n, v2.stride(0), int(k), out.data_ptr(),
                                    _lib.stream_of(values)))
    return out


def attention_workspace_bytes(batch: int, q_heads: int, kv_heads: int, head_dim: int, n_sel: int,
                              block: int) -> int:
    n = _lib.load().qkv_sparse_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, n_sel, block)
    _require(n >= 0, "unsupported sparse-attention configuration")
    return int(n)


def attention_workspace(batch: int, q_heads: int, kv_heads: int, head_dim: int, n_sel: int, block: int,
                        device) -> torch.Tensor:
    """Zero-filled workspace for ``sparse_attention`` calls with these
    heads and at most n_sel * block selected slots.  Its leading ticket words must be zero before the first call; every
    completed call leaves them zero, so one workspace serves any number of
    calls.  Calls sharing a workspace must not overlap in time."""
    need = attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, n_sel, block)
    return torch.zeros((need + 3) // 4, dtype=torch.float32, device=device)


def protected_count(history: int, protect_sink: int = 0, protect_recent: int = 0, keep_self: bool = False) -> int:
    """Tokens the reference adds to every selection (EV:2938-2982): the sink
    range, the recent range (not overlapping the sink) and the current token."""
    if not (protect_sink > 0 or protect_recent > 0 or keep_self):
        return 0
    n = _lib.load().qkv_final_list_count(int(history), 0, int(protect_sink), int(protect_recent), int(bool(keep_self)))
    _require(n >= 0, f"bad history {history}")
    return int(n)


def protected_workspace_blocks(n_sel: int, block: int, history: int, protect_sink: int = 0,
                               protect_recent: int = 0, keep_self: bool = False) -> int:
    """Selection size whose attention workspace also covers the protected slots."""
    return int(n_sel) + -(-protected_count(history, protect_sink, protect_recent, keep_self) // int(block))


def _protected(protect_sink: int, protect_recent: int, keep_self: bool) -> bool:
    return protect_sink > 0 or protect_recent > 0 or bool(keep_self)


def _output(out: torch.Tensor | None, q: torch.Tensor) -> torch.Tensor:
    """The attention output [B,Hq,D] in q's dtype: ``out`` checked, or a new tensor."""
    if out is None:
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _require(out.dtype == q.dtype and tuple(out.shape) == tuple(q.shape) and out.is_contiguous(),
             f"out must be contiguous {q.dtype} {tuple(q.shape)}")
    return out


def sparse_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                     block_ids: torch.Tensor, block: int, tokens: int, scaling: float, *,
                     workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                     protect_sink: int = 0, protect_recent: int = 0, keep_self: bool = False) -> torch.Tensor:
    """GQA-native attention of query [B,Hq,D] over the selected blocks
    (int32 [B,Hkv,n]) of K/V [B,Hkv,*,D]; returns [B,Hq,D].  query, K, V and
    the output share one dtype, bf16 or fp16.

    With protection (the reference's --protect_sink_tokens,
    --protect_recent_tokens, --always_keep_self; EV:2938-2982) ``tokens`` is
    the history the blocks were chosen from, and the attention also covers
    the sink range, the recent range and the current token ``tokens`` (each
    token once; K/V then hold tokens + 1 rows)."""
    lib = _lib.load()
    code = _check_qkv(query, key, value)
    q = query.contiguous()
    b, hq, d = q.shape
    hkv = key.size(1)
    _require(block_ids.dtype == torch.int32 and block_ids.is_contiguous(), "block_ids must be contiguous int32")
    n = block_ids.size(-1)
    prot = _protected(protect_sink, protect_recent, keep_self)
    _require(not keep_self or key.size(2) > int(tokens), "keep_self needs the current token's K/V row")
    n_ws = protected_workspace_blocks(n, block, tokens, protect_sink, protect_recent, keep_self) if prot else n
    if workspace is None:
        workspace = attention_workspace(b, hq, hkv, d, n_ws, block, q.device)
    out = _output(out, q)
    with _lib.on_device(q.device):
        if prot:
            _lib.check(lib.qkv_sparse_attention_protected(
                q.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.strides(*key.stride()[:3]), b, hq, hkv,
                int(tokens), d, block_ids.data_ptr(), None, 0, n, int(block), int(protect_sink), int(protect_recent),
                int(bool(keep_self)), float(scaling), workspace.data_ptr(), workspace.numel() * 4, None,
                out.data_ptr(), code, _lib.stream_of(q)))
        else:
            _lib.check(lib.qkv_sparse_attention(q.data_ptr(), key.data_ptr(), value.data_ptr(),
                                                _lib.strides(*key.stride()[:3]), b, hq, hkv, int(tokens), d,
                                                block_ids.data_ptr(), n, int(block), float(scaling),
                                                workspace.data_ptr(), workspace.numel() * 4, out.data_ptr(),
                                                code, _lib.stream_of(q)))
    return out


# Rows of at most this many blocks can select inside the attention kernel.
SELECT_MAX_BLOCKS = 4096


def sparse_attention_select(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            bmax: torch.Tensor, n_sel: int, block: int, tokens: int, scaling: float, *,
                            workspace: torch.Tensor | None = None, sel_out: torch.Tensor | None = None,
                            out: torch.Tensor | None = None, protect_sink: int = 0, protect_recent: int = 0,
                            keep_self: bool = False) -> torch.Tensor:
    """``sparse_attention`` over the n_sel blocks with the largest block
    maxima (f32 [B,Hkv,>=ceil(tokens/block)], the selection of ``block_topk``),
    selected inside the attention kernel.  sel_out (int32 [B,Hkv,n_sel]), when
    given, receives the selection.  Protection and dtypes as for
    ``sparse_attention``.  Returns [B,Hq,D] in the query's dtype."""
    lib = _lib.load()
    code = _check_qkv(query, key, value)
    q = query.contiguous()
    b, hq, d = q.shape
    hkv = key.size(1)
    _require(bmax.is_cuda and bmax.dtype == torch.float32, "bmax must be CUDA float32")
    nb = math.ceil(int(tokens) / int(block))
    _require(bmax.dim() == 3 and bmax.shape[:2] == (b, hkv) and bmax.size(2) >= nb and bmax.stride(2) == 1
             and bmax.stride(1) == bmax.size(2) and bmax.stride(0) == hkv * bmax.size(2),
             "bmax must be contiguous [B, Hkv, >= blocks]")
    if sel_out is not None:
        _require(sel_out.dtype == torch.int32 and sel_out.is_contiguous() and sel_out.numel() == b * hkv * n_sel,
                 "sel_out must be contiguous int32 [B, Hkv, n_sel]")
    prot = _protected(protect_sink, protect_recent, keep_self)
    _require(not keep_self or key.size(2) > int(tokens), "keep_self needs the current token's K/V row")
    n_ws = protected_workspace_blocks(n_sel, block, tokens, protect_sink, protect_recent, keep_self) if prot else n_sel
    if workspace is None:
        workspace = attention_workspace(b, hq, hkv, d, n_ws, block, q.device)
    out = _output(out, q)
    with _lib.on_device(q.device):
        if prot:
            _lib.check(lib.qkv_sparse_attention_protected(
                q.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.strides(*key.stride()[:3]), b, hq, hkv,
                int(tokens), d, None, bmax.data_ptr(), bmax.size(2), int(n_sel), int(block), int(protect_sink),
                int(protect_recent), int(bool(keep_self)), float(scaling), workspace.data_ptr(),
                workspace.numel() * 4, _lib.ptr(sel_out), out.data_ptr(), code, _lib.stream_of(q)))
        else:
            _lib.check(lib.qkv_sparse_attention_select(
                q.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.strides(*key.stride()[:3]), b, hq, hkv,
                int(tokens), d, bmax.data_ptr(), bmax.size(2), int(n_sel), int(block), float(scaling),
                workspace.data_ptr(), workspace.numel() * 4, _lib.ptr(sel_out), out.data_ptr(), code,
                _lib.stream_of(q)))
    return out


class Int4KCache:
    """int4 view of one layer's K cache: packed K, the static channel subset
    of every KV head, and the subset slab decode scoring streams.

    Built once from the prefill K (``from_prefill``); the reference keeps the
    analogous per-layer state in ``SparQMeanState.key_dim_major``
    (evaluate_qwen3_top2_head_limit3_ppl.py:2018-2042)."""

    def __init__(self, packed, scales, chan_idx, slab, slab_scales, tokens, group):
        self.packed, self.scales = packed, scales
        self.chan_idx = chan_idx
        self.slab, self.slab_scales = slab, slab_scales
        self.tokens = int(tokens)
        self.group = int(group)

    @property
    def capacity(self) -> int:
        return self.slab.size(2)

    @property
    def selected(self) -> int:
        return self.chan_idx.size(-1)

    @classmethod
    def from_prefill(cls, key: torch.Tensor, group: int, selected: int,
                     capacity: int | None = None) -> "Int4KCache":
        t = key.size(2)
        cap = round_capacity(t) if capacity is None else int(capacity)
        packed, scales = int4_pack_k(key, group, capacity=cap)
        chan, _ = select_channels(packed, scales, t, group, selected)
        slab, slab_scales = build_slab(key, chan, capacity=cap)
        return cls(packed, scales, chan, slab, slab_scales, t, group)


class SparseDecodeStep:
    """One layer's decode step with every buffer allocated up front:
    scoring + block max -> top-k blocks -> GQA sparse attention.

    ``tokens`` is the cache length the step runs at.  With protection (the
    reference's --protect_sink_tokens, --protect_recent_tokens,
    --always_keep_self) or ``history_only``, the step follows the
    reference's decode semantics (EV:4419-4460): the blocks are chosen over
    the history ``tokens - 1`` (the current token is not a candidate), and the
    attention covers them plus the sink range, the recent range and, with
    keep_self, the current token, each token once (EV:2938-2982).  ``dtype``
    (bf16 or fp16) is the query / K / V / output dtype the step runs on."""

    def __init__(self, batch: int, q_heads: int, kv_heads: int, head_dim: int, tokens: int,
                 block: int, topk: int, device: torch.device | str = "cuda", *, protect_sink: int = 0,
                 protect_recent: int = 0, keep_self: bool = False, history_only: bool | None = None,
                 dtype: torch.dtype = torch.bfloat16):
        self.batch, self.q_heads, self.kv_heads = batch, q_heads, kv_heads
        self.head_dim, self.tokens, self.block, self.topk = head_dim, tokens, block, topk
        self.protect_sink, self.protect_recent = max(0, int(protect_sink)), max(0, int(protect_recent))
        self.keep_self = bool(keep_self)
        prot = _protected(self.protect_sink, self.protect_recent, self.keep_self)
        self.history_only = prot if history_only is None else bool(history_only)
        _require(self.history_only or not prot, "protected tokens need history_only (the current token is not scored)")
        self.scored = tokens - 1 if self.history_only else tokens   # keys the selection ranks
        _require(self.scored >= 1, f"no keys to select from at {tokens} tokens")
        nb = math.ceil(self.scored / block)
        _require(1 <= topk <= nb, f"topk {topk} must be in [1, {nb}]")
        self.bmax = torch.empty((batch, kv_heads, nb), dtype=torch.float32, device=device)
        self.sel = torch.empty((batch, kv_heads, topk), dtype=torch.int32, device=device)
        self.topk_ws = topk_workspace(batch * kv_heads, nb, topk, device)
        n_ws = protected_workspace_blocks(topk, block, self.scored, self.protect_sink, self.protect_recent,
                                          self.keep_self)
        self.workspace = attention_workspace(batch, q_heads, kv_heads, head_dim, n_ws, block, device)
        _require(dtype in (torch.bfloat16, torch.float16), f"dtype must be bfloat16 or float16, got {dtype}")
        self.out = torch.empty((batch, q_heads, head_dim), dtype=dtype, device=device)
        self.fused = nb <= SELECT_MAX_BLOCKS

    @classmethod
    def for_mode(cls, mode: str, batch: int, q_heads: int, kv_heads: int, head_dim: int, tokens: int,
                 device: torch.device | str = "cuda", *, protect_sink: int = 0, protect_recent: int = 0,
                 keep_self: bool = True, dtype: torch.dtype = torch.bfloat16) -> "SparseDecodeStep":
        """The int4 step for a reference mode string at a cache of ``tokens``
        keys (the current token included): ``qabs{S}cand{pct}attn`` keeps
        ``ceil(pct * history)`` tokens (one-token blocks), ``qboracle{bs}q{S}
        s{scan}cand{pct}`` the ``ceil(scan * history / bs)`` best blocks; both
        add the protected tokens (the reference's defaults: no sink or recent
        tokens, keep the current token) and select over the history only.
        What stays the int4 path's own is the scoring: one GQA-summed int8
        query per KV head over a static channel subset, instead of the
        reference's per-head top-|q| channels in fp32, so the G heads of a KV
        head share their selection.  The cache must have ``plan.selected``
        channels (``modes.decode_plan``)."""
        from .modes import decode_plan

        plan = decode_plan(mode, tokens, head_dim)
        _require(plan is not None, f"mode {mode!r} is not a decode mode of this path (or no history yet)")
        step = cls(batch, q_heads, kv_heads, head_dim, tokens, plan.block,
                   min(plan.topk, math.ceil(plan.history / plan.block)), device, protect_sink=protect_sink,
                   protect_recent=protect_recent, keep_self=keep_self, history_only=True, dtype=dtype)
        step.plan = plan
        return step

    def __call__(self, query: torch.Tensor, cache: Int4KCache, key: torch.Tensor, value: torch.Tensor,
                 scaling: float) -> torch.Tensor:
        """Rows of at most SELECT_MAX_BLOCKS blocks select inside the attention
        kernel (two launches); longer rows run the top-k launch between.  The
        selection lands in ``self.sel`` either way."""
        _require(key.size(2) >= self.tokens, f"K/V hold {key.size(2)} tokens, the step needs {self.tokens}")
        _require(query.dtype == self.out.dtype, f"this step runs on {self.out.dtype}; got a {query.dtype} query")
        prot = dict(protect_sink=self.protect_sink, protect_recent=self.protect_recent, keep_self=self.keep_self)
        if self.fused:
            decode_scores(query, cache.chan_idx, cache.slab, cache.slab_scales, self.scored, self.block,
                          bmax=self.bmax)
            return sparse_attention_select(query, key, value, self.bmax, self.topk, self.block, self.scored,
                                           scaling, workspace=self.workspace, sel_out=self.sel, out=self.out, **prot)
        if self.block == 1:   # token selection: the scoring launch feeds the top-k its chunk histograms
            decode_topk(query, cache.chan_idx, cache.slab, cache.slab_scales, self.scored, self.topk,
                        scores=self.bmax, out=self.sel, workspace=self.topk_ws)
        else:
            decode_scores(query, cache.chan_idx, cache.slab, cache.slab_scales, self.scored, self.block,
                          bmax=self.bmax)
            block_topk(self.bmax, self.topk, out=self.sel, workspace=self.topk_ws)
        return sparse_attention(query, key, value, self.sel, self.block, self.scored, scaling,
                                workspace=self.workspace, out=self.out, **prot)
