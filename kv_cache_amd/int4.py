"""Host API of the int4 sparse-attention KV-retrieval path on MI355X.

The path (no int4 counterpart in the reference; its fp32 equivalent is the
``qabs{S}cand{pct}attn`` / ``qboracle`` decode of evaluate_qwen3_top2_head_
limit3_ppl.py:4400-4502 and 5008-5097):

1. ``int4_pack_k``      -- K bf16 -> symmetric int4, fp16 scale per group.
2. ``select_channels``  -- per KV head, the S channels of largest mean |K|.
3. ``build_slab``       -- those S channels re-quantized as one int4 group:
                           the S/2 + 2 bytes per token that decode scoring streams
                           (codes swizzled in 4 KiB tiles, scales in key order).
4. ``decode_scores``    -- GQA-summed int8 query . int4 slab -> int32, ranking
                           key fp32(scale) * I, max-pooled per block
                           (``query_words`` exposes the int8 query alone).
5. ``block_topk``       -- top-k blocks, lowest index wins ties, ascending.
6. ``sparse_attention`` -- every query head of a KV head attends over the
                           selected blocks of bf16 K/V.

All tensors live on the GPU; every function launches on the current stream
and raises ``RuntimeError`` on bad input or a missing library (there is no
CPU fallback).  Layouts: K/V [B, Hkv, T, D] bf16 with contiguous channels;
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


def _check_kv(name: str, t: torch.Tensor) -> None:
    _require(t.is_cuda, f"{name} must be CUDA")
    _require(t.dtype == torch.bfloat16, f"{name} must be bfloat16")
    _require(t.dim() == 4, f"{name} must have shape [batch, kv_heads, tokens, dim]")
    _require(t.stride(3) == 1, f"{name} channels must be contiguous")


def int4_pack_k(key: torch.Tensor, group: int, *, capacity: int | None = None,
                packed: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                t_begin: int = 0, t_end: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize tokens [t_begin, t_end) of K into (packed uint8 [B,Hkv,cap,D/2],
    scales fp16 [B,Hkv,cap,D/group]); existing outputs are written in place."""
    lib = _lib.load()
    _check_kv("key", key)
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
    with torch.cuda.device(key.device):
        _lib.check(lib.qkv_int4_pack_k(key.data_ptr(), _lib.strides(*key.stride()[:3]), b, h, int(t_begin),
                                       t_end, d, int(group), packed.data_ptr(), scales.data_ptr(), cap,
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
    with torch.cuda.device(packed.device):
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
    _check_kv("key", key)
    b, h, t, d = key.shape
    _require(chan_idx.dtype == torch.int32 and chan_idx.is_contiguous(), "chan_idx must be contiguous int32")
    s = chan_idx.size(-1)
    t_end = t if t_end is None else int(t_end)
    if slab is None or slab_scales is None:
        cap = round_capacity(t) if capacity is None else int(capacity)
        slab = torch.empty((b, h, cap, s // 2), dtype=torch.uint8, device=key.device)
        slab_scales = torch.empty((b, h, cap), dtype=torch.float16, device=key.device)
    cap = slab.size(2)
    with torch.cuda.device(key.device):
        _lib.check(lib.qkv_int4_build_slab(key.data_ptr(), _lib.strides(*key.stride()[:3]), b, h, int(t_begin),
                                           t_end, d, chan_idx.data_ptr(), s, slab.data_ptr(),
                                           slab_scales.data_ptr(), cap, _lib.stream_of(key)))
    return slab, slab_scales


def query_words(query: torch.Tensor, chan_idx: torch.Tensor, *, qwords: torch.Tensor | None = None,
                qscale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Per-row int8 query of decode scoring: (qwords int32 [B,Hkv,S/4] holding
    the packed uint32 words, qscale f32 [B,Hkv] or None)."""
    lib = _lib.load()
    _require(query.is_cuda and query.dtype == torch.bfloat16 and query.dim() == 3, "query must be CUDA bf16 [B,Hq,D]")
    q = query.contiguous()
    b, hq, d = q.shape
    _require(chan_idx.dtype == torch.int32 and chan_idx.is_contiguous() and chan_idx.dim() == 3,
             "chan_idx must be contiguous int32 [B,Hkv,S]")
    hkv, s = chan_idx.size(1), chan_idx.size(2)
    _require(chan_idx.size(0) == b, "chan_idx batch mismatch")
    if qwords is None:
        qwords = torch.empty((b, hkv, s // 4), dtype=torch.int32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.check(lib.qkv_int4_query_words(q.data_ptr(), b, hq, hkv, d, chan_idx.data_ptr(), s,
                                            qwords.data_ptr(), _lib.ptr(qscale), _lib.stream_of(q)))
    return qwords, qscale


def decode_scores(query: torch.Tensor, chan_idx: torch.Tensor, slab: torch.Tensor,
                  slab_scales: torch.Tensor, tokens: int, block: int, *,
                  bmax: torch.Tensor | None = None, debug: bool = False):
    """Fused int4 scoring + block max over tokens [0, tokens).

    query bf16 [B, Hq, D].  Returns bmax f32 [B, Hkv, ceil(tokens/block)];
    with ``debug=True`` returns (bmax, isum int32 [B,Hkv,T], keys f32
    [B,Hkv,T], qscale f32 [B,Hkv])."""
    lib = _lib.load()
    _require(query.is_cuda and query.dtype == torch.bfloat16 and query.dim() == 3, "query must be CUDA bf16 [B,Hq,D]")
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
    with torch.cuda.device(q.device):
        _lib.check(lib.qkv_int4_decode_scores(q.data_ptr(), b, hq, hkv, d, chan_idx.data_ptr(), s, slab.data_ptr(),
                                              slab_scales.data_ptr(), cap, int(tokens), int(block),
                                              bmax.data_ptr(), _lib.ptr(isum), _lib.ptr(keys),
                                              _lib.ptr(qscale), _lib.stream_of(q)))
    if debug:
        return bmax, isum, keys, qscale
    return bmax


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
    with torch.cuda.device(values.device):
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


def sparse_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                     block_ids: torch.Tensor, block: int, tokens: int, scaling: float, *,
                     workspace: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """GQA-native attention of query bf16 [B,Hq,D] over the selected blocks
    (int32 [B,Hkv,n]) of K/V bf16 [B,Hkv,*,D]; returns bf16 [B,Hq,D]."""
    lib = _lib.load()
    _check_kv("key", key)
    _check_kv("value", value)
    _require(key.stride() == value.stride() and key.shape == value.shape, "key/value layout mismatch")
    q = query.contiguous()
    b, hq, d = q.shape
    hkv = key.size(1)
    _require(block_ids.dtype == torch.int32 and block_ids.is_contiguous(), "block_ids must be contiguous int32")
    n = block_ids.size(-1)
    need = attention_workspace_bytes(b, hq, hkv, d, n, block)
    if workspace is None:
        workspace = attention_workspace(b, hq, hkv, d, n, block, q.device)
    if out is None:
        out = torch.empty((b, hq, d), dtype=torch.bfloat16, device=q.device)
    with torch.cuda.device(q.device):
        _lib.check(lib.qkv_sparse_attention(q.data_ptr(), key.data_ptr(), value.data_ptr(),
                                            _lib.strides(*key.stride()[:3]), b, hq, hkv, int(tokens), d,
                                            block_ids.data_ptr(), n, int(block), float(scaling),
                                            workspace.data_ptr(), workspace.numel() * 4, out.data_ptr(),
                                            _lib.stream_of(q)))
    return out


# Rows of at most this many blocks can select inside the attention kernel.
SELECT_MAX_BLOCKS = 4096


def sparse_attention_select(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            bmax: torch.Tensor, n_sel: int, block: int, tokens: int, scaling: float, *,
                            workspace: torch.Tensor | None = None, sel_out: torch.Tensor | None = None,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """``sparse_attention`` over the n_sel blocks with the largest block
    maxima (f32 [B,Hkv,>=ceil(tokens/block)], the selection of ``block_topk``),
    selected inside the attention kernel.  sel_out (int32 [B,Hkv,n_sel]), when
    given, receives the selection.  Returns bf16 [B,Hq,D]."""
    lib = _lib.load()
    _check_kv("key", key)
    _check_kv("value", value)
    _require(key.stride() == value.stride() and key.shape == value.shape, "key/value layout mismatch")
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
    if workspace is None:
        workspace = attention_workspace(b, hq, hkv, d, n_sel, block, q.device)
    if out is None:
        out = torch.empty((b, hq, d), dtype=torch.bfloat16, device=q.device)
    with torch.cuda.device(q.device):
        _lib.check(lib.qkv_sparse_attention_select(
            q.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.strides(*key.stride()[:3]), b, hq, hkv,
            int(tokens), d, bmax.data_ptr(), bmax.size(2), int(n_sel), int(block), float(scaling),
            workspace.data_ptr(), workspace.numel() * 4, _lib.ptr(sel_out), out.data_ptr(), _lib.stream_of(q)))
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
    scoring + block max -> top-k blocks -> GQA sparse attention."""

    def __init__(self, batch: int, q_heads: int, kv_heads: int, head_dim: int, tokens: int,
                 block: int, topk: int, device: torch.device | str = "cuda"):
        self.batch, self.q_heads, self.kv_heads = batch, q_heads, kv_heads
        self.head_dim, self.tokens, self.block, self.topk = head_dim, tokens, block, topk
        nb = math.ceil(tokens / block)
        _require(1 <= topk <= nb, f"topk {topk} must be in [1, {nb}]")
        self.bmax = torch.empty((batch, kv_heads, nb), dtype=torch.float32, device=device)
        self.sel = torch.empty((batch, kv_heads, topk), dtype=torch.int32, device=device)
        self.topk_ws = topk_workspace(batch * kv_heads, nb, topk, device)
        self.workspace = attention_workspace(batch, q_heads, kv_heads, head_dim, topk, block, device)
        self.out = torch.empty((batch, q_heads, head_dim), dtype=torch.bfloat16, device=device)
        self.fused = nb <= SELECT_MAX_BLOCKS

    @classmethod
    def for_mode(cls, mode: str, batch: int, q_heads: int, kv_heads: int, head_dim: int, tokens: int,
                 device: torch.device | str = "cuda") -> "SparseDecodeStep":
        """The step for a reference mode string (``qabs{S}cand{pct}attn`` or
        ``qboracle{bs}q{S}s{scan}cand{pct}``) at ``tokens`` keys; the cache it
        runs on must have ``plan.selected`` channels (``modes.decode_plan``)."""
        from .modes import decode_plan

        plan = decode_plan(mode, tokens, head_dim)
        _require(plan is not None, f"mode {mode!r} is not a decode mode of this path (or no history yet)")
        step = cls(batch, q_heads, kv_heads, head_dim, tokens, plan.block,
                   min(plan.topk, math.ceil(tokens / plan.block)), device)
        step.plan = plan
        return step

    def __call__(self, query: torch.Tensor, cache: Int4KCache, key: torch.Tensor, value: torch.Tensor,
                 scaling: float) -> torch.Tensor:
        """Rows of at most SELECT_MAX_BLOCKS blocks select inside the attention
        kernel (two launches); longer rows run the top-k launch between.  The
        selection lands in ``self.sel`` either way."""
        decode_scores(query, cache.chan_idx, cache.slab, cache.slab_scales, self.tokens, self.block,
                      bmax=self.bmax)
        if self.fused:
            return sparse_attention_select(query, key, value, self.bmax, self.topk, self.block, self.tokens,
                                           scaling, workspace=self.workspace, sel_out=self.sel, out=self.out)
        block_topk(self.bmax, self.topk, out=self.sel, workspace=self.topk_ws)
        return sparse_attention(query, key, value, self.sel, self.block, self.tokens, scaling,
                                workspace=self.workspace, out=self.out)
