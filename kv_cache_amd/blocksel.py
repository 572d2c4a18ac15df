"""Block selectors: the reference's ``qbb{bs}q{S}s{scan}cand{c}``
(Quest-style per-block channel bounds), ``brep{bs}r{R}q{S}s{scan}cand{c}``
(block representatives) and ``qboracle{bs}q{S}s{scan}cand{c}`` (block maxima
of the partial scores, EV:5008-5097) decode steps on MI355X.

Per layer and decode token the reference ("EV" =
evaluate_qwen3_top2_head_limit3_ppl.py) scores every block of the history by
metadata — the bound sum_s q_s * (q_s >= 0 ? max : min) over each block's
per-channel extremes on the S largest-|q| dims (EV:5508-5617), or the best
partial score of the block's R largest-norm tokens (EV:5361-5505, kept in
``BlockRepState``, EV:1853-1918) — keeps the ``ceil(scan * history / bs)`` best
blocks, scores their tokens on the S dims, keeps the ``ceil(cand * history)``
best, reranks those by the full-D score and keeps ``ceil(top * history)``,
then attends over them plus the sink / recent tokens and the current token.

``BlockSelectDecodeStep`` runs that step with libqkv kernels on GQA-shaped K/V
(no ``repeat_interleave``).  The metadata lives on the GPU per KV head and is
rebuilt only for the blocks new tokens touch (the reference recomputes the
qbb extremes from all of K every step); the block tokens' partial scores read
a dim-major K copy, where a block's tokens are contiguous.
"""

from __future__ import annotations

import math
import re

import torch

from . import _lib
from .int4 import block_topk, topk_workspace
from .reuse import dim_major_append, token_attention

QBB, BREP = 0, 1   # QKV_BLOCK_QBB, QKV_BLOCK_BREP
QBORACLE = 2       # block maxima of the partial scores: no per-block metadata


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _pct(x: str) -> float:
    return float(x.replace("p", ".")) / 100.0


def parse_block_mode(mode: str) -> tuple[int, int, int, int, float, float]:
    """``qbb{bs}q{S}s{scan}cand{c}`` / ``brep{bs}r{R}q{S}s{scan}cand{c}`` /
    ``qboracle{bs}q{S}s{scan}cand{c}`` -> (kind, block, reps, dims, scan
    fraction, candidate fraction), with the reference's readings
    (parse_qbb_params EV:856-864, parse_brep_params EV:835-844,
    parse_qboracle_params EV:798-806: block and reps at least 1, ``p`` as the
    decimal point)."""
    m = re.fullmatch(r"qbb(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)", mode)
    if m:
        return QBB, max(1, int(m.group(1))), 1, int(m.group(2)), _pct(m.group(3)), _pct(m.group(4))
    m = re.fullmatch(r"qboracle(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)", mode)
    if m:   # parse_qboracle_params, EV:798-806
        return QBORACLE, max(1, int(m.group(1))), 1, int(m.group(2)), _pct(m.group(3)), _pct(m.group(4))
    m = re.fullmatch(r"brep(\d+)r(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)", mode)
    _require(m is not None, f"{mode!r} is not a qbb, brep or qboracle mode")
    return (BREP, max(1, int(m.group(1))), max(1, int(m.group(2))), int(m.group(3)), _pct(m.group(4)),
            _pct(m.group(5)))


def step_counts(history: int, block: int, scan: float, cand: float, top: float,
                unscanned: bool = False) -> tuple[int, int, int, int]:
    """(blocks, scanned blocks, candidates, kept) for a history, as the
    reference computes them (EV:5535, 5563, 5583, 5590).  qbb / brep rank
    the scanned tokens only; qboracle (``unscanned``) ranks every history
    token (EV:5055-5058)."""
    nb = math.ceil(history / block)
    n_scan = min(nb, max(1, math.ceil(scan * history / block)))
    n_req = max(1, math.ceil(cand * history))
    n_cand = min(history, n_req) if unscanned else min(n_scan * block, n_req)
    n_keep = min(n_cand, max(1, math.ceil(top * history)))
    return nb, n_scan, n_cand, n_keep


class BlockSelectDecodeStep:
    """One layer's qbb / brep / qboracle decode step with its block metadata, for
    K/V caches [B, Hkv, T, 128] of up to ``capacity`` tokens in ``dtype``
    (bf16 or fp16; the query and the output share it).  Call it once
    per decode token with the cache including the current token; a call
    whose history is not the previous call's plus one starts a new sequence
    (the metadata and the dim-major copy are rebuilt)."""

    def __init__(self, mode: str, batch: int, q_heads: int, kv_heads: int, head_dim: int, capacity: int, *,
                 top_fraction: float = 0.02, protect_sink: int = 0, protect_recent: int = 0,
                 keep_self: bool = True, device: torch.device | str = "cuda", dtype: torch.dtype = torch.bfloat16):
        lib = _lib.load()
        _require(dtype in (torch.bfloat16, torch.float16), f"dtype must be bfloat16 or float16, got {dtype}")
        self.dtype = dtype
        self.dtype_code = _lib.DTYPE_CODES[dtype]
        self.mode = mode
        self.kind, self.block, reps, self.dims, self.scan, self.cand = parse_block_mode(mode)
        self.reps = max(1, min(reps, self.block))
        _require(self.reps <= 64, f"{mode}: at most 64 representatives per block")
        _require(head_dim == 128, "block selectors need head_dim 128")
        _require(q_heads % kv_heads == 0, "q_heads must be a multiple of kv_heads")
        self.batch, self.q_heads, self.kv_heads, self.head_dim = batch, q_heads, kv_heads, head_dim
        self.capacity = int(capacity)
        self.top_fraction = float(top_fraction)
        self.sink, self.recent, self.keep_self = max(0, int(protect_sink)), max(0, int(protect_recent)), bool(keep_self)
        self.device = device
        rows = batch * q_heads
        self.rows = rows
        cap = self.capacity
        self.meta_blocks = math.ceil(cap / self.block)
        if self.kind == QBORACLE:   # scores every block from the dim-major copy
            self.meta = None
        else:
            nbytes = lib.qkv_block_meta_bytes(self.kind, batch, kv_heads, self.meta_blocks, self.reps)
            _require(nbytes > 0, "bad block metadata size")
            self.meta = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self.kdm = torch.empty((batch, kv_heads, head_dim, cap), dtype=dtype, device=device)
        self.unscanned = self.kind == QBORACLE
        nb, n_scan, n_cand, n_keep = step_counts(cap - 1, self.block, self.scan, self.cand, self.top_fraction,
                                                 self.unscanned)
        # rows past the one-workgroup rerank (more than 40960 scanned tokens or
        # 4096 candidates, qboracle candidates past the scanned tokens) rerank
        # over this workspace; sized at the capacity, grown if a shorter history needs more
        need = lib.qkv_block_rerank_workspace_bytes(rows, cap - 1, n_scan, self.block, n_cand, n_keep,
                                                    int(self.unscanned))
        _require(need >= 0, "bad rerank sizes")
        self.rerank_ws = torch.empty(max(1, (need + 3) // 4), dtype=torch.float32, device=device)
        self.bscore = torch.empty((rows, self.meta_blocks), dtype=torch.float32, device=device)
        self.blocks = torch.empty(rows * n_scan, dtype=torch.int32, device=device)
        self.topk_ws = topk_workspace(rows, self.meta_blocks, n_scan, device)
        self.partial = torch.empty(rows * n_scan * self.block, dtype=torch.float32, device=device)
        self.full = torch.empty_like(self.partial)   # full-D scores of the scanned tokens (rerank's candidates)
        self.keep = torch.zeros((rows, cap), dtype=torch.uint8, device=device)
        self.n_out_max = int(lib.qkv_final_list_count(cap - 1, n_keep, self.sink, self.recent, int(self.keep_self)))
        self.attn_ids = torch.empty(rows * self.n_out_max, dtype=torch.int32, device=device)
        need = lib.qkv_sparse_attention_workspace_bytes(batch, q_heads, q_heads, head_dim, self.n_out_max, 1)
        self.attn_ws = torch.zeros((need + 3) // 4, dtype=torch.float32, device=device)
        self.out = torch.empty((batch, q_heads, head_dim), dtype=dtype, device=device)
        self.reset()

    def reset(self) -> None:
        """Forget the metadata and the dim-major copy (a new sequence)."""
        self.meta_len = 0
        self.kdm_len = 0
        self.last_history = None

    def _sync_cache(self, key: torch.Tensor, history: int) -> None:
        lib = _lib.load()
        if self.meta_len < history and self.meta is None:
            self.meta_len = history
        if self.meta_len < history:
            with _lib.on_device(key.device):
                _lib.check(lib.qkv_block_meta_update(
                    self.kind, key.data_ptr(), _lib.strides(*key.stride()), self.batch, self.kv_heads, self.head_dim,
                    self.block, self.reps, self.meta_len, history, self.meta.data_ptr(), self.meta_blocks,
                    self.dtype_code, _lib.stream_of(key)))
            self.meta_len = history
        if self.kdm_len < history:
            dim_major_append(key, self.kdm, self.kdm_len, history)
            self.kdm_len = history

    def prefill(self, key: torch.Tensor) -> None:
        """Build the metadata and the dim-major copy of the cached tokens."""
        self._sync_cache(key, key.size(2))

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float) -> torch.Tensor:
        """query [B, Hq, 128]; key/value [B, Hkv, T, 128], the current token
        last, all in the step's dtype.  Returns [B, Hq, 128] in that dtype."""
        key_count = key.size(2)
        _require(key_count <= self.capacity, f"cache holds {key_count} tokens, capacity {self.capacity}")
        _require(query.dtype == key.dtype == value.dtype == self.dtype,
                 f"this step takes {self.dtype} q/K/V (got {query.dtype}, {key.dtype}, {value.dtype})")
        g = self.q_heads // self.kv_heads
        if key_count <= 1:   # EV:5523-5525
            self.out.copy_(value[:, :, -1, :].repeat_interleave(g, dim=1))
            return self.out
        history = key_count - 1
        if self.last_history is not None and history != self.last_history + 1:
            self.reset()     # not the next token of the last sequence: a new sequence
        if self.meta_len > history or self.kdm_len > history:
            self.reset()
        self._sync_cache(key, history)
        self.last_history = history
        return self.launch(query, key, value, scaling)

    def launch(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float) -> torch.Tensor:
        """The step's selection and attention kernels at the history
        key.size(2) - 1, with the metadata and the dim-major copy already
        holding it (``__call__`` brings them up to date first)."""
        lib = _lib.load()
        key_count = key.size(2)
        history = key_count - 1
        _require(self.meta_len >= history and self.kdm_len >= history, "block metadata does not hold the history")
        q = query.contiguous()
        nb, n_scan, n_cand, n_keep = step_counts(history, self.block, self.scan, self.cand, self.top_fraction,
                                                 self.unscanned)
        stream = _lib.stream_of(q)
        ks = _lib.strides(*key.stride())
        ws_need = int(lib.qkv_block_rerank_workspace_bytes(self.rows, history, n_scan, self.block, n_cand, n_keep,
                                                           int(self.unscanned)))
        _require(ws_need >= 0, "bad rerank sizes")
        if ws_need > self.rerank_ws.numel() * 4:
            self.rerank_ws = torch.empty((ws_need + 3) // 4, dtype=torch.float32, device=q.device)
        with _lib.on_device(q.device):
            if self.kind == QBORACLE:
                _lib.check(lib.qkv_block_max_partial_scores(
                    q.data_ptr(), self.kdm.data_ptr(), _lib.strides(*self.kdm.stride()), self.batch, self.q_heads,
                    self.kv_heads, history, self.head_dim, self.block, self.dims, self.bscore.data_ptr(),
                    self.meta_blocks, self.dtype_code, stream))
            else:
                _lib.check(lib.qkv_block_scores(
                    self.kind, q.data_ptr(), key.data_ptr(), ks, self.meta.data_ptr(), self.meta_blocks, self.batch,
                    self.q_heads, self.kv_heads, history, self.head_dim, self.block, self.reps, self.dims,
                    self.bscore.data_ptr(), self.meta_blocks, self.dtype_code, stream))
            blocks = self.blocks[: self.rows * n_scan].view(self.rows, n_scan)
            block_topk(self.bscore[:, :nb], n_scan, out=blocks, workspace=self.topk_ws)
            n_tok = n_scan * self.block
            partial = self.partial[: self.rows * n_tok]
            # the one-workgroup rerank ranks its candidates by the full scores the
            # scan computes for every scanned token; the general one (ws_need > 0)
            # computes them for its candidates only
            full = self.full[: self.rows * n_tok] if ws_need == 0 else None
            _lib.check(lib.qkv_block_scan_scores(
                q.data_ptr(), self.kdm.data_ptr(), _lib.strides(*self.kdm.stride()), key.data_ptr(), ks, self.batch,
                self.q_heads, self.kv_heads, history, self.head_dim, blocks.data_ptr(), n_scan, self.block,
                self.dims, float(scaling), partial.data_ptr(), _lib.ptr(full), n_tok, self.dtype_code, stream))
            n_out = int(lib.qkv_final_list_count(history, n_keep, self.sink, self.recent, int(self.keep_self)))
            ids = self.attn_ids[: self.rows * n_out]
            _lib.check(lib.qkv_block_rerank(
                q.data_ptr(), key.data_ptr(), ks, self.batch, self.q_heads, self.kv_heads, key_count, self.head_dim,
                partial.data_ptr(), _lib.ptr(full), n_tok, blocks.data_ptr(), n_scan, self.block, n_cand, n_keep,
                self.sink, self.recent, int(self.keep_self), float(scaling), self.keep.data_ptr(), self.capacity,
                ids.data_ptr(), n_out, int(self.unscanned), self.rerank_ws.data_ptr(), self.rerank_ws.numel() * 4,
                self.dtype_code, stream))
        self.n_out = n_out
        self.key_count = key_count
        return token_attention(q, key, value, ids.view(self.rows, n_out), scaling, workspace=self.attn_ws,
                               out=self.out)

    def final_mask(self) -> torch.Tensor:
        """The last step's final keep mask, bool [B, Hq, key_count]."""
        return self.keep[:, : self.key_count].view(torch.bool).view(self.batch, self.q_heads, self.key_count)
