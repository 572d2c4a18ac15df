"""Candidate reuse and exact rerank: the reference's
``qabs{S}cand{pct}reuse[final|2set][blk{bs}]`` decode step on MI355X.

Per layer and decode token the reference (``_qabs_reuse_fast_attention_forward``,
evaluate_qwen3_top2_head_limit3_ppl.py:3991-4397, "EV") scores every history
token on the S largest-|q| dims of each query head, keeps the
``ceil(cand * history)`` best as the current candidates, unions them with the
previous step's candidates and/or final selection, reranks the union by the
full-D score, keeps ``ceil(top_fraction * history)`` of it, and attends over
that selection plus the protected sink/recent tokens and the current token.
The previous masks live in ``ReuseCandidateState`` (EV:1596-1759).

``ReuseDecodeStep`` runs that step with libqkv kernels on GQA-shaped K/V (no
``repeat_interleave``): the dim-major K copy for the partial scores
(``qkv_dim_major_append``, EV:2018-2042), ``qkv_reuse_partial_scores``,
``qkv_threshold_mask``, ``qkv_reuse_select`` (+ ``qkv_reuse_expand_blocks``
for the blk modes) and ``qkv_token_attention``.
The masks stay on the GPU in capacity-sized buffers; nothing is allocated per
step once the step is built.
"""

from __future__ import annotations

import ctypes

import math
import re

import torch

from . import _lib


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _dtype_code(t: torch.Tensor) -> int:
    code = _lib.DTYPE_CODES.get(t.dtype)
    _require(code is not None, f"unsupported dtype {t.dtype}")
    return code


def budget_count(history: int, fraction: float) -> int:
    """``min(history, max(1, ceil(fraction * history)))`` (EV:4132, 4270)."""
    return min(int(history), max(1, math.ceil(float(fraction) * int(history))))


def parse_reuse_mode(mode: str) -> tuple[int, float, bool, bool, int | None]:
    """``qabs{S}cand{pct}reuse[final|2set][blk{bs}]`` -> (S, candidate
    fraction, use the previous candidates, use the previous final selection,
    block size or None).  The percentage takes ``p`` as the decimal point
    (``cand6p25`` = 6.25 %), as ``parse_qabs_partial_rerank_params`` reads it
    (EV:748-754).  A mode ending in ``reusefinal`` drops the previous
    candidates and one ending in ``reuse2set`` the previous final selection
    (EV:955-960): the reference tests the suffix, so a ``finalblk`` or
    ``2setblk`` mode keeps both.  ``blk{bs}`` expands the final selection to
    aligned blocks of max(1, bs) positions (EV:757-761, 4314-4316)."""
    m = re.fullmatch(r"qabs(\d+)cand(\d+(?:p\d+)?)reuse(2set|final)?(?:blk(\d+))?", mode)
    _require(m is not None, f"{mode!r} is not a qabs{{S}}cand{{pct}}reuse[final|2set][blk{{bs}}] mode")
    frac = float(m.group(2).replace("p", ".")) / 100.0
    block = max(1, int(m.group(4))) if m.group(4) is not None else None
    return int(m.group(1)), frac, not mode.endswith("reusefinal"), not mode.endswith("reuse2set"), block


# Rows of at most this many history positions have their block expansion run by
# the final selection's launch (one 1024-thread workgroup per row holds the
# row's bitset in LDS); longer rows expand in a launch of their own.
BLOCK_BITS_MAX_HISTORY = 40960

CANDIDATE_SELECTIONS = {"topk": 0, "sample_quantile": 1, "previous_threshold": 2}   # QKV_CAND_*


def sample_columns(history: int, sample_size: int) -> torch.Tensor | None:
    """Sampled positions of the ``sample_quantile`` candidate selection, int32
    on the host: the reference's ``linspace(0, history - 1, steps)`` in
    float32, rounded and deduplicated (EV:3973-3981), by the same torch call
    (its float32 values at .5 ties are torch's own).  None when the sample
    covers the row."""
    count = min(int(history), max(1, int(sample_size)))
    if count >= history:
        return None
    cols = torch.linspace(0, history - 1, steps=count, dtype=torch.float32).round().long().unique()
    return cols.to(torch.int32)


class SampleColumnTable:
    """``sample_columns`` on the device, one row per history below
    ``capacity``: int32 [capacity, sample_size], row h padded with its last
    column, so a decode step reads its row in place (no per-token host copy
    inside a captured step).  A row is computed (by the same torch call as
    ``sample_columns``) and copied to the device on the first use of its
    history, so that use must not be inside a graph capture; the table belongs
    to the step that made it."""

    def __init__(self, capacity: int, sample_size: int, device):
        self.capacity = int(capacity)
        self.size = max(1, int(sample_size))
        self.rows = torch.empty((self.capacity, self.size), dtype=torch.int32, device=device)
        self._counts: dict[int, int] = {}

    @property
    def max_count(self) -> int:
        """Largest column count of any row (0 when every row's sample covers it)."""
        return self.size if self.capacity - 1 > self.size else 0

    FILL = 64   # rows filled per miss: a decode step's next histories come with it

    def count(self, history: int) -> int:
        """Columns of ``history``'s sample (0 when the sample covers the row)."""
        h = int(history)
        n = self._counts.get(h)
        if n is None:
            _require(0 <= h < self.capacity, f"history {h} outside the table (capacity {self.capacity})")
            # this row and the next ones not yet filled, staged in pinned memory
            # and copied in one asynchronous transfer (a pageable copy per row
            # would wait for the stream's earlier work at every decode step)
            end = h + 1
            while end < min(h + self.FILL, self.capacity) and end not in self._counts:
                end += 1
            host = torch.empty((end - h, self.size), dtype=torch.int32, pin_memory=self.rows.is_cuda)
            for j in range(h, end):
                cols = sample_columns(j, self.size) if j else None
                c = 0 if cols is None else cols.numel()
                if c:
                    host[j - h, :c] = cols
                    host[j - h, c:] = cols[-1]
                self._counts[j] = c
            self.rows[h:end].copy_(host, non_blocking=True)
            n = self._counts[h]
        return n

    def row(self, history: int) -> torch.Tensor:
        """``history``'s row on the device (filled on first use)."""
        self.count(history)
        return self.rows[int(history)]


def candidate_mask(values: torch.Tensor, n: int, selection: str, k: int, mask: torch.Tensor,
                   thresholds: torch.Tensor | None, workspace: torch.Tensor, sample_cols: torch.Tensor | None = None,
                   n_sample: int = 0) -> torch.Tensor:
    """mask[:, :n] = values[:, :n] >= the row's threshold under ``selection``
    (EV:3958-3989): the k-th largest value (``topk``), the k-th largest of
    the ``n_sample`` columns ``sample_cols`` (``sample_quantile``), or
    ``thresholds`` as given (``previous_threshold``).  The first two write
    the threshold to ``thresholds`` (f32 [rows]; optional for ``topk``).
    ``mask`` is a byte mask (uint8 [rows, >= n]) or a bitset (int64 [rows,
    >= ceil(n / 64)] words, bit t % 64 of word t // 64)."""
    lib = _lib.load()
    code = CANDIDATE_SELECTIONS.get(selection)
    _require(code is not None, f"unknown candidate selection {selection!r}")
    _require(values.is_cuda and values.dtype == torch.float32 and values.dim() == 2 and values.stride(1) == 1
             and values.size(1) >= n, "values must be CUDA f32 [rows, >= n]")
    bits = mask.dtype == torch.int64
    _require(mask.dim() == 2 and mask.size(0) == values.size(0) and mask.stride(1) == 1
             and (mask.size(1) >= n if not bits else mask.size(1) * 64 >= n)
             and mask.dtype in (torch.uint8, torch.int64), "mask must be uint8 [rows, >= n] or int64 bit words")
    _require(thresholds is not None or selection == "topk", f"{selection} needs the thresholds array")
    _require(thresholds is None or (thresholds.dtype == torch.float32 and thresholds.is_contiguous()
                                    and thresholds.is_cuda and thresholds.numel() >= values.size(0)),
             "thresholds must be CUDA f32 [rows]")
    if selection == "sample_quantile":
        _require(sample_cols is not None and sample_cols.dtype == torch.int32 and sample_cols.is_contiguous()
                 and 1 <= n_sample <= sample_cols.numel(), "sample_cols must be int32 [>= n_sample]")
        if not sample_cols.is_cuda:   # host columns are checked, then copied (device ones must lie in [0, n))
            _require(bool(((sample_cols[:n_sample] >= 0) & (sample_cols[:n_sample] < n)).all()),
                     "sample_cols must lie in [0, n)")
            sample_cols = sample_cols.to(values.device)
    with _lib.on_device(values.device):
        _lib.check(lib.qkv_candidate_mask(
            values.data_ptr(), values.size(0), int(n), values.stride(0), code, int(k), _lib.ptr(sample_cols),
            int(n_sample), _lib.ptr(thresholds), None if bits else mask.data_ptr(), 0 if bits else mask.stride(0),
            mask.data_ptr() if bits else None, mask.stride(0) if bits else 0, workspace.data_ptr(),
            workspace.numel() * 4, _lib.stream_of(values)))
    return mask


def expand_bits(words: torch.Tensor, n: int) -> torch.Tensor:
    """bool [rows, n] from bitset words (int64 [rows, W], bit t % 64 of word t // 64)."""
    b = words.contiguous().view(torch.uint8).view(words.size(0), -1)
    shifts = torch.arange(8, dtype=torch.uint8, device=words.device)
    return ((b.unsqueeze(-1) >> shifts) & 1).view(words.size(0), -1)[:, :n].bool()


def reuse_partial_scores(query: torch.Tensor, key_dim_major: torch.Tensor, history: int, dim_count: int, *,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [B*Hq, >= history] partial scores over each head's top-|q| dims;
    key_dim_major [B, Hkv, D, *] with the token axis contiguous."""
    lib = _lib.load()
    q = query.contiguous()
    b, hq, d = q.shape
    hkv = key_dim_major.size(1)
    _require(q.is_cuda and key_dim_major.device == q.device, "query and key_dim_major must be on one CUDA device")
    _require(key_dim_major.dim() == 4 and key_dim_major.size(0) == b and key_dim_major.size(2) == d
             and key_dim_major.size(3) >= history and key_dim_major.dtype == q.dtype,
             "key_dim_major must be [B, Hkv, D, >= history] in the query dtype")
    if out is None:
        out = torch.empty((b * hq, history), dtype=torch.float32, device=q.device)
    _require(out.dtype == torch.float32 and out.dim() == 2 and out.size(0) == b * hq and out.size(1) >= history
             and out.stride(1) == 1, "out must be f32 [B*Hq, >= history]")
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_reuse_partial_scores(
            q.data_ptr(), key_dim_major.data_ptr(), _lib.strides(*key_dim_major.stride()), _dtype_code(q), b, hq,
            hkv, int(history), d, int(dim_count), out.data_ptr(), out.stride(0), _lib.stream_of(q)))
    return out


def threshold_mask(values: torch.Tensor, n: int, k: int, mask: torch.Tensor, workspace: torch.Tensor) -> torch.Tensor:
    """mask[:, :n] = values[:, :n] >= each row's k-th largest value."""
    lib = _lib.load()
    _require(values.is_cuda and values.dtype == torch.float32 and values.dim() == 2 and values.stride(1) == 1
             and values.size(1) >= n, "values must be CUDA f32 [rows, >= n]")
    _require(mask.dtype == torch.uint8 and mask.dim() == 2 and mask.size(0) == values.size(0) and mask.size(1) >= n
             and mask.stride(1) == 1, "mask must be uint8 [rows, >= n]")
    with _lib.on_device(values.device):
        _lib.check(lib.qkv_threshold_mask(values.data_ptr(), values.size(0), int(n), values.stride(0), int(k),
                                          mask.data_ptr(), mask.stride(0), workspace.data_ptr(),
                                          workspace.numel() * 4, _lib.stream_of(values)))
    return mask


def expand_blocks(history_final: torch.Tensor, key_count: int, block: int, protect_sink: int, protect_recent: int,
                  top_fraction: float, keep_self: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Expands the final mask (uint8 [rows, >= history], in place) to whole
    aligned blocks and returns the final list (int64 indices, bool validity,
    int32 attention ids), [rows, n] with n from
    ``qkv_reuse_block_final_count`` (EV:4314-4316, 2914-2922, 2938-2982)."""
    lib = _lib.load()
    history = int(key_count) - 1
    _require(history_final.is_cuda and history_final.dtype == torch.uint8 and history_final.dim() == 2
             and history_final.stride(1) == 1 and history_final.size(1) >= history,
             "history_final must be CUDA uint8 [rows, >= history]")
    rows = history_final.size(0)
    n = int(lib.qkv_reuse_block_final_count(history, int(block), int(protect_sink), int(protect_recent),
                                            float(top_fraction), int(keep_self)))
    _require(n >= 0, "need history >= 1 and block >= 1")
    dev = history_final.device
    idx = torch.empty((rows, n), dtype=torch.int64, device=dev)
    valid = torch.empty((rows, n), dtype=torch.uint8, device=dev)
    ids = torch.empty((rows, n), dtype=torch.int32, device=dev)
    with _lib.on_device(dev):
        _lib.check(lib.qkv_reuse_expand_blocks(
            history_final.data_ptr(), history_final.stride(0), rows, int(key_count), int(block), int(protect_sink),
            int(protect_recent), float(top_fraction), int(keep_self), idx.data_ptr(), valid.data_ptr(),
            ids.data_ptr(), n, _lib.stream_of(history_final)))
    return idx, valid.view(torch.bool), ids


def dim_major_append(key: torch.Tensor, key_dim_major: torch.Tensor, t_begin: int, t_end: int) -> None:
    """key_dim_major[:, :, :, t] = key[:, :, t, :] for t in [t_begin, t_end)."""
    lib = _lib.load()
    b, hkv, _, d = key.shape
    _require(key.is_cuda and key_dim_major.device == key.device and key_dim_major.dtype == key.dtype,
             "key and key_dim_major must share a CUDA device and dtype")
    _require(0 <= t_begin <= t_end <= key.size(2), "token range outside the key cache")
    _require(key_dim_major.dim() == 4 and tuple(key_dim_major.shape[:3]) == (b, hkv, d)
             and key_dim_major.size(3) >= t_end, "key_dim_major must be [B, Hkv, D, >= t_end]")
    with _lib.on_device(key.device):
        _lib.check(lib.qkv_dim_major_append(
            key.data_ptr(), _lib.strides(*key.stride()), _dtype_code(key), b, hkv, d, int(t_begin), int(t_end),
            key_dim_major.data_ptr(), _lib.strides(*key_dim_major.stride()), _lib.stream_of(key)))


def token_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, token_ids: torch.Tensor,
                    scaling: float, *, workspace: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Each query head attends over its own token list (int32 [B*Hq, n], -1
    skipped) of its K/V head; [B, Hq, D] in the dtype q, K and V share (bf16
    or fp16)."""
    lib = _lib.load()
    q = query.contiguous()
    b, hq, d = q.shape
    code = _lib.half_code("query", q)
    _require(q.dtype == key.dtype == value.dtype,
             f"token attention takes one dtype for q/K/V (got {q.dtype}, {key.dtype}, {value.dtype})")
    _require(key.shape == value.shape and key.stride() == value.stride() and key.stride(3) == 1,
             "key/value layout mismatch")
    _require(token_ids.dtype == torch.int32 and token_ids.is_contiguous() and token_ids.numel() ==
             b * hq * token_ids.size(-1), "token_ids must be contiguous int32 [B*Hq, n]")
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
    _require(out.dtype == q.dtype and out.is_contiguous() and out.numel() == b * hq * d,
             f"out must be contiguous {q.dtype} [B, Hq, D]")
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_token_attention(
            q.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.strides(*key.stride()[:3]), b, hq, key.size(1),
            key.size(2), d, token_ids.data_ptr(), token_ids.size(-1), float(scaling), workspace.data_ptr(),
            workspace.numel() * 4, out.data_ptr(), code, _lib.stream_of(q)))
    return out


def _check_step_dtype(dtype: torch.dtype, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
    _require(query.dtype == key.dtype == value.dtype == dtype,
             f"this step takes {dtype} q/K/V (got {query.dtype}, {key.dtype}, {value.dtype})")


class ReuseDecodeStep:
    _BITSET = True   # candidate and final state as bitsets (subclasses with byte kernels turn it off)

    """One layer's reuse decode step with its state, for K/V caches of up to
    ``capacity`` tokens ([B, Hkv, T, D] as HF stores them, in ``dtype``: bf16
    or fp16, shared by the query and the output).

    Call it once per decode token with the cache including the current token
    (T = history + 1).  The previous step's masks are used when the previous
    call had history - 1 tokens (the ``query_token`` check of EV:1651); any
    other history starts a new sequence (the dim-major copy is rebuilt and no
    previous mask is read), so ``reset()`` is needed only to restart a
    sequence at the very next history length."""

    def __init__(self, mode: str, batch: int, q_heads: int, kv_heads: int, head_dim: int, capacity: int, *,
                 top_fraction: float = 0.02, protect_sink: int = 0, protect_recent: int = 0,
                 keep_self: bool = True, candidate_selection: str = "topk", threshold_sample_size: int = 256,
                 device: torch.device | str = "cuda", dtype: torch.dtype = torch.bfloat16,
                 fused_attention: bool = False):
        lib = _lib.load()
        _require(dtype in (torch.bfloat16, torch.float16), f"dtype must be bfloat16 or float16, got {dtype}")
        self.dtype = dtype
        self.device = device
        self.mode = mode
        # the final selection's workgroups running the attention too (one launch less);
        # measured slower than the separate attention kernel at batch 1 and 4 and equal at
        # 8, so off unless asked for
        self.fused_attention = bool(fused_attention)
        (self.dims, self.cand_fraction, self.use_prev_candidate, self.use_prev_final,
         self.block) = self._parse_mode(mode)
        _require(self.block is None or self.block <= 4096, "reuse blocks hold at most 4096 tokens")
        # --qabs_candidate_selection / --qabs_threshold_sample_size (EV:245-258, 3958-3989)
        _require(candidate_selection in CANDIDATE_SELECTIONS, f"unknown candidate selection {candidate_selection!r}")
        self.selection = candidate_selection
        self.sample_size = max(1, int(threshold_sample_size))
        _require(q_heads % kv_heads == 0, "q_heads must be a multiple of kv_heads")
        self.batch, self.q_heads, self.kv_heads, self.head_dim = batch, q_heads, kv_heads, head_dim
        self.capacity = int(capacity)
        self.top_fraction = float(top_fraction)
        self.sink, self.recent, self.keep_self = max(0, int(protect_sink)), max(0, int(protect_recent)), bool(keep_self)
        rows = batch * q_heads
        cap = self.capacity
        self.rows = rows
        self.kdm = torch.empty((batch, kv_heads, head_dim, cap), dtype=dtype, device=device)
        # candidate and final masks: bitsets (64 positions per int64 word)
        self.bits = self._BITSET
        if self.bits:
            words = -(-cap // 64)
            self.cand = [torch.zeros((rows, words), dtype=torch.int64, device=device) for _ in range(2)]
            self.fin = torch.zeros((rows, words), dtype=torch.int64, device=device)
        else:
            self.cand = [torch.zeros((rows, cap), dtype=torch.uint8, device=device) for _ in range(2)]
            self.fin = torch.zeros((rows, cap), dtype=torch.uint8, device=device)
        self.partial = torch.empty((rows, cap), dtype=torch.float32, device=device)
        # the last step's candidate threshold per row (EV:1744-1745), written by the
        # previous_threshold and sample_quantile selections
        self.thresholds = torch.zeros(rows, dtype=torch.float32, device=device)
        self.columns = (SampleColumnTable(cap, self.sample_size, device)
                        if self.selection == "sample_quantile" else None)
        hist_max = cap - 1
        # every term of the counts grows with the history
        self.n_out_max = max(self._final_count(hist_max), int(lib.qkv_reuse_final_count(
            hist_max, self.sink, self.recent, self.top_fraction, int(self.keep_self))))
        self.final_idx = torch.empty(rows * self.n_out_max, dtype=torch.int64, device=device)
        self.final_valid = torch.empty(rows * self.n_out_max, dtype=torch.uint8, device=device)
        self.attn_ids = torch.empty(rows * self.n_out_max, dtype=torch.int32, device=device)
        self.mask_ws = self._ws(lib.qkv_threshold_mask_workspace_bytes(rows, hist_max, budget_count(hist_max,
                                                                                                    self.cand_fraction)))
        # qkv_reuse_candidates' own workspace: zero-filled (its selection state
        # starts at zero and every call leaves it so)
        need = lib.qkv_reuse_candidates_workspace_bytes(rows, hist_max, budget_count(hist_max, self.cand_fraction))
        _require(need >= 0, "bad workspace size")
        self.cand_ws = torch.zeros(max(1, (need + 3) // 4), dtype=torch.float32, device=device)
        n_s_max = self.columns.max_count if self.columns is not None else 0
        if n_s_max:   # sized once for the largest sample, so a captured step never reallocates
            self.mask_ws = self._grow(self.mask_ws, lib.qkv_candidate_mask_workspace_bytes(
                rows, hist_max, CANDIDATE_SELECTIONS["sample_quantile"], budget_count(n_s_max, self.cand_fraction),
                n_s_max))
        self.select_ws = self._ws(lib.qkv_reuse_select_workspace_bytes(rows, hist_max, self.top_fraction))
        need = lib.qkv_sparse_attention_workspace_bytes(batch, q_heads, q_heads, head_dim, self.n_out_max, 1)
        _require(need > 0, "unsupported attention shape (head_dim must be 128)")
        self.attn_ws = torch.zeros((need + 3) // 4, dtype=torch.float32, device=device)
        self.out = torch.empty((batch, q_heads, head_dim), dtype=dtype, device=device)
        self.reset()

    def _parse_mode(self, mode: str) -> tuple[int, float, bool, bool, int | None]:
        return parse_reuse_mode(mode)

    def _final_count(self, history: int) -> int:
        """Entries per row of the step's final index list."""
        lib = _lib.load()
        if self.block is None:
            return int(lib.qkv_reuse_final_count(history, self.sink, self.recent, self.top_fraction,
                                                 int(self.keep_self)))
        return int(lib.qkv_reuse_block_final_count(history, self.block, self.sink, self.recent, self.top_fraction,
                                                   int(self.keep_self)))

    def _ws(self, nbytes: int) -> torch.Tensor:
        _require(nbytes >= 0, "bad workspace size")
        return torch.empty(max(1, (nbytes + 3) // 4), dtype=torch.float32, device=self.device)

    def _grow(self, ws: torch.Tensor, nbytes: int) -> torch.Tensor:
        return ws if ws.numel() * 4 >= nbytes else self._ws(nbytes)

    def reset(self) -> None:
        """Forget the previous step and the dim-major copy (a new sequence)."""
        for m in (*self.cand, self.fin):
            m.zero_()
        self.kdm_len = 0
        self.flip = 0
        self.last_history = None

    def prefill(self, key: torch.Tensor) -> None:
        """Build the dim-major copy of the cached history in one launch."""
        t = key.size(2)
        if t > self.kdm_len:
            dim_major_append(key, self.kdm, self.kdm_len, t)
            self.kdm_len = t

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float) -> torch.Tensor:
        """query [B, Hq, D]; key/value [B, Hkv, T, D] (the current token
        last), in the step's dtype.  Returns [B, Hq, D] in that dtype."""
        key_count = key.size(2)
        _require(key_count <= self.capacity, f"cache holds {key_count} tokens, capacity {self.capacity}")
        _check_step_dtype(self.dtype, query, key, value)
        g = self.q_heads // self.kv_heads
        if key_count <= 1:   # EV:4012-4014: only the current token
            self.out.copy_(value[:, :, -1, :].repeat_interleave(g, dim=1))
            return self.out
        history = key_count - 1
        if self.last_history is not None and history != self.last_history + 1:
            # not the next token of the last sequence: a new sequence, whose
            # dim-major copy and previous masks must not carry over
            self.reset()
        if self.kdm_len < history:
            dim_major_append(key, self.kdm, self.kdm_len, history)
            self.kdm_len = history
        consecutive = self.last_history == history - 1
        cur, prev = self.cand[self.flip], self.cand[1 - self.flip]
        self.launch(query, key, value, scaling, cur, prev if consecutive and self.use_prev_candidate else None,
                    self.fin if consecutive and self.use_prev_final else None,
                    previous_thresholds=consecutive and self.selection == "previous_threshold")
        self.flip ^= 1
        self.last_history = history
        return self.out

    def launch(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float,
               current: torch.Tensor, previous: torch.Tensor | None, previous_final: torch.Tensor | None, *,
               previous_thresholds: bool = False) -> None:
        """The step's kernels at the history key.size(2) - 1 with explicit
        mask buffers (the step's byte masks or bitsets): the current candidates go to
        ``current``, the final mask to the final buffer (it may also be the
        ``previous_final`` read).  With ``previous_thresholds`` the
        ``previous_threshold`` selection compares with the thresholds the last
        step left (else it selects as ``topk``).  Touches no Python state but
        ``n_out``; the dim-major copy must already hold the history.  Output
        in ``self.out``; the step's thresholds in ``self.thresholds``."""
        key_count = key.size(2)
        history = key_count - 1
        _require(self.kdm_len >= history, "the dim-major copy does not hold the history")
        q = query.contiguous()
        self._candidates(q, history, current, previous_thresholds)
        self._select_attend(q, key, value, scaling, current, previous, previous_final)

    def _candidates(self, q: torch.Tensor, history: int, current: torch.Tensor, previous_thresholds: bool) -> None:
        """Every row's partial scores and its candidate mask under the step's
        selection (EV:3958-3989, 4116-4145) into ``current``; the thresholds
        into ``self.thresholds`` where a later step reads them."""
        lib = _lib.load()
        requested = budget_count(history, self.cand_fraction)
        n_s = self.columns.count(history) if self.selection == "sample_quantile" else 0
        topk_path = not (self.selection == "previous_threshold" and previous_thresholds) and not n_s
        if not topk_path:
            reuse_partial_scores(q, self.kdm, history, self.dims, out=self.partial)
        if self.selection == "previous_threshold" and previous_thresholds:   # EV:3967-3971
            candidate_mask(self.partial, history, "previous_threshold", requested, current, self.thresholds,
                           self.mask_ws)
        elif n_s:                                                             # EV:3972-3987
            k_s = budget_count(n_s, self.cand_fraction)
            self.mask_ws = self._grow(self.mask_ws, lib.qkv_candidate_mask_workspace_bytes(
                self.rows, history, CANDIDATE_SELECTIONS["sample_quantile"], k_s, n_s))
            candidate_mask(self.partial, history, "sample_quantile", k_s, current, self.thresholds, self.mask_ws,
                           self.columns.row(history), n_s)
        else:                                                                 # EV:3988
            need = lib.qkv_reuse_candidates_workspace_bytes(self.rows, history, requested)
            if self.cand_ws.numel() * 4 < need:   # (a fresh workspace starts zero-filled)
                self.cand_ws = torch.zeros((need + 3) // 4, dtype=torch.float32, device=self.device)
            # partial scores, threshold and mask in one launch where a row fits one
            # workgroup; the threshold is kept only where a later step reads it
            with _lib.on_device(q.device):
                bits = current.dtype == torch.int64
                _lib.check(lib.qkv_reuse_candidates(
                    q.data_ptr(), self.kdm.data_ptr(), _lib.strides(*self.kdm.stride()), _dtype_code(q), self.batch,
                    self.q_heads, self.kv_heads, history, self.head_dim, self.dims, requested,
                    self.partial.data_ptr(), self.partial.stride(0), None if bits else current.data_ptr(),
                    0 if bits else current.stride(0), current.data_ptr() if bits else None,
                    current.stride(0) if bits else 0,
                    _lib.ptr(self.thresholds) if self.selection != "topk" else None, self.cand_ws.data_ptr(),
                    self.cand_ws.numel() * 4, _lib.stream_of(q)))

    def _select_attend(self, q: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float,
                       current: torch.Tensor, previous: torch.Tensor | None,
                       previous_final: torch.Tensor | None) -> None:
        """The rerank of the union, the final selection (into ``self.fin``),
        its block expansion and the attention over it (EV:4200-4397)."""
        lib = _lib.load()
        key_count = key.size(2)
        history = key_count - 1
        n_sel = int(lib.qkv_reuse_final_count(history, self.sink, self.recent, self.top_fraction, int(self.keep_self)))
        n_out = self._final_count(history)
        self.select_ws = self._grow(self.select_ws,
                                    lib.qkv_reuse_select_workspace_bytes(self.rows, history, self.top_fraction))
        ids = self.attn_ids[: self.rows * n_out]
        bits = current.dtype == torch.int64
        if bits and self.block is not None and history > BLOCK_BITS_MAX_HISTORY:
            # past one workgroup's row: the selection, then the expansion on the bitset
            with _lib.on_device(q.device):
                _lib.check(lib.qkv_reuse_select_bits(
                    q.data_ptr(), key.data_ptr(), _lib.strides(*key.stride()), _dtype_code(q), self.batch,
                    self.q_heads, self.kv_heads, key_count, self.head_dim, current.data_ptr(), _lib.ptr(previous),
                    _lib.ptr(previous_final), current.stride(0), self.sink, self.recent, self.top_fraction,
                    int(self.keep_self), float(scaling), self.select_ws.data_ptr(), self.select_ws.numel() * 4,
                    self.final_idx.data_ptr(), self.final_valid.data_ptr(), None, n_sel, self.fin.data_ptr(),
                    self.fin.stride(0), None, None, None, _lib.stream_of(q)))
                _lib.check(lib.qkv_reuse_expand_blocks_bits(
                    self.fin.data_ptr(), self.fin.stride(0), self.rows, key_count, self.block, self.sink,
                    self.recent, self.top_fraction, int(self.keep_self), self.final_idx.data_ptr(),
                    self.final_valid.data_ptr(), ids.data_ptr(), n_out, _lib.stream_of(q)))
            self._attend(q, key, value, ids, n_out, scaling)
            self.n_out = n_out
            return
        if bits and self.block is not None:   # the selection and its block expansion in one launch
            with _lib.on_device(q.device):
                _lib.check(lib.qkv_reuse_select_bits_blocks(
                    q.data_ptr(), key.data_ptr(), _lib.strides(*key.stride()), _dtype_code(q), self.batch,
                    self.q_heads, self.kv_heads, key_count, self.head_dim, current.data_ptr(), _lib.ptr(previous),
                    _lib.ptr(previous_final), current.stride(0), self.sink, self.recent, self.top_fraction,
                    int(self.keep_self), float(scaling), self.block, self.select_ws.data_ptr(),
                    self.select_ws.numel() * 4, self.final_idx.data_ptr(), self.final_valid.data_ptr(),
                    ids.data_ptr(), n_out, self.fin.data_ptr(), self.fin.stride(0), _lib.stream_of(q)))
            self._attend(q, key, value, ids, n_out, scaling)
            self.n_out = n_out
            return
        # on bitsets the final selection's workgroups can also run the attention
        attended = ctypes.c_int(0)
        extra = ((value.data_ptr(), self.out.data_ptr(), ctypes.byref(attended)) if self.fused_attention
                 else (None, None, None)) if bits else ()
        select = lib.qkv_reuse_select_bits if bits else lib.qkv_reuse_select
        _require(not bits or (value.shape == key.shape and value.stride() == key.stride()),
                 "key/value layout mismatch")
        with _lib.on_device(q.device):
            _lib.check(select(
                q.data_ptr(), key.data_ptr(), _lib.strides(*key.stride()), _dtype_code(q), self.batch, self.q_heads,
                self.kv_heads, key_count, self.head_dim, current.data_ptr(), _lib.ptr(previous),
                _lib.ptr(previous_final), current.stride(0), self.sink, self.recent, self.top_fraction,
                int(self.keep_self), float(scaling), self.select_ws.data_ptr(), self.select_ws.numel() * 4,
                self.final_idx.data_ptr(), self.final_valid.data_ptr(),
                ids.data_ptr() if self.block is None else None, n_sel, self.fin.data_ptr(), self.fin.stride(0),
                *extra, _lib.stream_of(q)))
            if self.block is not None:   # EV:4314-4316: the final selection grows to whole blocks
                _lib.check(lib.qkv_reuse_expand_blocks(
                    self.fin.data_ptr(), self.capacity, self.rows, key_count, self.block, self.sink, self.recent,
                    self.top_fraction, int(self.keep_self), self.final_idx.data_ptr(), self.final_valid.data_ptr(),
                    ids.data_ptr(), n_out, _lib.stream_of(q)))
        if not attended.value:
            self._attend(q, key, value, ids, n_out, scaling)
        self.n_out = n_out

    def _attend(self, q: torch.Tensor, key: torch.Tensor, value: torch.Tensor, ids: torch.Tensor, n_out: int,
                scaling: float) -> None:
        """token_attention over the step's own list into ``self.out`` (the
        step's buffers need none of that wrapper's checks)."""
        _require(key.shape == value.shape and key.stride() == value.stride() and key.stride(3) == 1,
                 "key/value layout mismatch")
        lib = _lib.load()
        with _lib.on_device(q.device):
            _lib.check(lib.qkv_token_attention(
                q.data_ptr(), key.data_ptr(), value.data_ptr(), _lib.strides(*key.stride()[:3]), self.batch,
                self.q_heads, key.size(1), key.size(2), self.head_dim, ids.data_ptr(), n_out, float(scaling),
                self.attn_ws.data_ptr(), self.attn_ws.numel() * 4, self.out.data_ptr(), _dtype_code(q),
                _lib.stream_of(q)))

    # -- state views (tests, tracing) ------------------------------------------
    def candidate_mask(self) -> torch.Tensor:
        """The last step's current candidates, bool [B, Hq, history]."""
        if self.bits:
            return expand_bits(self.cand[1 - self.flip], self.last_history).view(self.batch, self.q_heads,
                                                                                  self.last_history)
        return self.cand[1 - self.flip][:, : self.last_history].view(torch.bool).view(
            self.batch, self.q_heads, self.last_history)

    def final_mask(self) -> torch.Tensor:
        """The last step's final selection with the protected ranges, bool [B, Hq, history]."""
        if self.bits:
            return expand_bits(self.fin, self.last_history).view(self.batch, self.q_heads, self.last_history)
        return self.fin[:, : self.last_history].view(torch.bool).view(self.batch, self.q_heads, self.last_history)

    def final_indices(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The last step's final index list and validity, [B, Hq, N]."""
        n = self.n_out
        shape = (self.batch, self.q_heads, n)
        return (self.final_idx[: self.rows * n].view(shape), self.final_valid[: self.rows * n].view(torch.bool).view(shape))


# -- lagged reuse (EV:4020-4198) ----------------------------------------------
LAG_TESTS = {"dims": 0, "overlap": 1, "cos": 2, "ess": 3}                          # QKV_LAG_*
REFRESH = {"none": 0, "all": 1, "per_row": 2, "any": 3, "majority": 4}           # QKV_REFRESH_*
# kind -> (refresh test, which rows refresh once a previous step exists)
LAGGED_KINDS = {
    "lagtop2": (None, "none"),              # the previous final selection alone (EV:4110-4115)
    "lagrefresh": (None, None),             # every row when history % N == 0 (EV:4024)
    "qdrift": ("overlap", "any"),           # EV:4045-4048, 4064-4066
    "qdriftmaj": ("overlap", "majority"),   # EV:4062-4063
    "qdriftcos": ("cos", "any"),            # EV:4049-4057
    "qdrifthead": ("overlap", "per_row"),   # EV:4058-4059, 4089-4106
    "qdriftcoshead": ("cos", "per_row"),
    "qdriftshare": ("overlap", "per_row"),  # + the candidates shared across heads (EV:4107-4109)
    "pconf": ("ess", "per_row"),            # EV:4068-4087
}
_LAGGED = re.compile(r"(lagtop2|lagrefresh(\d+)|qdrift(?:maj|head|share|cos|coshead)?|pconf(\d+(?:p\d+)?))"
                     r"qabs(\d+)cand(\d+(?:p\d+)?)")


def is_lagged_mode(mode: str) -> bool:
    """Whether ``mode`` is one of the lagged reuse modes (EV:475)."""
    return _LAGGED.fullmatch(mode) is not None


def parse_lagged_mode(mode: str) -> tuple[str, float | int | None, int, float]:
    """``lagtop2 | lagrefresh{N} | qdrift[maj|head|share|cos|coshead] | pconf{T}``
    + ``qabs{S}cand{pct}`` -> (kind, parameter, S, candidate fraction): the
    parameter is max(1, N) for lagrefresh (EV:924-928) and T / 100 for pconf
    (``p`` as the decimal point, EV:918-922), else None; S and the fraction as
    ``parse_qabs_partial_rerank_params`` reads them (EV:748-754)."""
    m = _LAGGED.fullmatch(mode)
    _require(m is not None, f"{mode!r} is not a lagged reuse mode (lagtop2 / lagrefresh{{N}} / qdrift* / pconf{{T}} "
                            f"+ qabs{{S}}cand{{pct}})")
    if m.group(2) is not None:
        kind, param = "lagrefresh", max(1, int(m.group(2)))
    elif m.group(3) is not None:
        kind, param = "pconf", float(m.group(3).replace("p", ".")) / 100.0
    else:
        kind, param = m.group(1), None
    return kind, param, int(m.group(4)), float(m.group(5).replace("p", ".")) / 100.0


def lag_flags(query: torch.Tensor, kv_heads: int, test: str, dim_count: int, dims_out: torch.Tensor,
              values_out: torch.Tensor, flags: torch.Tensor | None = None, *, previous_dims: torch.Tensor | None = None,
              previous_values: torch.Tensor | None = None, key: torch.Tensor | None = None, history: int = 0,
              previous_final: torch.Tensor | None = None, scaling: float = 1.0, ess_threshold: float = 0.0,
              workspace: torch.Tensor | None = None) -> None:
    """The lagged modes' per-row refresh test (``qkv_reuse_lag_flags``):
    query [B, Hq, D]; dims_out int32 / values_out f32 [B*Hq, S] receive the
    row's top-|q| dims and q at them; flags uint8 [B*Hq] the test's result
    (``test`` in ``LAG_TESTS``).  The ``ess`` test reads key [B, Hkv, T, D]
    and previous_final rows of the history (uint8 masks, or int64 bitset
    words), and takes a workspace (allocated here when not given)."""
    lib = _lib.load()
    q = query.contiguous()
    b, hq, d = q.shape
    mask_ld = previous_final.stride(0) if previous_final is not None else 0
    bits = previous_final is not None and previous_final.dtype == torch.int64
    if test == "ess" and workspace is None:
        need = int(lib.qkv_reuse_lag_flags_workspace_bytes(b * hq, history))
        _require(need > 0, "bad ESS sizes")
        workspace = torch.empty((need + 3) // 4, dtype=torch.float32, device=q.device)
    with _lib.on_device(q.device):
        _lib.check((lib.qkv_reuse_lag_flags_bits if bits else lib.qkv_reuse_lag_flags)(
            q.data_ptr(), _dtype_code(q), b, hq, kv_heads, d, dim_count, LAG_TESTS[test], _lib.ptr(previous_dims),
            _lib.ptr(previous_values), dims_out.data_ptr(), values_out.data_ptr(), _lib.ptr(key),
            _lib.strides(*key.stride()) if key is not None else None, history, _lib.ptr(previous_final), mask_ld,
            float(scaling), float(ess_threshold), _lib.ptr(flags), _lib.ptr(workspace),
            workspace.numel() * workspace.element_size() if workspace is not None else 0, _lib.stream_of(q)))


def lag_candidates(query: torch.Tensor, key_dim_major: torch.Tensor, history: int, dim_count: int, k: int,
                   flags: torch.Tensor | None, refresh: str, partial: torch.Tensor, mask: torch.Tensor,
                   workspace: torch.Tensor) -> None:
    """Partial scores and candidate mask (``partial >= the row's k-th
    largest``) of the rows that refresh (``qkv_reuse_lag_candidates``);
    query [B, Hq, D], key_dim_major [B, Hkv, D, >= history]; partial f32 /
    mask uint8 rows of >= history.  An int64 ``mask`` is a bitset
    (``qkv_reuse_lag_candidates_bits``), whose workspace is zero-filled."""
    lib = _lib.load()
    q = query.contiguous()
    b, hq, d = q.shape
    bits = mask.dtype == torch.int64
    with _lib.on_device(q.device):
        _lib.check((lib.qkv_reuse_lag_candidates_bits if bits else lib.qkv_reuse_lag_candidates)(
            q.data_ptr(), key_dim_major.data_ptr(), _lib.strides(*key_dim_major.stride()), _dtype_code(q), b, hq,
            key_dim_major.size(1), history, d, dim_count, k, _lib.ptr(flags), REFRESH[refresh], partial.data_ptr(),
            partial.stride(0), mask.data_ptr(), mask.stride(0), workspace.data_ptr(), workspace.numel() * 4,
            _lib.stream_of(q)))


def lag_union(current: torch.Tensor, previous_final: torch.Tensor | None, flags: torch.Tensor | None, batch: int,
              q_heads: int, history: int, refresh: str, share: bool, protect_sink: int, protect_recent: int,
              out: torch.Tensor) -> torch.Tensor:
    """The lagged modes' candidate union (``qkv_reuse_lag_union``) into
    ``out``; ``current`` rows of the rows that do not refresh are cleared.
    Masks uint8 [B*Hq, >= history] (row strides of their own), or int64
    bitset words [B*Hq, >= ceil(history / 64)] (``qkv_reuse_lag_union_bits``)."""
    lib = _lib.load()
    _require(previous_final is None or previous_final.stride(0) == current.stride(0),
             "current and previous_final must share a row stride")
    bits = current.dtype == torch.int64
    _require(out.dtype == current.dtype and (previous_final is None or previous_final.dtype == current.dtype),
             "the masks must all be bytes or all bitsets")
    with _lib.on_device(current.device):
        _lib.check((lib.qkv_reuse_lag_union_bits if bits else lib.qkv_reuse_lag_union)(
            current.data_ptr(), _lib.ptr(previous_final), current.stride(0), _lib.ptr(flags), batch, q_heads, history,
            REFRESH[refresh], int(share), protect_sink, protect_recent, out.data_ptr(), out.stride(0),
            _lib.stream_of(current)))
    return out


class LaggedReuseDecodeStep(ReuseDecodeStep):
    """The lagged reuse modes' decode step (``lagtop2qabs8cand5``,
    ``lagrefresh4qabs8cand5``, ``qdriftheadqabs8cand5``, ``pconf50qabs8cand5``
    ...; ``_qabs_reuse_fast_attention_forward`` EV:4020-4198).  Per step: the
    refresh test on the GPU (``lag_flags``, also recording the top-|q| dims for
    the next step), the partial scores and candidate threshold of every row
    unless no row can refresh, the union with the previous final selection
    (``lag_union``: the rows that do not refresh keep no candidates), then the
    rerank, final selection and attention of the reuse step.  Same call
    convention and state views as ``ReuseDecodeStep``.

    ``candidate_selection`` (``--qabs_candidate_selection``) applies where
    every row thresholds its scores -- a sequence's first step, a
    ``lagrefresh`` step, a step-wide ``qdrift`` / ``qdriftmaj`` / ``qdriftcos``
    refresh -- as in the reference (EV:4116-4145); per-row refreshes threshold
    by ``topk`` (EV:4089-4106), and ``previous_threshold`` reads thresholds only
    from a step that thresholded every row (EV:1686-1694, 1744-1745).  With
    ``topk`` the step-wide any / majority decisions are taken on the GPU, so a
    step needs no host round trip and can be captured; with the other
    selections those two kinds read the decision on the host."""

    def __init__(self, mode: str, batch: int, q_heads: int, kv_heads: int, head_dim: int, capacity: int, *,
                 top_fraction: float = 0.02, protect_sink: int = 0, protect_recent: int = 0,
                 keep_self: bool = True, candidate_selection: str = "topk", threshold_sample_size: int = 256,
                 device: torch.device | str = "cuda", dtype: torch.dtype = torch.bfloat16):
        super().__init__(mode, batch, q_heads, kv_heads, head_dim, capacity, top_fraction=top_fraction,
                         protect_sink=protect_sink, protect_recent=protect_recent, keep_self=keep_self,
                         candidate_selection=candidate_selection, threshold_sample_size=threshold_sample_size,
                         device=device, dtype=dtype)
        s = min(max(1, self.dims), head_dim)
        _require(head_dim <= 128, "the lagged reuse modes take head_dim <= 128")
        # rows that keep skip the partial scores; past 40960 positions the staged
        # top-k still reads their rows, which then hold finite (stale) scores
        self.partial.zero_()
        self.qdims = [torch.zeros((self.rows, s), dtype=torch.int32, device=device) for _ in range(2)]
        self.qvals = [torch.zeros((self.rows, s), dtype=torch.float32, device=device) for _ in range(2)]
        self.flags = torch.zeros(self.rows, dtype=torch.uint8, device=device)
        self.union = torch.zeros_like(self.fin)   # bitset words (or bytes, as the step's masks)
        # the ESS test's per-span sums: at most rows * ceil(1024 / rows) spans
        self.ess_ws = torch.empty(self.rows * -(-1024 // self.rows) * 4 if self.kind == "pconf" else 1,
                                  dtype=torch.float32, device=device)

    def reset(self) -> None:
        super().reset()
        self.thr_valid = False   # the last step thresholded every row (its thresholds are current)

    def _parse_mode(self, mode: str) -> tuple[int, float, bool, bool, int | None]:
        self.kind, self.param, dims, frac = parse_lagged_mode(mode)
        # the lagged modes read the previous final selection only (EV:4147-4152)
        return dims, frac, False, True, None

    def refresh_of(self, history: int, has_previous: bool) -> str:
        """Which rows take new candidates at ``history`` (``REFRESH`` key)."""
        if not has_previous:
            return "all"   # no previous final selection: every row selects (EV:4116)
        if self.kind == "lagrefresh":
            return "all" if history % int(self.param) == 0 else "none"
        return LAGGED_KINDS[self.kind][1]

    def launch(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float,
               current: torch.Tensor, previous: torch.Tensor | None, previous_final: torch.Tensor | None, *,
               previous_thresholds: bool = False) -> None:
        """The lagged step's kernels at the history key.size(2) - 1:
        ``previous_final`` (None on a sequence's first step) is the last
        step's final mask; ``previous`` is not read.  The top-|q| dims go to
        ``self.qdims[self.flip]``, the last step's are read from the other."""
        lib = _lib.load()
        key_count = key.size(2)
        history = key_count - 1
        _require(self.kdm_len >= history, "the dim-major copy does not hold the history")
        q = query.contiguous()
        has_prev = previous_final is not None
        test = LAGGED_KINDS[self.kind][0]
        refresh = self.refresh_of(history, has_prev)
        if test is not None:
            cur_d, prev_d = self.qdims[self.flip], self.qdims[1 - self.flip]
            cur_v, prev_v = self.qvals[self.flip], self.qvals[1 - self.flip]
            run = test if has_prev else "dims"
            lag_flags(q, self.kv_heads, run, self.dims, cur_d, cur_v, self.flags, previous_dims=prev_d,
                      previous_values=prev_v, key=key if run == "ess" else None, history=history,
                      previous_final=previous_final if run == "ess" else None, scaling=scaling,
                      ess_threshold=float(self.param) if self.kind == "pconf" else 0.0,
                      workspace=self.ess_ws if run == "ess" else None)
        if self.selection != "topk" and refresh in ("any", "majority"):
            # the step-wide decision decides whether every row thresholds under
            # the selection (EV:4116-4145) or none takes candidates: read on
            # the host here (one byte per row); with topk it stays on the GPU
            n_flagged = int(self.flags[: self.rows].sum())
            refresh = "all" if (n_flagged > 0 if refresh == "any" else 2 * n_flagged > self.rows) else "none"
        every_row = refresh == "all"
        if every_row and self.selection != "topk":
            # every row thresholds under the selection; previous thresholds only
            # from a step that did the same (EV:1686-1694, 1744-1745)
            self._candidates(q, history, current, previous_thresholds and self.thr_valid)
        elif refresh != "none":   # the rows that refresh score and threshold (EV:3988-3989, 4089-4106)
            requested = budget_count(history, self.cand_fraction)
            if self.bits:   # the candidates' zero-filled workspace (grown zero-filled)
                need = lib.qkv_reuse_candidates_workspace_bytes(self.rows, history, requested)
                if self.cand_ws.numel() * 4 < need:
                    self.cand_ws = torch.zeros((need + 3) // 4, dtype=torch.float32, device=self.device)
                ws = self.cand_ws
            else:
                self.mask_ws = self._grow(self.mask_ws,
                                          lib.qkv_threshold_mask_workspace_bytes(self.rows, history, requested))
                ws = self.mask_ws
            lag_candidates(q, self.kdm, history, self.dims, requested, self.flags, refresh, self.partial, current,
                           ws)
        self.thr_valid = every_row
        lag_union(current, previous_final, self.flags, self.batch, self.q_heads, history, refresh,
                  self.kind == "qdriftshare" and has_prev, self.sink, self.recent, self.union)
        self._select_attend(q, key, value, scaling, self.union, None, None)


# -- candidate attention (qabs{S}cand{pct}attn / appendattn, EV:4400-4502) ----
_QABS_ATTN = re.compile(r"qabs(\d+)cand(\d+(?:p\d+)?)(?:(append)|r(\d+))?attn")


def parse_qabs_attn_mode(mode: str) -> tuple[int, float, bool, int | None]:
    """``qabs{S}cand{pct}[append|r{N}]attn`` -> (S, candidate fraction, append,
    refresh interval or None): ``appendattn`` keeps the selected copies of
    protected tokens (EV:4451, 2985-3022); ``r{N}attn`` reselects only when the
    query token is a multiple of max(1, N) and otherwise reuses the last
    selection (EV:778-782, 4505-4609); the fraction reads ``p`` as the decimal
    point (EV:748-754)."""
    m = _QABS_ATTN.fullmatch(mode)
    _require(m is not None, f"{mode!r} is not a qabs{{S}}cand{{pct}}[append|r{{N}}]attn mode")
    return (int(m.group(1)), float(m.group(2).replace("p", ".")) / 100.0, m.group(3) is not None,
            max(1, int(m.group(4))) if m.group(4) is not None else None)


def final_indices_from_selected(selected: torch.Tensor, n_sel: int, key_count: int, protect_sink: int,
                                protect_recent: int, keep_self: bool, *, out: tuple | None = None):
    """The final index list of a given selection (``qkv_final_indices_from_selected``,
    EV:2938-2982): selected int64 [rows, >= n_sel]; returns (final_indices
    int64, final_valid bool, attn_ids int32), each [rows, n_sel + protected]."""
    lib = _lib.load()
    _require(selected.dtype == torch.int64 and selected.dim() == 2 and selected.stride(1) == 1
             and selected.size(1) >= n_sel, "selected must be int64 [rows, >= n_sel]")
    rows, history = selected.size(0), int(key_count) - 1
    _require(history >= 1, "need key_count >= 2")
    n_out = n_sel + int(lib.qkv_reuse_final_count(history, protect_sink, protect_recent, 0.0, int(keep_self))) - 1
    if out is None:
        dev = selected.device
        out = (torch.empty((rows, n_out), dtype=torch.int64, device=dev),
               torch.empty((rows, n_out), dtype=torch.bool, device=dev),
               torch.empty((rows, n_out), dtype=torch.int32, device=dev))
    fi, fv, ids = out
    with _lib.on_device(selected.device):
        _lib.check(lib.qkv_final_indices_from_selected(
            selected.data_ptr(), selected.stride(0), n_sel, rows, key_count, protect_sink, protect_recent,
            int(keep_self), fi.data_ptr(), fv.data_ptr(), _lib.ptr(ids), n_out, _lib.stream_of(selected)))
    return fi, fv, ids


def qabs_candidate_select(scores: torch.Tensor, key_count: int, candidate_fraction: float, protect_sink: int,
                          protect_recent: int, keep_self: bool, append: bool = False, *,
                          workspace: torch.Tensor | None = None, out: tuple | None = None):
    """The qabs{S}cand{pct}attn candidate selection (``qkv_qabs_candidate_select``)
    on fp32 scores [rows, >= history]: returns (final_indices int64 [rows, N],
    final_valid bool [rows, N], attn_ids int32 [rows, N], history_final bool
    [rows, history]), the selection in ascending order, then the sink range,
    the recent range and the current token (EV:2938-3022)."""
    lib = _lib.load()
    _require(scores.is_cuda and scores.dtype == torch.float32 and scores.dim() == 2 and scores.stride(1) == 1,
             "scores must be CUDA f32 [rows, >= history]")
    rows, history = scores.size(0), int(key_count) - 1
    _require(history >= 1 and scores.size(1) >= history, "need 2 <= key_count <= scores' width + 1")
    n_out = int(lib.qkv_reuse_final_count(history, protect_sink, protect_recent, float(candidate_fraction),
                                          int(keep_self)))
    if out is None:
        dev = scores.device
        out = (torch.empty((rows, n_out), dtype=torch.int64, device=dev),
               torch.empty((rows, n_out), dtype=torch.bool, device=dev),
               torch.empty((rows, n_out), dtype=torch.int32, device=dev),
               torch.empty((rows, history), dtype=torch.bool, device=dev))
    fi, fv, ids, hf = out
    need = int(lib.qkv_qabs_candidate_select_workspace_bytes(rows, history, float(candidate_fraction)))
    _require(need >= 0, "bad candidate selection sizes")
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need + 3) // 4, dtype=torch.float32, device=scores.device)
    with _lib.on_device(scores.device):
        _lib.check(lib.qkv_qabs_candidate_select(
            scores.data_ptr(), rows, key_count, scores.stride(0), float(candidate_fraction), protect_sink,
            protect_recent, int(keep_self), int(append), _lib.ptr(workspace) if need else None,
            workspace.numel() * workspace.element_size() if need else 0, fi.data_ptr(), fv.data_ptr(),
            _lib.ptr(ids), n_out, hf.data_ptr(), hf.stride(0), _lib.stream_of(scores)))
    return fi, fv, ids, hf


class QabsCandidateAttentionStep:
    """One layer's ``qabs{S}cand{pct}attn`` / ``appendattn`` decode step
    (``_qabs_candidate_attention_forward`` EV:4400-4502) with the reference's
    exact arithmetic, for K/V caches of up to ``capacity`` tokens
    ([B, Hkv, T, D], D = 128, bf16 or fp16 as ``dtype`` says): per query head the fp32 partial score of every
    history token on its top-|q| dims (from a per-KV-head dim-major K copy kept
    current one token per step; products and sums in selection order as
    QK:63-96), the ``min(history, max(1, ceil(pct * history)))`` best (ties to
    the lower index), the protected tokens (EV:2938-3022), then attention
    over that list.  Rows are (sequence, query head), each reading its KV head
    directly.  A call whose history is not the previous call's plus one starts
    a new sequence (the dim-major copy is rebuilt)."""

    def __init__(self, mode: str, batch: int, q_heads: int, kv_heads: int, head_dim: int, capacity: int, *,
                 protect_sink: int = 0, protect_recent: int = 0, keep_self: bool = True,
                 device: torch.device | str = "cuda", dtype: torch.dtype = torch.bfloat16):
        lib = _lib.load()
        _require(dtype in (torch.bfloat16, torch.float16), f"dtype must be bfloat16 or float16, got {dtype}")
        self.dtype = dtype
        self.mode = mode
        self.dims, self.cand_fraction, self.append, self.interval = parse_qabs_attn_mode(mode)
        _require(q_heads % kv_heads == 0, "q_heads must be a multiple of kv_heads")
        self.batch, self.q_heads, self.kv_heads, self.head_dim = batch, q_heads, kv_heads, head_dim
        self.capacity = int(capacity)
        self.sink, self.recent, self.keep_self = max(0, int(protect_sink)), max(0, int(protect_recent)), bool(keep_self)
        self.device = device
        rows = batch * q_heads
        self.rows = rows
        cap = self.capacity
        hist_max = cap - 1
        self.n_out_max = int(lib.qkv_reuse_final_count(hist_max, self.sink, self.recent, self.cand_fraction,
                                                       int(self.keep_self)))
        self.kdm = torch.empty((batch, kv_heads, head_dim, cap), dtype=dtype, device=device)
        self.partial = torch.empty((rows, cap), dtype=torch.float32, device=device)
        self.final_idx = torch.empty(rows * self.n_out_max, dtype=torch.int64, device=device)
        self.final_valid = torch.empty(rows * self.n_out_max, dtype=torch.bool, device=device)
        self.attn_ids = torch.empty(rows * self.n_out_max, dtype=torch.int32, device=device)
        self.hf = torch.zeros((rows, cap), dtype=torch.bool, device=device)
        # qkv_qabs_candidates' workspace: zero-filled (its selection state starts
        # at zero and every call leaves it so)
        need = int(lib.qkv_qabs_candidates_workspace_bytes(rows, hist_max, self.cand_fraction))
        _require(need >= 0, "bad candidate selection sizes")
        self.sel_ws = torch.zeros(max(1, (need + 3) // 4), dtype=torch.float32, device=device)
        need = lib.qkv_sparse_attention_workspace_bytes(batch, q_heads, q_heads, head_dim, self.n_out_max, 1)
        _require(need > 0, "unsupported attention shape (head_dim must be 128)")
        self.attn_ws = torch.zeros((need + 3) // 4, dtype=torch.float32, device=device)
        self.out = torch.empty((batch, q_heads, head_dim), dtype=dtype, device=device)
        # r{N}attn: the last refreshing step's selection (EV:1722-1733), its length
        self.kept = torch.empty((rows, self.n_out_max), dtype=torch.int64, device=device) if self.interval else None
        self.n_kept = 0
        self.kdm_len = 0
        self.last_history = None
        self.n_out = 0

    def reset(self) -> None:
        """Forget the dim-major copy and the kept selection (a new sequence)."""
        self.kdm_len = 0
        self.last_history = None
        self.n_kept = 0

    def prefill(self, key: torch.Tensor) -> None:
        """Build the dim-major copy of the cached history in one launch."""
        t = key.size(2)
        if t > self.kdm_len:
            dim_major_append(key, self.kdm, self.kdm_len, t)
            self.kdm_len = t

    def __call__(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float) -> torch.Tensor:
        """query [B, Hq, D]; key/value [B, Hkv, T, D] (the current token
        last), in the step's dtype.  Returns [B, Hq, D] in that dtype."""
        key_count = key.size(2)
        _require(key_count <= self.capacity, f"cache holds {key_count} tokens, capacity {self.capacity}")
        _check_step_dtype(self.dtype, query, key, value)
        if key_count <= 1:   # EV:4415-4417: only the current token
            self.out.copy_(value[:, :, -1, :].repeat_interleave(self.q_heads // self.kv_heads, dim=1))
            return self.out
        history = key_count - 1
        if self.last_history is not None and history != self.last_history + 1:
            self.reset()
        # r{N}attn: between refreshes the previous step's selection is reused (EV:4534-4548)
        reuse = (self.interval is not None and history % self.interval != 0 and self.n_kept > 0
                 and self.last_history == history - 1)
        if self.kdm_len < history and not reuse:
            dim_major_append(key, self.kdm, self.kdm_len, history)
            self.kdm_len = history
        self.launch(query, key, value, scaling, reuse_selection=reuse)
        self.last_history = history
        return self.out

    def launch(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float, *,
               reuse_selection: bool = False) -> None:
        """The step's kernels at the history key.size(2) - 1 (the dim-major
        copy must hold it unless ``reuse_selection``, which rebuilds the final
        list from the kept selection instead, r{N}attn); output in ``self.out``."""
        lib = _lib.load()
        key_count = key.size(2)
        history = key_count - 1
        q = query.contiguous()
        rows = self.rows
        if reuse_selection:
            n_out = self.n_kept + int(lib.qkv_reuse_final_count(history, self.sink, self.recent, 0.0,
                                                                int(self.keep_self))) - 1
            out = (self.final_idx[: rows * n_out].view(rows, n_out),
                   self.final_valid[: rows * n_out].view(rows, n_out), self.attn_ids[: rows * n_out].view(rows, n_out))
            final_indices_from_selected(self.kept, self.n_kept, key_count, self.sink, self.recent, self.keep_self,
                                        out=out)
        else:
            _require(self.kdm_len >= history, "the dim-major copy does not hold the history")
            n_out = int(lib.qkv_reuse_final_count(history, self.sink, self.recent, self.cand_fraction,
                                                  int(self.keep_self)))
            out = (self.final_idx[: rows * n_out].view(rows, n_out),
                   self.final_valid[: rows * n_out].view(rows, n_out), self.attn_ids[: rows * n_out].view(rows, n_out),
                   self.hf)
            # partial scores and the selection in one call (across workgroups
            # where the rows are few and short enough)
            with _lib.on_device(q.device):
                _lib.check(lib.qkv_qabs_candidates(
                    q.data_ptr(), self.kdm.data_ptr(), _lib.strides(*self.kdm.stride()), _dtype_code(q), self.batch,
                    self.q_heads, self.kv_heads, key_count, self.head_dim, self.dims, self.cand_fraction, self.sink,
                    self.recent, int(self.keep_self), int(self.append), self.partial.data_ptr(),
                    self.partial.stride(0), self.sel_ws.data_ptr(), self.sel_ws.numel() * 4, out[0].data_ptr(),
                    out[1].data_ptr(), out[2].data_ptr(), n_out, self.hf.data_ptr(), self.hf.stride(0),
                    _lib.stream_of(q)))
            if self.interval is not None:   # the selection the next steps reuse (EV:4574-4580)
                keep = budget_count(history, self.cand_fraction)
                self.kept[:, :keep].copy_(out[0][:, :keep])
                self.n_kept = keep
        token_attention(q, key, value, out[2], scaling, workspace=self.attn_ws, out=self.out)
        self.n_out = n_out

    def final_indices(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The last step's final index list and validity, [B, Hq, N]."""
        n = self.n_out
        shape = (self.batch, self.q_heads, n)
        return self.final_idx[: self.rows * n].view(shape), self.final_valid[: self.rows * n].view(shape)

    def final_mask(self) -> torch.Tensor:
        """The last selecting step's selection plus the protected ranges, bool
        [B, Hq, history] (r{N}attn steps that reuse a selection leave it as it
        was; their list is ``final_indices()``)."""
        h = self.last_history
        return self.hf[:, :h].reshape(self.batch, self.q_heads, h)
