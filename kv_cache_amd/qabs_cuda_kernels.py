"""Drop-in for the reference's ``qabs_cuda_kernels`` module on MI355X.

Same four functions, argument meaning, output shapes and error behaviour as
ymluo/projects/qwen3_top2_head_limit3_ppl/src/qabs_cuda_kernels.py:654-705,
backed by libqkv's gfx950 kernels instead of a JIT-built CUDA extension,
plus the two the reference's harness imports from that module but which it
never shipped: ``reuse_select`` (EV:3881-3919) and ``brep_partial_scores``
(EV:3847-3877).
Shape/dtype violations raise ``RuntimeError`` with the reference's
``TORCH_CHECK`` messages; inputs are made contiguous exactly where the
reference does so; outputs are allocated here (fp32 scores, query-dtype
attention) and the kernels run on the current stream.
"""

from __future__ import annotations

import torch

from . import _lib


def _load_extension():
    """The reference's loader name (QK:642-651); returns the C-ABI library."""
    return _lib.load()


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _dtype_code(t: torch.Tensor) -> int:
    code = _lib.DTYPE_CODES.get(t.dtype)
    if code is None:
        raise RuntimeError(f"unsupported dtype {t.dtype}")
    return code


def partial_scores(query: torch.Tensor, key_history: torch.Tensor, dim_count: int) -> torch.Tensor:
    """QK:654-656 (host QK:421-459): fp32 [B,H,T] partial QK over the
    ``dim_count`` largest-|q| dims of each query row, token-major K."""
    lib = _lib.load()
    _check(query.is_cuda, "query must be CUDA")
    _check(key_history.is_cuda, "key must be CUDA")
    _check(query.dim() == 3, "query must have shape [batch, heads, dim]")
    _check(key_history.dim() == 4, "key must have shape [batch, heads, key, dim]")
    _check(query.dtype == key_history.dtype, "query/key dtype mismatch")
    _check(query.size(0) == key_history.size(0) and query.size(1) == key_history.size(1)
           and query.size(2) == key_history.size(3), "query/key shape mismatch")
    q = query.contiguous()
    b, h, d = q.shape
    t = key_history.size(2)
    out = torch.empty((b, h, t), dtype=torch.float32, device=q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_partial_scores(
            q.data_ptr(), key_history.data_ptr(), out.data_ptr(), _dtype_code(q), b, h, t, d,
            _lib.strides(*key_history.stride()), int(dim_count), _lib.stream_of(q)))
    return out


def partial_scores_dim_major(query: torch.Tensor, key_dim_major: torch.Tensor,
                             dim_indices: torch.Tensor) -> torch.Tensor:
    """QK:659-665 (host QK:461-504): fp32 [B,H,T] over dim-major K [B,H,D,T]
    and int64 dim indices [B,H,S], accumulated in the given index order."""
    lib = _lib.load()
    _check(query.is_cuda, "query must be CUDA")
    _check(key_dim_major.is_cuda, "key_dim_major must be CUDA")
    _check(dim_indices.is_cuda, "dim_indices must be CUDA")
    _check(query.dim() == 3, "query must have shape [batch, heads, dim]")
    _check(key_dim_major.dim() == 4, "key_dim_major must have shape [batch, heads, dim, key]")
    _check(dim_indices.dim() == 3, "dim_indices must have shape [batch, heads, selected_dim]")
    _check(query.dtype == key_dim_major.dtype, "query/key dtype mismatch")
    _check(dim_indices.dtype == torch.int64, "dim_indices must be int64")
    _check(query.size(0) == key_dim_major.size(0) and query.size(1) == key_dim_major.size(1)
           and query.size(2) == key_dim_major.size(2), "query/key shape mismatch")
    _check(dim_indices.size(0) == query.size(0) and dim_indices.size(1) == query.size(1),
           "dim_indices shape mismatch")
    q = query.contiguous()
    idx = dim_indices.contiguous()
    b, h, d = q.shape
    t = key_dim_major.size(3)
    out = torch.empty((b, h, t), dtype=torch.float32, device=q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_partial_scores_dim_major(
            q.data_ptr(), key_dim_major.data_ptr(), idx.data_ptr(), out.data_ptr(), _dtype_code(q),
            b, h, t, d, idx.size(2), _lib.strides(*key_dim_major.stride()), _lib.stream_of(q)))
    return out


def candidate_full_scores(query: torch.Tensor, key_history: torch.Tensor,
                          current_candidate: torch.Tensor, previous_candidate: torch.Tensor | None,
                          previous_final: torch.Tensor | None, protect_sink_tokens: int,
                          protect_recent_tokens: int, scaling: float) -> torch.Tensor:
    """QK:668-691 (host QK:506-567): full-D scores * scaling on candidate,
    previous, sink and recent tokens, -inf elsewhere; fp32 [B,H,T]."""
    lib = _lib.load()
    _check(query.is_cuda, "query must be CUDA")
    _check(key_history.is_cuda, "key must be CUDA")
    _check(current_candidate.is_cuda, "current_candidate must be CUDA")
    _check(query.dim() == 3, "query must have shape [batch, heads, dim]")
    _check(key_history.dim() == 4, "key must have shape [batch, heads, key, dim]")
    _check(current_candidate.dim() == 3, "current_candidate must have shape [batch, heads, key]")
    _check(query.dtype == key_history.dtype, "query/key dtype mismatch")
    _check(current_candidate.dtype == torch.bool, "current_candidate must be bool")
    _check(previous_candidate is None or previous_candidate.dtype == torch.bool,
           "previous_candidate must be bool")
    _check(previous_final is None or previous_final.dtype == torch.bool, "previous_final must be bool")
    _check(query.size(0) == key_history.size(0) and query.size(1) == key_history.size(1)
           and query.size(2) == key_history.size(3), "query/key shape mismatch")
    _check(current_candidate.size(0) == key_history.size(0)
           and current_candidate.size(1) == key_history.size(1)
           and current_candidate.size(2) == key_history.size(2), "candidate shape mismatch")
    q = query.contiguous()
    cur = current_candidate.contiguous()
    prev = previous_candidate.contiguous() if previous_candidate is not None else None
    fin = previous_final.contiguous() if previous_final is not None else None
    for name, m in (("previous_candidate", prev), ("previous_final", fin)):
        _check(m is None or m.shape == cur.shape, f"{name} shape mismatch")
    b, h, d = q.shape
    t = key_history.size(2)
    out = torch.empty((b, h, t), dtype=torch.float32, device=q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_candidate_full_scores(
            q.data_ptr(), key_history.data_ptr(), cur.data_ptr(), _lib.ptr(prev), _lib.ptr(fin),
            out.data_ptr(), _dtype_code(q), b, h, t, d, _lib.strides(*key_history.stride()),
            int(protect_sink_tokens), int(protect_recent_tokens), float(scaling), _lib.stream_of(q)))
    return out


_WORKSPACES: dict = {}


def _token_attention_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A zeroed workspace for qkv_token_attention, one per (device, current
    stream), grown on demand: its row tickets start at zero and every
    completed launch leaves them zero, so launches in one stream's order
    share it (launches on other streams get their own)."""
    stream = torch.cuda.current_stream(device)
    key = (device, stream.cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        ws = torch.zeros((nbytes + 3) // 4, dtype=torch.float32, device=device)
        _WORKSPACES[key] = ws
    return ws


def final_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    indices: torch.Tensor, valid: torch.Tensor, scaling: float) -> torch.Tensor:
    """QK:694-705 (host QK:569-638): softmax attention over the valid
    ``indices`` of each (b, h); returns [B, 1, H, D] in the query dtype.
    bf16 and fp16 inputs at D = 128 run on the matrix-core list attention
    (``qkv_token_attention``, 226 -> ~9 us at 32 heads x ~1000 entries over
    32768 keys); fp32 (or another D) on ``qkv_final_attention``'s fp32 loop in
    the reference's order."""
    lib = _lib.load()
    valid_u8 = valid   # bool (or uint8) [B,H,N]; the fp32-loop kernel reads it as bytes (QK:703)
    _check(query.is_cuda, "query must be CUDA")
    _check(key.is_cuda, "key must be CUDA")
    _check(value.is_cuda, "value must be CUDA")
    _check(indices.is_cuda, "indices must be CUDA")
    _check(valid_u8.is_cuda, "valid must be CUDA")
    _check(query.device == key.device, "query/key device mismatch")
    _check(query.device == value.device, "query/value device mismatch")
    _check(query.device == indices.device, "query/indices device mismatch")
    _check(query.device == valid_u8.device, "query/valid device mismatch")
    _check(query.dim() == 3, "query must have shape [batch, heads, dim]")
    _check(key.dim() == 4, "key must have shape [batch, heads, key, dim]")
    _check(value.shape == key.shape, "value must match key shape")
    _check(indices.dim() == 3, "indices must have shape [batch, heads, selected]")
    _check(valid_u8.shape == indices.shape, "valid must match indices shape")
    _check(query.dtype == key.dtype, "query/key dtype mismatch")
    _check(query.dtype == value.dtype, "query/value dtype mismatch")
    _check(indices.dtype == torch.int64, "indices must be int64")
    q = query.contiguous()
    k = key.contiguous()
    v = value.contiguous()
    idx = indices.contiguous()
    val = valid_u8.contiguous()
    b, h, d = q.shape
    t = k.size(2)
    n = idx.size(2)
    _check(k.size(0) == b and k.size(1) == h and k.size(3) == d, "key shape mismatch")
    _check(idx.size(0) == b and idx.size(1) == h, "indices shape mismatch")
    _check(n > 0, "select_count must be positive")
    half = q.dtype in (torch.bfloat16, torch.float16)
    ws_bytes = int(lib.qkv_sparse_attention_workspace_bytes(b, h, h, d, n, 1)) if half else 0
    if ws_bytes > 0:
        # bf16 / fp16: the list-per-head attention on the matrix cores (qkv_token_attention,
        # G = 1 on these head-expanded K/V), the invalid and out-of-range entries
        # as skipped ids; a row with none valid gives 0, as QK:388, 404 do
        with _lib.on_device(q.device):
            # ids outside [0, t) are skipped (int64 values clamped first so none wraps)
            keep = val if val.dtype == torch.bool else val != 0
            ids = torch.where(keep, idx.clamp(-1, t), -1).to(torch.int32).view(b * h, n)
            ws = _token_attention_workspace(q.device, ws_bytes)
            out = torch.empty((b, h, d), dtype=q.dtype, device=q.device)
            _lib.check(lib.qkv_token_attention(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.strides(*k.stride()[:3]), b, h, h, t, d,
                ids.data_ptr(), n, float(scaling), ws.data_ptr(), ws_bytes, out.data_ptr(), _dtype_code(q),
                _lib.stream_of(q)))
        return out[:, None, :, :]
    out = torch.empty((b, h, d), dtype=q.dtype, device=q.device)
    val = val.to(torch.uint8)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_final_attention(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), idx.data_ptr(), val.data_ptr(), out.data_ptr(),
            _dtype_code(q), b, h, t, n, d, float(scaling), _lib.stream_of(q)))
    return out[:, None, :, :].contiguous()


def brep_partial_scores(query: torch.Tensor, key_history: torch.Tensor, rep_indices: torch.Tensor,
                        rep_valid: torch.Tensor, block_size: int, dim_count: int, scan_fraction: float) -> torch.Tensor:
    """The block-representative scan the reference imports from this module
    but never shipped (wrapper EV:3847-3877, called at EV:5419-5431 with the
    fp32 query, the history keys and BlockRepState's representatives).

    query [B,H,D] (any float dtype; scored as fp32); key_history [B,H,T,D];
    rep_indices int64 / rep_valid bool [B,H,ceil(T/block_size),R].  Returns
    fp32 [B,H,T]: the partial score on the ``dim_count`` largest-|q| dims of
    every token of the ``min(blocks, max(1, ceil(scan_fraction*T/block_size)))``
    blocks whose best valid representative scores highest, -inf elsewhere --
    so the caller's ``topk`` + ``isfinite`` (EV:5426-5428) picks candidates
    from the scanned blocks only, as its fallback does (EV:5442-5470)."""
    lib = _lib.load()
    _check(query.is_cuda, "query must be CUDA")
    _check(key_history.is_cuda, "key must be CUDA")
    _check(rep_indices.is_cuda and rep_valid.is_cuda, "representatives must be CUDA")
    _check(query.dim() == 3, "query must have shape [batch, heads, dim]")
    _check(key_history.dim() == 4, "key must have shape [batch, heads, key, dim]")
    _check(query.is_floating_point(), "query must be floating point")
    _check(query.size(0) == key_history.size(0) and query.size(1) == key_history.size(1)
           and query.size(2) == key_history.size(3), "query/key shape mismatch")
    _check(int(block_size) > 0, "block_size must be positive")
    b, h, d = query.shape
    t = key_history.size(2)
    nb = -(-t // int(block_size))
    _check(rep_indices.dim() == 4 and tuple(rep_indices.shape[:3]) == (b, h, nb),
           "rep_indices must have shape [batch, heads, blocks, reps]")
    _check(rep_indices.dtype == torch.int64, "rep_indices must be int64")
    _check(rep_valid.dtype == torch.bool and rep_valid.shape == rep_indices.shape,
           "rep_valid must be bool with the shape of rep_indices")
    out = torch.empty((b, h, t), dtype=torch.float32, device=query.device)
    if t == 0:
        return out
    q = query.float().contiguous()
    k = key_history.contiguous()
    idx = rep_indices.contiguous()
    val = rep_valid.contiguous().view(torch.uint8)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_brep_partial_scores(
            q.data_ptr(), k.data_ptr(), idx.data_ptr(), val.data_ptr(), out.data_ptr(), _dtype_code(k), b, h, t, d,
            _lib.strides(*k.stride()), idx.size(3), int(block_size), int(dim_count), float(scan_fraction),
            _lib.stream_of(q)))
    return out


def reuse_select(query: torch.Tensor, key_states: torch.Tensor, current_candidate: torch.Tensor,
                 previous_candidate: torch.Tensor | None, previous_final: torch.Tensor | None,
                 protect_sink_tokens: int, protect_recent_tokens: int, top_fraction: float,
                 always_keep_self: bool, scaling: float):
    """The fused selector the reference imports from this module but never
    shipped (called at EV:3901-3914, signature EV:3881-3892): rerank the
    union of the candidate masks by full-D scores, keep the
    ``ceil(top_fraction * history)`` best, and build the final index list.

    query [B,H,D]; key_states [B,H,K,D] including the current token
    (history = K - 1); masks bool [B,H,history].  Returns (final_indices
    int64 [B,H,N], final_valid bool [B,H,N], history_final bool
    [B,H,history]) with the meaning of the fallback path EV:4257-4365.  The
    selection comes in ascending index order (the fallback's comes in
    descending score order; the attention over it is the same set)."""
    lib = _lib.load()
    _check(query.is_cuda and key_states.is_cuda and current_candidate.is_cuda, "inputs must be CUDA")
    _check(query.dim() == 3, "query must have shape [batch, heads, dim]")
    _check(key_states.dim() == 4, "key must have shape [batch, heads, key, dim]")
    _check(query.dtype == key_states.dtype, "query/key dtype mismatch")
    _check(current_candidate.dtype == torch.bool, "current_candidate must be bool")
    b, h, d = query.shape
    key_count = key_states.size(2)
    history = key_count - 1
    _check(key_states.size(0) == b and key_states.size(1) == h and key_states.size(3) == d, "query/key shape mismatch")
    _check(history >= 1, "reuse_select needs at least one history token")
    _check(tuple(current_candidate.shape) == (b, h, history), "candidate shape mismatch")
    masks = []
    for name, m in (("previous_candidate", previous_candidate), ("previous_final", previous_final)):
        _check(m is None or (m.dtype == torch.bool and tuple(m.shape) == (b, h, history)), f"{name} shape mismatch")
        masks.append(m.contiguous() if m is not None else None)
    q = query.contiguous()
    k = key_states if key_states.stride(3) == 1 else key_states.contiguous()
    cur = current_candidate.contiguous()
    sink, recent = max(0, int(protect_sink_tokens)), max(0, int(protect_recent_tokens))
    n_out = lib.qkv_reuse_final_count(history, sink, recent, float(top_fraction), int(bool(always_keep_self)))
    ws_bytes = lib.qkv_reuse_select_workspace_bytes(b * h, history, float(top_fraction))
    _check(n_out > 0 and ws_bytes > 0, "bad reuse_select sizes")
    ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=q.device)
    final_indices = torch.empty((b, h, n_out), dtype=torch.int64, device=q.device)
    final_valid = torch.empty((b, h, n_out), dtype=torch.bool, device=q.device)
    history_final = torch.empty((b, h, history), dtype=torch.bool, device=q.device)
    with _lib.on_device(q.device):
        _lib.check(lib.qkv_reuse_select(
            q.data_ptr(), k.data_ptr(), _lib.strides(*k.stride()), _dtype_code(q), b, h, h, key_count, d,
            cur.data_ptr(), _lib.ptr(masks[0]), _lib.ptr(masks[1]), history, sink, recent, float(top_fraction),
            int(bool(always_keep_self)), float(scaling), ws.data_ptr(), ws.numel() * 4, final_indices.data_ptr(),
            final_valid.data_ptr(), None, n_out, history_final.data_ptr(), history, _lib.stream_of(q)))
    return final_indices, final_valid, history_final
