"""Chunked-prefill block selection on int8 MFMA (MI355X).

A query chunk (positions q_pos0 .. q_pos0 + Nq - 1) is scored against every
cached key of its KV head: the query rows are quantized to int8 per row,
K is int4 packed with one fp16 scale per token (``int4_pack_k`` with
group 128), I = q8 . code over all 128 channels in int32 on MFMA, the
ranking key is fp32(scale) * fp32(I), keys are max-pooled per 64-key block
under the causal mask, and the top-k blocks are kept per query row.

No reference counterpart: the reference prefills with dense attention
(evaluate_qwen3_top2_head_limit3_ppl.py:7079-7111).  Everything runs on the
GPU on the current stream and raises RuntimeError on bad input.
"""

from __future__ import annotations

import torch

from . import _lib

BLOCK = 64


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def quantize_query(query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """query bf16 or fp16 [..., 128] -> (q8 int8 [..., 128] in the MFMA operand
    order, qscale f32 [...])."""
    lib = _lib.load()
    _require(query.is_cuda and query.size(-1) == 128, "query must be CUDA [..., 128]")
    code = _lib.half_code("query", query)
    q = query.reshape(-1, 128)
    _require(q.stride(1) == 1, "query channels must be contiguous")
    rows = q.size(0)
    q8 = torch.empty((*query.shape[:-1], 128), dtype=torch.int8, device=query.device)
    qscale = torch.empty(query.shape[:-1], dtype=torch.float32, device=query.device)
    with _lib.on_device(query.device):
        _lib.check(lib.qkv_prefill_quantize_query(q.data_ptr(), rows, 128, q.stride(0), q8.data_ptr(),
                                                  qscale.data_ptr(), code, _lib.stream_of(query)))
    return q8, qscale


def block_scores(q8: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, tokens: int, q_pos0: int,
                 *, bmax: torch.Tensor | None = None) -> torch.Tensor:
    """q8 int8 [B,Hq,Nq,128]; packed uint8 [B,Hkv,cap,64]; scales fp16
    [B,Hkv,cap] or [B,Hkv,cap,1].  Returns bmax f32 [B,Hq,Nq,ceil(tokens/64)]."""
    lib = _lib.load()
    _require(q8.is_cuda and q8.dtype == torch.int8 and q8.dim() == 4 and q8.is_contiguous(),
             "q8 must be contiguous CUDA int8 [B,Hq,Nq,128]")
    _require(packed.dtype == torch.uint8 and packed.dim() == 4 and packed.is_contiguous(),
             "packed K must be contiguous uint8 [B,Hkv,cap,64]")
    b, hq, nq, d = q8.shape
    _, hkv, cap, half = packed.shape
    _require(half * 2 == d == 128, "packed K must hold 128 channels")
    sc = scales.reshape(b, hkv, cap)
    _require(sc.dtype == torch.float16 and sc.is_contiguous(), "scales must be contiguous fp16, one per token")
    nb = -(-int(tokens) // BLOCK)
    if bmax is None:
        bmax = torch.empty((b, hq, nq, nb), dtype=torch.float32, device=q8.device)
    with _lib.on_device(q8.device):
        _lib.check(lib.qkv_prefill_block_scores(q8.data_ptr(), b, hq, hkv, nq, packed.data_ptr(), sc.data_ptr(),
                                                cap, int(tokens), int(q_pos0), d, BLOCK, bmax.data_ptr(),
                                                _lib.stream_of(q8)))
    return bmax


def block_topk(bmax: torch.Tensor, k: int, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Top-k finite blocks per row (lowest index wins ties), ascending, padded
    with -1 when a row has fewer than k visible blocks; int32 [..., k]."""
    lib = _lib.load()
    _require(bmax.is_cuda and bmax.dtype == torch.float32, "bmax must be CUDA float32")
    n = bmax.size(-1)
    v2 = bmax.reshape(-1, n)
    _require(v2.stride(1) == 1, "bmax must be contiguous along the last axis")
    if out is None:
        out = torch.empty((*bmax.shape[:-1], int(k)), dtype=torch.int32, device=bmax.device)
    with _lib.on_device(bmax.device):
        _lib.check(lib.qkv_prefill_block_topk(v2.data_ptr(), v2.size(0), n, v2.stride(0), int(k), out.data_ptr(),
                                              _lib.stream_of(bmax)))
    return out


def select_blocks(query: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, tokens: int, q_pos0: int,
                  k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """query bf16 or fp16 [B,Hq,Nq,128] -> (top-k block ids int32 [B,Hq,Nq,k], bmax)."""
    q8, _ = quantize_query(query)
    bmax = block_scores(q8, packed, scales, tokens, q_pos0)
    return block_topk(bmax, k), bmax
