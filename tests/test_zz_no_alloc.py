"""The allocation-free entry point (qkv_sparse_attention_select_noalloc),
called through the C ABI, against qkv_sparse_attention_select with a
caller-owned workspace: the same kernel on the same inputs, so the selected
block ids and the bf16 outputs are equal bit for bit.  Two calls in a row on
the same GPU (the second one smaller) check that the shared static scratch
carries nothing from one call into the next."""

import ctypes

import pytest
import torch

from kv_cache_amd import _lib
from kv_cache_amd import int4 as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH_BYTES = 8 << 20   # QKV_NOALLOC_SCRATCH_BYTES


def _inputs(batch, q_heads, kv_heads, tokens, block, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn((batch, q_heads, 128), generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn((batch, kv_heads, tokens, 128), generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn((batch, kv_heads, tokens, 128), generator=g, device=DEV).to(torch.bfloat16)
    nb = -(-tokens // block)
    # block maxima with many exact ties (values on a coarse grid)
    bmax = (torch.randn((batch, kv_heads, nb), generator=g, device=DEV) * 4).round() / 4
    return q, k, v, bmax.contiguous()


def _call(noalloc, q, k, v, bmax, n_sel, block, tokens, scaling):
    lib = _lib.load()
    b, hq, d = q.shape
    hkv = k.size(1)
    sel = torch.full((b, hkv, n_sel), -7, dtype=torch.int32, device=DEV)
    out = torch.zeros((b, hq, d), dtype=torch.bfloat16, device=DEV)
    stream = _lib.stream_of(q)
    ks = _lib.strides(*k.stride()[:3])
    with torch.cuda.device(q.device):
        if noalloc:
            rc = lib.qkv_sparse_attention_select_noalloc(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), ks, b, hq, hkv, tokens, d, bmax.data_ptr(), bmax.size(2),
                n_sel, block, ctypes.c_float(scaling), sel.data_ptr(), out.data_ptr(), 0, stream)
        else:
            ws = K.attention_workspace(b, hq, hkv, d, n_sel, block, q.device)
            rc = lib.qkv_sparse_attention_select(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), ks, b, hq, hkv, tokens, d, bmax.data_ptr(), bmax.size(2),
                n_sel, block, ctypes.c_float(scaling), ws.data_ptr(), ws.numel() * 4, sel.data_ptr(), out.data_ptr(),
                0, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return sel, out


# (batch, q_heads, kv_heads, tokens, block, n_sel): a cfg2-sized call, then a
# smaller G = 4 call with a partial last block.
CALLS = [(8, 16, 8, 32768, 16, 128), (2, 32, 8, 4000, 16, 64)]


def test_noalloc_matches_workspace_entry_two_calls():
    for i, (b, hq, hkv, t, blk, n_sel) in enumerate(CALLS):
        print(f"noalloc call {i}: B={b} Hq={hq} Hkv={hkv} T={t} block={blk} n_sel={n_sel}", flush=True)
        assert _lib.load().qkv_sparse_attention_workspace_bytes(b, hq, hkv, 128, n_sel, blk) <= SCRATCH_BYTES
        q, k, v, bmax = _inputs(b, hq, hkv, t, blk, seed=100 + i)
        scaling = 128 ** -0.5
        want_sel, want_out = _call(False, q, k, v, bmax, n_sel, blk, t, scaling)
        got_sel, got_out = _call(True, q, k, v, bmax, n_sel, blk, t, scaling)
        assert torch.equal(got_sel, want_sel), f"call {i}: selections differ"
        assert torch.equal(got_out.view(torch.int16), want_out.view(torch.int16)), f"call {i}: outputs differ"
        # and the selection is the top-k of the block maxima (lowest index wins ties)
        assert torch.equal(got_sel, K.block_topk(bmax, n_sel))


def test_noalloc_rejects_sizes_beyond_scratch():
    lib = _lib.load()
    b, hq, hkv, t, blk, n_sel = 64, 64, 64, 65536, 16, 4096
    assert lib.qkv_sparse_attention_workspace_bytes(b, hq, hkv, 128, n_sel, blk) > SCRATCH_BYTES
    p = ctypes.c_void_p(256)
    rc = lib.qkv_sparse_attention_select_noalloc(p, p, p, _lib.strides(1024, 1024, 128), b, hq, hkv, t, 128, p,
                                                 t // blk, n_sel, blk, ctypes.c_float(0.1), None, p, 0, None)
    assert rc == -3
    assert "static scratch holds" in lib.qkv_last_error().decode()
