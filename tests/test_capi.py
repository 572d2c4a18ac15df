"""The C-ABI library loads on a CPU-only host, exports every entry point the
header declares, and rejects bad arguments on the host side before any GPU
call (no kernel is launched here)."""

import ctypes

import pytest

from kv_cache_amd import _lib

lib = _lib.load()


def test_abi_version():
    assert lib.qkv_abi_version() == _lib.ABI_VERSION


def test_every_header_symbol_is_exported_and_bound():
    names = _lib.header_functions()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib._PROTOTYPES, f"{name} has no ctypes prototype"
    assert set(_lib._PROTOTYPES) == set(names)


def _err():
    return lib.qkv_last_error().decode()


@pytest.mark.parametrize("call,msg", [
    (lambda: lib.qkv_topk(None, 1, 10, 10, 3, None, None), "null pointer"),
    (lambda: lib.qkv_topk(ctypes.c_void_p(16), 1, 10, 10, 11, ctypes.c_void_p(16), None), "1 <= k <= n"),
    (lambda: lib.qkv_topk(ctypes.c_void_p(16), 1, 10, 5, 3, ctypes.c_void_p(16), None), "bad sizes"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 24,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4096, 4096, 16,
                                        ctypes.c_void_p(16), None, None, None, 0, None), "selected must be"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 32,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4032, 4000, 16,
                                        ctypes.c_void_p(16), None, None, None, 0, None), "multiple of 256"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 32,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4096, 4096, 12,
                                        ctypes.c_void_p(16), None, None, None, 0, None), "power of two"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 64,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4096, 4096, 256,
                                        ctypes.c_void_p(16), None, None, None, 0, None), "<= 128"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 32,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4096, 4096, 16,
                                        None, None, None, None, 0, None), "need bmax"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 15, 8, 128, ctypes.c_void_p(16), 32,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4096, 4096, 16,
                                        ctypes.c_void_p(16), None, None, None, 0, None), "multiple of kv_heads"),
    (lambda: lib.qkv_int4_query_words(ctypes.c_void_p(16), 1, 15, 8, 128, ctypes.c_void_p(16), 32,
                                      ctypes.c_void_p(16), None, 0, None), "multiple of kv_heads"),
    (lambda: lib.qkv_int4_query_words(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 48,
                                      ctypes.c_void_p(16), None, 0, None), "selected must be"),
    (lambda: lib.qkv_int4_pack_k(ctypes.c_void_p(16), _lib.strides(8, 8, 8), 1, 1, 0, 10, 128, 48,
                                 ctypes.c_void_p(16), ctypes.c_void_p(16), 64, 0, None), "group"),
    (lambda: lib.qkv_int4_pack_k(ctypes.c_void_p(16), _lib.strides(8, 8, 8), 1, 1, 0, 100, 128, 32,
                                 ctypes.c_void_p(16), ctypes.c_void_p(16), 64, 0, None), "token range"),
    (lambda: lib.qkv_int4_pack_k(ctypes.c_void_p(18), _lib.strides(8, 8, 8), 1, 1, 0, 10, 128, 32,
                                 ctypes.c_void_p(16), ctypes.c_void_p(16), 64, 0, None), "16-byte aligned"),
    (lambda: lib.qkv_sparse_attention(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                      _lib.strides(8, 8, 8), 1, 16, 8, 100, 64, ctypes.c_void_p(16), 4, 16,
                                      1.0, ctypes.c_void_p(16), 1 << 20, ctypes.c_void_p(16), 0, None), "128"),
    (lambda: lib.qkv_sparse_attention(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                      _lib.strides(8, 8, 8), 1, 16, 8, 100, 128, ctypes.c_void_p(16), 4, 16,
                                      1.0, ctypes.c_void_p(16), 16, ctypes.c_void_p(16), 0, None), "workspace"),
    (lambda: lib.qkv_final_attention(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                     ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 0,
                                     1, 1, 10, 0, 128, 1.0, None), "select_count must be positive"),
    (lambda: lib.qkv_partial_scores(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 7,
                                    1, 1, 10, 128, _lib.strides(1, 1, 1, 1), 8, None), "dtype"),
    (lambda: lib.qkv_reuse_expand_blocks(None, 10, 1, 11, 4, 0, 0, 0.1, 1, ctypes.c_void_p(16),
                                         ctypes.c_void_p(16), None, 5, None), "null pointer"),
    (lambda: lib.qkv_reuse_expand_blocks(ctypes.c_void_p(16), 10, 1, 11, 5000, 0, 0, 0.1, 1, ctypes.c_void_p(16),
                                         ctypes.c_void_p(16), None, 5, None), "block must be"),
    (lambda: lib.qkv_reuse_expand_blocks(ctypes.c_void_p(16), 10, 1, 11, 4, 0, 0, 0.1, 1, ctypes.c_void_p(16),
                                         ctypes.c_void_p(16), None, 5, None), "expanded selection needs"),
    (lambda: lib.qkv_reuse_expand_blocks(ctypes.c_void_p(16), 8, 1, 11, 4, 0, 0, 0.1, 1, ctypes.c_void_p(16),
                                         ctypes.c_void_p(16), None, 5, None), "stride"),
    (lambda: lib.qkv_sparse_attention_select_noalloc(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                                     _lib.strides(8, 8, 8), 1, 16, 8, 100, 128, None, 7, 4, 16,
                                                     1.0, None, ctypes.c_void_p(16), 0, None), "null pointer"),
    (lambda: lib.qkv_sparse_attention_select_noalloc(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                                     _lib.strides(8, 8, 8), 1, 16, 8, 100, 64, ctypes.c_void_p(16), 7,
                                                     4, 16, 1.0, None, ctypes.c_void_p(16), 0, None), "unsupported sizes"),
    # 4096 rows x 65536 selected slots: far beyond the 8 MiB static scratch
    (lambda: lib.qkv_sparse_attention_select_noalloc(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                                     _lib.strides(8, 8, 8), 64, 64, 64, 65536, 128,
                                                     ctypes.c_void_p(16), 4096, 4096, 16, 1.0, None,
                                                     ctypes.c_void_p(16), 0, None), "static scratch holds"),
    # the 16-bit entry points take bf16 (0) or fp16 (1); fp32 is unsupported, other codes invalid
    (lambda: lib.qkv_int4_pack_k(ctypes.c_void_p(16), _lib.strides(8, 8, 8), 1, 1, 0, 10, 128, 32,
                                 ctypes.c_void_p(16), ctypes.c_void_p(16), 64, 2, None), "is not bf16"),
    (lambda: lib.qkv_int4_decode_scores(ctypes.c_void_p(16), 1, 16, 8, 128, ctypes.c_void_p(16), 32,
                                        ctypes.c_void_p(16), ctypes.c_void_p(16), 4096, 4096, 16,
                                        ctypes.c_void_p(16), None, None, None, 5, None), "is not bf16"),
    (lambda: lib.qkv_sparse_attention(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                      _lib.strides(8, 8, 8), 1, 16, 8, 100, 128, ctypes.c_void_p(16), 4, 16,
                                      1.0, ctypes.c_void_p(16), 1 << 20, ctypes.c_void_p(16), 2, None), "is not bf16"),
    (lambda: lib.qkv_prefill_quantize_query(ctypes.c_void_p(16), 4, 128, 128, ctypes.c_void_p(16), None, -1, None),
     "is not bf16"),
])
def test_host_side_validation(call, msg):
    rc = call()
    assert rc == -1 or rc == -3
    assert msg in _err()


def _attn_splits(rows, n_slots, g, target=256):
    """Splits per row of qkv_sparse_attention: a workgroup round covers
    4 waves x 32 slots (G = 1, VALU kernel) or 4 waves x 16 slots (G >= 2,
    MFMA kernel); chunks per wave double (up to 16 for G = 1, else 32) while
    one workgroup does not cover the row and the grid keeps at least
    ``target`` workgroups."""
    per_iter = 128 if g == 1 else 64
    max_iters = 16 if g == 1 else 32
    it = 1
    while it < max_iters and per_iter * it < n_slots and rows * -(-n_slots // (per_iter * it * 2)) >= target:
        it *= 2
    return -(-n_slots // (per_iter * it))


def test_workspace_size_formula():
    # 65536 ticket words + rows * splits * G * (D + 2) floats
    t = 65536
    assert _attn_splits(64, 2048, 2) == 4             # cfg2: 4 splits of 512 slots
    assert _attn_splits(256, 4096, 4) == 2            # cfg3: 2 splits of 2048 slots
    assert _attn_splits(8, 300, 8) == 5
    # sized for the larger of the call's own splits and the bound on the
    # splits of smaller calls, 2 * (ceil(256 / rows) - 1) (capped by the
    # slot count): 6 at cfg2 (64 rows), 0 at cfg3 (256 rows)
    for b, hq, hkv, n_sel, block, splits in [(8, 32, 8, 128, 16, 6), (32, 32, 8, 256, 16, 2),
                                             (1, 8, 8, 7, 64, 4), (8, 16, 8, 2048, 16, 16)]:
        rows, g = b * hkv, hq // hkv
        assert lib.qkv_sparse_attention_workspace_bytes(b, hq, hkv, 128, n_sel, block) == \
            4 * (t + rows * splits * g * 130)
    assert lib.qkv_sparse_attention_workspace_bytes(1, 16, 8, 64, 256, 1) == -1


@pytest.mark.parametrize("b,hq,hkv,block", [(1, 32, 8, 16), (8, 32, 8, 16), (1, 16, 8, 1), (1, 64, 8, 1),
                                            (2, 8, 4, 16), (4, 16, 8, 64), (32, 32, 8, 16)])
def test_workspace_covers_every_smaller_selection(b, hq, hkv, block):
    # The split count is not monotonic in the slot count; a workspace sized
    # for n_sel must still serve every call with fewer blocks (brute force).
    rows, g = b * hkv, hq // hkv
    t = 65536
    worst = 0
    for n_sel in range(1, 1200 if block > 1 else 9000, 1 if block > 1 else 7):
        worst = max(worst, 4 * (t + rows * _attn_splits(rows, n_sel * block, g) * g * 130))
        got = lib.qkv_sparse_attention_workspace_bytes(b, hq, hkv, 128, n_sel, block)
        assert got >= worst, (n_sel, got, worst)


def test_python_wrappers_refuse_cpu_tensors():
    import torch

    from kv_cache_amd import qabs_cuda_kernels as Q

    q = torch.zeros(1, 2, 8)
    with pytest.raises(RuntimeError, match="query must be CUDA"):
        Q.partial_scores(q, torch.zeros(1, 2, 4, 8), 2)
    with pytest.raises(RuntimeError, match="query must be CUDA"):
        Q.final_attention(q, torch.zeros(1, 2, 4, 8), torch.zeros(1, 2, 4, 8),
                          torch.zeros(1, 2, 3, dtype=torch.long), torch.ones(1, 2, 3, dtype=torch.bool), 1.0)


def test_reuse_block_final_count():
    # keep = ceil(0.02 * 100) = 2; body = min(open range, keep * bs + 2 * (bs - 1))
    assert lib.qkv_reuse_block_final_count(100, 16, 0, 0, 0.02, 0) == min(100, 2 * 16 + 30)
    # sink 4, recent 8: open range 88, body 62, + 4 + 8 + self
    assert lib.qkv_reuse_block_final_count(100, 16, 4, 8, 0.02, 1) == 62 + 4 + 8 + 1
    assert lib.qkv_reuse_block_final_count(1000, 64, 0, 0, 0.5, 0) == 1000
    for hist, sink, recent, frac, ks in [(100, 4, 8, 0.02, 1), (5000, 10, 10, 0.03, 1)]:
        # blocks of one position: the plain final list
        assert lib.qkv_reuse_block_final_count(hist, 1, sink, recent, frac, ks) == \
            lib.qkv_reuse_final_count(hist, sink, recent, frac, ks)
    # a sink over the whole history leaves no body; the plain list keeps 4 invalid slots
    assert lib.qkv_reuse_block_final_count(37, 1, 50, 0, 0.1, 0) == 37
    assert lib.qkv_reuse_final_count(37, 50, 0, 0.1, 0) == 4 + 37
    assert lib.qkv_reuse_block_final_count(0, 16, 0, 0, 0.1, 1) == -1
    assert lib.qkv_reuse_block_final_count(10, 0, 0, 0, 0.1, 1) == -1
