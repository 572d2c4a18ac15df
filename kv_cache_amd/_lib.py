"""ctypes binding of libqkv.so, the gfx950 C-ABI library.

``load()`` is the singleton that replaces the reference's lazily JIT-built
extension (``_load_extension``, qabs_cuda_kernels.py:642-651).  There is no
fallback: if the library is missing or does not load, calls raise
``RuntimeError``.  torch is imported first so that the library binds to the
HIP runtime torch already loaded (both carry the soname libamdhip64.so.7),
which makes torch's device pointers and streams valid in it.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import re
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL so the HIP runtime is shared)

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libqkv.so"
HEADER = PKG.parent / "include" / "qkv.h"
ABI_VERSION = 2

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_c = ctypes
_vp, _i64, _i32, _f32, _f64 = _c.c_void_p, _c.c_int64, _c.c_int, _c.c_float, _c.c_double
_P = _c.POINTER

# name -> (restype, argtypes); mirrors include/qkv.h.
_PROTOTYPES = {
    "qkv_abi_version": (_i32, []),
    "qkv_last_error": (_c.c_char_p, []),
    "qkv_partial_scores": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _P(_i64), _i64, _vp]),
    "qkv_partial_scores_dim_major": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64,
                                            _P(_i64), _vp]),
    "qkv_candidate_full_scores": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64,
                                         _P(_i64), _i64, _i64, _f32, _vp]),
    "qkv_final_attention": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64,
                                   _f32, _vp]),
    "qkv_int4_pack_k": (_i32, [_vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i32, _vp]),
    "qkv_int4_select_channels": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "qkv_int4_build_slab": (_i32, [_vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp,
                                   _i64, _i32, _vp]),
    "qkv_int4_query_words": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i32, _vp]),
    "qkv_int4_decode_scores": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64,
                                      _i64, _vp, _vp, _vp, _vp, _i32, _vp]),
    "qkv_topk": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "qkv_topk_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "qkv_topk_ws": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp]),
    "qkv_topk_set_wait_limit": (_i32, [_i64]),
    "qkv_prefill_quantize_query": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _vp]),
    "qkv_prefill_block_scores": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                        _vp, _vp]),
    "qkv_prefill_block_topk": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "qkv_sparse_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "qkv_sparse_attention": (_i32, [_vp, _vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                    _i64, _f32, _vp, _i64, _vp, _i32, _vp]),
    "qkv_sparse_attention_select": (_i32, [_vp, _vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                           _i64, _i64, _f32, _vp, _i64, _vp, _vp, _i32, _vp]),
    "qkv_sparse_attention_protected": (_i32, [_vp, _vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64,
                                              _i64, _i64, _i64, _i64, _i32, _f32, _vp, _i64, _vp, _vp, _i32, _vp]),
    "qkv_hbm_read_probe_sink_words": (_i64, [_i64]),
    "qkv_hbm_read_probe": (_i32, [_vp, _i64, _vp, _i64, _vp]),
    "qkv_sparse_attention_select_noalloc": (_i32, [_vp, _vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp,
                                                   _i64, _i64, _i64, _f32, _vp, _vp, _i32, _vp]),
    "qkv_token_attention": (_i32, [_vp, _vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _i64, _f32, _vp,
                                   _i64, _vp, _i32, _vp]),
    "qkv_reuse_final_count": (_i64, [_i64, _i64, _i64, _f64, _i32]),
    "qkv_reuse_select_workspace_bytes": (_i64, [_i64, _i64, _f64]),
    "qkv_reuse_select": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
                                _i64, _f64, _i32, _f32, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "qkv_candidate_mask_workspace_bytes": (_i64, [_i64, _i64, _i32, _i64, _i64]),
    "qkv_candidate_mask": (_i32, [_vp, _i64, _i64, _i64, _i32, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _i64,
                                  _vp]),
    "qkv_reuse_lag_flags": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _P(_i64),
                                   _i64, _vp, _i64, _f32, _f32, _vp, _vp, _i64, _vp]),
    "qkv_reuse_lag_flags_workspace_bytes": (_i64, [_i64, _i64]),
    "qkv_qabs_candidate_select_workspace_bytes": (_i64, [_i64, _i64, _f64]),
    "qkv_final_indices_from_selected": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i64,
                                               _vp]),
    "qkv_qabs_candidate_select": (_i32, [_vp, _i64, _i64, _i64, _f64, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _vp,
                                         _vp, _i64, _vp, _i64, _vp]),
    "qkv_reuse_lag_candidates": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                                        _i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "qkv_reuse_lag_union": (_i32, [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _i32, _i64, _i64, _vp, _i64, _vp]),
    "qkv_reuse_lag_flags_bits": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp,
                                        _P(_i64), _i64, _vp, _i64, _f32, _f32, _vp, _vp, _i64, _vp]),
    "qkv_reuse_lag_candidates_bits": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                             _vp, _i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "qkv_reuse_lag_union_bits": (_i32, [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _i32, _i64, _i64, _vp, _i64,
                                        _vp]),
    "qkv_reuse_block_final_count": (_i64, [_i64, _i64, _i64, _i64, _f64, _i32]),
    "qkv_reuse_expand_blocks_bits": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _f64, _i32, _vp, _vp, _vp,
                                            _i64, _vp]),
    "qkv_reuse_expand_blocks": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _f64, _i32, _vp, _vp, _vp, _i64,
                                       _vp]),
    "qkv_reuse_partial_scores": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                        _vp]),
    "qkv_threshold_mask_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "qkv_threshold_mask": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "qkv_dim_major_append": (_i32, [_vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _vp, _P(_i64), _vp]),
    "qkv_block_meta_bytes": (_i64, [_i32, _i64, _i64, _i64, _i64]),
    "qkv_block_meta_update": (_i32, [_i32, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                     _i32, _vp]),
    "qkv_block_scores": (_i32, [_i32, _vp, _vp, _P(_i64), _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                _vp, _i64, _i32, _vp]),
    "qkv_block_scan_scores": (_i32, [_vp, _vp, _P(_i64), _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                     _i64, _i64, _f32, _vp, _vp, _i64, _i32, _vp]),
    "qkv_block_max_partial_scores": (_i32, [_vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                                            _i64, _i32, _vp]),
    "qkv_brep_partial_scores": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _P(_i64), _i64, _i64,
                                       _i64, _f64, _vp]),
    "qkv_final_list_count": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "qkv_block_rerank": (_i32, [_vp, _vp, _P(_i64), _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _i64,
                                _i64, _i64, _i64, _i64, _i32, _f32, _vp, _i64, _vp, _i64, _i32, _vp, _i64, _i32, _vp]),
    "qkv_block_rerank_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i32]),
    "qkv_reuse_candidates_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "qkv_qabs_candidates_workspace_bytes": (_i64, [_i64, _i64, _f64]),
    "qkv_qabs_candidates": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _i64, _f64, _i64, _i64,
                                   _i32, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "qkv_int4_decode_topk": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp,
                                    _vp, _i64, _i32, _vp]),
    "qkv_reuse_candidates": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64,
                                    _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp]),
    "qkv_reuse_select_bits": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64,
                                     _i64, _i64, _f64, _i32, _f32, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp,
                                     _vp, _P(_i32), _vp]),
    "qkv_reuse_select_bits_blocks": (_i32, [_vp, _vp, _P(_i64), _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp,
                                            _i64, _i64, _i64, _f64, _i32, _f32, _i64, _vp, _i64, _vp, _vp, _vp,
                                            _i64, _vp, _i64, _vp]),
}

_LIB = None


def header_functions() -> list[str]:
    """Function names declared in include/qkv.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(qkv_\w+)\s*\(", text, re.M)))


def load() -> ctypes.CDLL:
    """Load libqkv.so once; raises RuntimeError if it is absent or stale."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("QKV_LIBRARY", LIB_PATH))
    if not path.exists():
        raise RuntimeError(f"{path} is not built: run `python -m kv_cache_amd.build` "
                           "(or __graft_entry__.build()) first")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.qkv_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI {lib.qkv_abi_version()}, expected {ABI_VERSION}: rebuild it")
    _LIB = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(load().qkv_last_error().decode())


def strides(*vals: int):
    arr = (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])
    return arr


_SAME_DEVICE = contextlib.nullcontext()


def on_device(device: torch.device):
    """torch.cuda.device(device), or a no-op when that device is already
    current (the per-call guard costs more than the launch it guards)."""
    idx = device.index
    if idx is None or torch.cuda.current_device() == idx:
        return _SAME_DEVICE
    return torch.cuda.device(device)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The current stream of t's device as a raw handle (without building a
    torch Stream object where torch offers that)."""
    if _RAW_STREAM is not None and t.device.type == "cuda":
        return _RAW_STREAM(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def half_code(name: str, t: torch.Tensor) -> int:
    """The C ABI dtype code of a bf16 or fp16 tensor (the 16-bit entry points);
    raises for any other dtype."""
    if t.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"{name} must be bfloat16 or float16, got {t.dtype}")
    return DTYPE_CODES[t.dtype]


def require_cuda(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be CUDA")
