"""MI355X-native Qwen3 sparse-attention KV-retrieval path (gfx950 HIP kernels
behind a C-ABI library, ``libqkv.so``, driven from PyTorch-ROCm).

``kv_cache_amd.qabs_cuda_kernels`` is the drop-in for the reference module
of the same name; ``kv_cache_amd.int4`` is the int4 scoring / selection /
sparse-attention path.
"""

from . import _lib
from .int4 import (
    Int4KCache,
    SparseDecodeStep,
    block_topk,
    build_slab,
    decode_scores,
    int4_pack_k,
    query_words,
    select_channels,
    sparse_attention,
)
from .qabs_cuda_kernels import (
    candidate_full_scores,
    final_attention,
    partial_scores,
    partial_scores_dim_major,
)

load = _lib.load

__all__ = [
    "Int4KCache", "SparseDecodeStep", "block_topk", "build_slab", "decode_scores", "int4_pack_k", "query_words",
    "select_channels", "sparse_attention", "candidate_full_scores", "final_attention",
    "partial_scores", "partial_scores_dim_major", "load",
]
