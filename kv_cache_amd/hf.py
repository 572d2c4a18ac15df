"""HuggingFace transformers integration: decode-time append of the int4 K
structures inside a ``Cache``, and an attention function that runs the int4
sparse decode step on it.

The reference reaches its selection through HF's eager attention, which it
patches (evaluate_qwen3_top2_head_limit3_ppl.py:6934-6944), and keeps an
auxiliary K copy (dim-major bf16) that it grows by one column per decode step
(EV:2018-2042).  Here the auxiliary structure is the int4 cache of
``int4.Int4KCache``: after prefill the packed K, the static channel subset and
the subset slab are built once; every later token is quantized into them in
place (``int4_pack_k`` / ``build_slab`` over ``[t, t+1)``) as HF appends it to
the bf16 (or fp16) cache.  K/V live in preallocated buffers of a fixed capacity, so no
step reallocates or copies the history.

Use:

    from kv_cache_amd import hf
    hf.register()                                         # attn_implementation "int4_sparse"
    model.config._attn_implementation = "int4_sparse"
    cache = hf.Int4SparseCache(capacity=40960, group=32, selected=32, block=16, topk=128)
    out = model(input_ids, past_key_values=cache, use_cache=True)       # prefill: dense SDPA
    out = model(next_ids, past_key_values=cache, use_cache=True)        # decode: int4 sparse

Prefill (more than one query per call) runs dense SDPA on the GPU, as the
reference's prefill runs dense HF attention (EV:7079-7111), with transformers'
SDPA mask (``register`` registers it for the new name, so padding is applied).
Decode steps with one query per sequence run the int4 path with the
reference's decode semantics (EV:4419-4460, 2938-2982): the blocks are chosen
over the history (every cached token but the current one), and the attention
covers them plus the protected tokens -- ``protect_sink`` first tokens,
``protect_recent`` last history tokens and, with ``keep_self`` (the
reference's default), the current token.  The int4 kernels take no per-token
mask, so a decode step on a padded batch (a mask that hides cached positions)
raises instead of attending to the padding.  The channel subset is the one
chosen when the int4 structures are built at the first decode step (the
static per-KV-head subset of the int4 design); later tokens are quantized
into it.

The reference's other decode modes run through ``register_mode(mode,
capacity)``: the candidate-reuse modes (``qabs{S}cand{pct}reuse…``), the
lagged modes (``lagtop2`` / ``lagrefresh{N}`` / ``qdrift…`` / ``pconf{T}`` +
``qabs{S}cand{pct}``), the exact candidate attention (``qabs{S}cand{pct}
[append|r{N}]attn``) and the block selectors (``qbb…`` / ``brep…`` /
``qboracle…``), each through its native decode step (``reuse.ReuseDecodeStep``,
``reuse.LaggedReuseDecodeStep``, ``reuse.QabsCandidateAttentionStep``,
``blocksel.BlockSelectDecodeStep``), one per attention layer, on any HF cache
(K/V [B, Hkv, T, D] with the current token last).  As the reference's hook
dispatches these modes only for one query per sequence (EV:6236, 6308,
6414-6448), prefill stays dense SDPA.
"""

from __future__ import annotations

import functools
import math
import weakref

import torch

from . import int4 as K

# Cache layers by the address of their K buffer: the attention function gets
# K as a view of that buffer and finds the layer's int4 state through it.
# Weak references, so a freed cache's address cannot match a later tensor.
_LAYERS: "weakref.WeakValueDictionary[int, Int4CacheLayer]" = weakref.WeakValueDictionary()


class Int4CacheLayer:
    """One layer's K/V (bf16 or fp16) in preallocated buffers plus its int4 structures."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, capacity: int, group: int, selected: int, block: int, topk: int, protect_sink: int = 0,
                 protect_recent: int = 0, keep_self: bool = True):
        self.capacity = K.round_capacity(capacity)
        self.group, self.selected, self.block, self.topk = int(group), int(selected), int(block), int(topk)
        self.protect = dict(protect_sink=max(0, int(protect_sink)), protect_recent=max(0, int(protect_recent)),
                            keep_self=bool(keep_self))
        self.keys = self.values = None
        self.is_initialized = False
        self.length = 0
        self.int4 = None          # Int4KCache once built
        self.bufs = None          # decode-step buffers

    def __repr__(self):
        return f"Int4CacheLayer(length={self.length}, capacity={self.capacity})"

    # -- CacheLayerMixin protocol ------------------------------------------
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        b, h, _, d = key_states.shape
        dev = key_states.device
        self.dtype, self.device = key_states.dtype, dev
        self._k = torch.empty((b, h, self.capacity, d), dtype=key_states.dtype, device=dev)
        self._v = torch.empty((b, h, self.capacity, d), dtype=value_states.dtype, device=dev)
        _LAYERS[self._k.data_ptr()] = self
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.size(-2)
        t0, t1 = self.length, self.length + n
        if t1 > self.capacity:
            raise RuntimeError(f"Int4 cache capacity {self.capacity} exceeded ({t1} tokens)")
        self._k[:, :, t0:t1].copy_(key_states)
        self._v[:, :, t0:t1].copy_(value_states)
        self.length = t1
        self.keys, self.values = self._k[:, :, :t1], self._v[:, :, :t1]
        if self.int4 is not None:
            self.append_int4(t0, t1)
        return self.keys, self.values

    def get_mask_sizes(self, query_length: int):
        return self.length + query_length, 0

    def get_seq_length(self) -> int:
        return self.length

    def get_max_length(self) -> int:
        return self.capacity

    def reset(self) -> None:
        self.length = 0
        self.int4 = None

    def offload(self):
        raise RuntimeError("Int4CacheLayer cannot be offloaded")

    prefetch = offload

    # -- int4 structures ---------------------------------------------------
    def build_int4(self) -> None:
        """Pack the cached tokens, choose the channel subset, build the slab."""
        if self.keys.dtype not in (torch.bfloat16, torch.float16):
            raise RuntimeError(f"the int4 path needs bfloat16 or float16 K/V, got {self.keys.dtype}")
        t = self.length
        packed, scales = K.int4_pack_k(self._k, self.group, capacity=self.capacity, t_end=t)
        chan, _ = K.select_channels(packed, scales, t, self.group, self.selected)
        slab, slab_scales = K.build_slab(self._k, chan, capacity=self.capacity, t_end=t)
        self.int4 = K.Int4KCache(packed, scales, chan, slab, slab_scales, t, self.group)

    def append_int4(self, t0: int, t1: int) -> None:
        """Quantize tokens [t0, t1) into the packed K and the slab (the channel
        subset stays the one chosen at prefill)."""
        c = self.int4
        K.int4_pack_k(self._k, self.group, packed=c.packed, scales=c.scales, t_begin=t0, t_end=t1)
        K.build_slab(self._k, c.chan_idx, slab=c.slab, slab_scales=c.slab_scales, t_begin=t0, t_end=t1)
        c.tokens = t1

    def decode_buffers(self, batch: int, q_heads: int, kv_heads: int, head_dim: int):
        """Block maxima, selection, workspaces and output sized for the full
        capacity, allocated once (flat, so that each step takes a contiguous
        view of its own size)."""
        if self.bufs is None:
            nb = math.ceil(self.capacity / self.block)
            k = min(self.topk, nb)
            dev = self.device
            n_ws = K.protected_workspace_blocks(k, self.block, self.capacity - 1, **self.protect)
            self.bufs = {
                "bmax": torch.empty(batch * kv_heads * nb, dtype=torch.float32, device=dev),
                "sel": torch.empty(batch * kv_heads * k, dtype=torch.int32, device=dev),
                "topk_ws": K.topk_workspace(batch * kv_heads, nb, k, dev),
                "attn_ws": K.attention_workspace(batch, q_heads, kv_heads, head_dim, n_ws, self.block, dev),
            }
        return self.bufs


class Int4SparseCache:
    """A transformers ``Cache`` whose layers keep K/V in preallocated buffers
    and append the int4 structures at every decode step."""

    def __new__(cls, capacity: int, group: int = 32, selected: int = 32, block: int = 16, topk: int = 128, *,
                protect_sink: int = 0, protect_recent: int = 0, keep_self: bool = True):
        from transformers.cache_utils import Cache, CacheLayerMixin

        layer_cls = _layer_class(CacheLayerMixin)
        cache = Cache(layer_class_to_replicate=functools.partial(
            layer_cls, capacity, group, selected, block, topk, protect_sink, protect_recent, keep_self))
        return cache


@functools.lru_cache(maxsize=1)
def _layer_class(mixin):
    # Int4CacheLayer registered as a CacheLayerMixin so transformers' checks accept it.
    return type("Int4CacheLayerHF", (Int4CacheLayer, mixin), {"__init__": Int4CacheLayer.__init__})


def int4_sparse_attention_forward(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                  attention_mask, scaling: float | None = None, dropout: float = 0.0, **kwargs):
    """HF attention interface (query [B,Hq,q,D]; key/value [B,Hkv,T,D]) ->
    (out [B,q,Hq,D], None).  One query per sequence on an Int4SparseCache:
    int4 scoring of the history + top-k blocks + GQA sparse attention over
    them and the protected tokens; otherwise dense SDPA."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    layer = _LAYERS.get(key.data_ptr())
    if query.size(2) != 1 or layer is None or layer.keys is None or key.size(2) != layer.length:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    if layer.int4 is None:
        # once per sequence, when the int4 structures are built: the cached
        # positions' padding does not change later, and new tokens are real
        if attention_mask is not None and not _all_visible(attention_mask, layer.length):
            raise RuntimeError("int4 sparse decode does not support padded batches (the attention mask hides cached "
                               "positions); decode such batches with dense attention")
        layer.build_int4()
    b, hq, _, d = query.shape
    hkv = key.size(1)
    t = layer.length
    history = t - 1                       # the current token is not a candidate (EV:4414-4415)
    if history < 1:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    scaling = d ** -0.5 if scaling is None else float(scaling)
    bufs = layer.decode_buffers(b, hq, hkv, d)
    c = layer.int4
    nb = math.ceil(history / layer.block)
    k = min(layer.topk, nb)
    q = query[:, :, 0, :].contiguous()
    bmax = bufs["bmax"][: b * hkv * nb].view(b, hkv, nb)
    K.decode_scores(q, c.chan_idx, c.slab, c.slab_scales, history, layer.block, bmax=bmax)
    sel = bufs["sel"][: b * hkv * k].view(b, hkv, k)
    if nb <= K.SELECT_MAX_BLOCKS:
        out = K.sparse_attention_select(q, layer.keys, layer.values, bmax, k, layer.block, history, scaling,
                                        workspace=bufs["attn_ws"], sel_out=sel, **layer.protect)
    else:
        K.block_topk(bmax, k, out=sel, workspace=bufs["topk_ws"])
        out = K.sparse_attention(q, layer.keys, layer.values, sel, layer.block, history, scaling,
                                 workspace=bufs["attn_ws"], **layer.protect)
    # a fresh output per call: callers may keep a step's attention output
    # (hooks, captured activations) while later steps run
    return out[:, None].to(query.dtype), None


def _all_visible(mask: torch.Tensor, length: int) -> bool:
    """True when a decode step's attention mask ([B, 1, q, T], bool or
    additive float) hides none of the first ``length`` positions."""
    m = mask[..., -1, :length]
    return bool(m.all()) if m.dtype == torch.bool else bool((m == 0).all())


def register(name: str = "int4_sparse") -> str:
    """Register the attention function with transformers under ``name``."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

    AttentionInterface.register(name, int4_sparse_attention_forward)
    # without a mask function of its own a custom implementation gets no mask
    # at all, padding included; SDPA's mask is the one its prefill path uses
    AttentionMaskInterface.register(name, sdpa_mask)
    return name


def native_step_class(mode: str):
    """The decode step that serves a reference mode string, or ValueError."""
    from . import blocksel, reuse

    if reuse.is_lagged_mode(mode):
        return reuse.LaggedReuseDecodeStep
    for parse, cls in ((reuse.parse_reuse_mode, reuse.ReuseDecodeStep),
                       (reuse.parse_qabs_attn_mode, reuse.QabsCandidateAttentionStep),
                       (blocksel.parse_block_mode, blocksel.BlockSelectDecodeStep)):
        try:
            parse(mode)
        except (RuntimeError, ValueError):
            continue
        return cls
    raise ValueError(f"{mode!r} is not a mode served by a native decode step")


def register_mode(mode: str, capacity: int, *, name: str | None = None, **step_kwargs) -> str:
    """Register an attention implementation (default name ``qkv_<mode>``) that
    runs ``mode``'s native decode step for one query per sequence and dense
    SDPA otherwise.  ``capacity`` bounds the cached tokens per sequence;
    ``step_kwargs`` go to the step (``top_fraction``, ``protect_sink``,
    ``protect_recent``, ``keep_self``, ``candidate_selection``, …, as the
    reference's flags).  The steps, one per attention module, are in the
    returned function's ``steps`` (``ATTENTION_STEPS[name]``); each starts a
    new sequence by itself when the history does not continue its last call's
    (EV:1651's query-token check)."""
    from transformers import AttentionInterface
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

    cls = native_step_class(mode)
    steps: weakref.WeakKeyDictionary = weakref.WeakKeyDictionary()

    def forward(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, attention_mask,
                scaling: float | None = None, dropout: float = 0.0, **kwargs):
        if query.size(2) != 1:
            return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                          scaling=scaling, **kwargs)
        if attention_mask is not None and not _all_visible(attention_mask, key.size(2)):
            raise RuntimeError(f"{mode} decode does not support padded batches (the attention mask hides cached "
                               "positions); decode such batches with dense attention")
        b, hq, _, d = query.shape
        hkv = key.size(1)
        step = steps.get(module)
        if (step is None or (step.batch, step.q_heads, step.kv_heads, step.head_dim) != (b, hq, hkv, d)
                or step.dtype != query.dtype):
            step = cls(mode, b, hq, hkv, d, capacity, device=query.device, **{**step_kwargs, "dtype": query.dtype})
            steps[module] = step
        scaling = d ** -0.5 if scaling is None else float(scaling)
        out = step(query[:, :, 0, :], key, value, scaling)
        # the step's output buffer is overwritten by its next call
        return out[:, None].clone(), None

    forward.steps = steps
    name = name or f"qkv_{mode}"
    AttentionInterface.register(name, forward)
    AttentionMaskInterface.register(name, sdpa_mask)
    ATTENTION_STEPS[name] = steps
    return name


ATTENTION_STEPS: dict = {}
