"""Mode strings and budget arithmetic of the reference's sparse decode, mapped
onto the int4 step's parameters.

The reference selects its decode path with a mode string (evaluate_qwen3_top2_
head_limit3_ppl.py, parse_mode_config EV:451-476, 495) and derives the budget
from it:

* ``qabs{S}cand{pct}attn`` (EV:473, 748-754): score every history key on the S
  channels of largest |q|, keep ``ceil(pct% * history)`` of them, attend
  (EV:4400-4502).
* ``qboracle{bs}q{S}s{scan}cand{pct}`` (EV:495, 798-806): max-pool the partial
  scores per block of bs keys, keep the ``ceil(scan% * history / bs)`` best
  blocks (EV:5038-5046), then a candidate top-k inside them.

``history`` is the key count without the current token (EV:4014-4015,
5026).  The int4 path (``int4.SparseDecodeStep``) scores the S channels of a
static per-KV-head subset, max-pools per block and attends over the kept
blocks; ``decode_plan`` gives its (channels, block, top-k blocks) for a mode.
Channel counts round up to the slab sizes the kernels build (16, 32, 64, 128).
"""

from __future__ import annotations

import math
import re
from dataclasses import dataclass

# Suffixes of the qabs family that share the (S, pct) prefix (EV:749).  The
# int4 step plans "attn" only; the exact fp32 "attn" / "appendattn" /
# "r{N}attn" steps, the "reuse..." steps and the lagged prefixes are served by
# kv_cache_amd.reuse (QabsCandidateAttentionStep, ReuseDecodeStep,
# LaggedReuseDecodeStep); the shared / top2 suffixes are other selectors.
_QABS = re.compile(
    r"(?:qabs|lagtop2qabs|lagrefresh\d+qabs|qdrift(?:maj|head|share|cos|coshead)?qabs|pconf\d+(?:p\d+)?qabs)"
    r"(\d+)cand(\d+(?:p\d+)?)"
    r"(keep|rerank|reuse(?:2set|final)?(?:blk\d+)?|r\d+attn|sharedr\d+attn|sharedtop2attn|sharedattn|"
    r"top2(?:hlim\d+|global)?attn|appendattn|attn)?")
_QBORACLE = re.compile(r"qboracle(\d+)q(\d+)s(\d+(?:p\d+)?)cand(\d+(?:p\d+)?)")
SLAB_SIZES = (16, 32, 64, 128)


def _percent(text: str) -> float:
    """'6p25' -> 0.0625 (the reference writes a decimal point as 'p')."""
    return float(text.replace("p", ".")) / 100.0


def parse_qabs_partial_rerank_params(mode: str) -> tuple[int, float] | None:
    """(dim_count, candidate_fraction) of a qabs-family mode, else None (EV:748-754)."""
    m = _QABS.fullmatch(mode)
    if not m:
        return None
    return int(m.group(1)), _percent(m.group(2))


def parse_qboracle_params(mode: str) -> tuple[int, int, float, float] | None:
    """(block_size, dim_count, scan_fraction, candidate_fraction), else None (EV:798-806)."""
    m = _QBORACLE.fullmatch(mode)
    if not m:
        return None
    return max(1, int(m.group(1))), int(m.group(2)), _percent(m.group(3)), _percent(m.group(4))


def history_count(key_count: int) -> int:
    """Keys a decode step may select: all but the current token (EV:4014-4015)."""
    return max(0, int(key_count) - 1)


def candidate_count(fraction: float, history: int) -> int:
    """min(history, max(1, ceil(fraction * history))) (EV:4087, 4423, 5050)."""
    return min(int(history), max(1, math.ceil(fraction * history)))


def scan_block_count(scan_fraction: float, history: int, block: int) -> int:
    """min(ceil(history / block), max(1, ceil(scan_fraction * history / block))) (EV:5044-5045)."""
    blocks = math.ceil(history / block)
    return min(blocks, max(1, math.ceil(scan_fraction * history / block)))


def selected_dims(dim_count: int, head_dim: int) -> int:
    """Channel count after the reference's clamp to [1, min(D, 128)] (QK:120, EV:4025),
    rounded up to a slab size of the int4 kernels."""
    s = min(max(1, int(dim_count)), min(int(head_dim), 128))
    for size in SLAB_SIZES:
        if s <= size:
            return min(size, int(head_dim))
    return SLAB_SIZES[-1]


@dataclass(frozen=True)
class DecodePlan:
    """Parameters of one int4 sparse decode step for a reference mode."""
    mode: str
    selected: int        # channels of the scoring slab
    block: int           # keys per selection block
    topk: int            # selected blocks per (sequence, KV head)
    history: int         # keys the budget was computed on

    @property
    def tokens_kept(self) -> int:
        return min(self.history, self.topk * self.block)


def decode_plan(mode: str, key_count: int, head_dim: int = 128) -> DecodePlan | None:
    """The int4 step for a qabs{S}cand{pct}attn or qboracle mode at key_count
    keys (None for other modes or an empty history)."""
    history = history_count(key_count)
    if history == 0:
        return None
    qb = parse_qboracle_params(mode)
    if qb is not None:
        block, dims, scan, _ = qb
        return DecodePlan(mode, selected_dims(dims, head_dim), block, scan_block_count(scan, history, block), history)
    m = _QABS.fullmatch(mode)
    if m is not None and m.group(3) == "attn" and mode.startswith("qabs"):
        dims, frac = int(m.group(1)), _percent(m.group(2))
        return DecodePlan(mode, selected_dims(dims, head_dim), 1, candidate_count(frac, history), history)
    return None
