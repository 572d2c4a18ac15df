"""The benchmark configurations and their seeded synthetic inputs.

There are no checkpoints or datasets: K, V and q are drawn from N(0, 1) in
fp32 and cast to bf16, with 4 fixed outlier channels (one draw per seed,
shared by every head and layer) scaled x8 in K and V.  Configs 3 and 4 apply
RoPE (theta 1e6, the Qwen3 rotate-half form) to K at positions 0..T-1 and to
q at position T.  Config 4 plants one key per KV head whose cosine with the
group's mean query is 0.9.  Layer l of a run uses seed ``seed + l``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    tokens: int
    group: int         # int4 quantization group of the packed K cache
    selected: int      # channels per KV head in the scoring slab (S)
    block: int         # tokens per selection block
    topk: int          # selected blocks per (sequence, KV head)
    layers: int
    rope: bool
    planted: bool = False
    seed: int = 1234

    @property
    def g(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def rows(self) -> int:
        return self.batch * self.kv_heads

    @property
    def n_blocks(self) -> int:
        return -(-self.tokens // self.block)

    @property
    def scaling(self) -> float:
        return self.head_dim ** -0.5

    def slab_bytes_per_key(self) -> int:
        return self.selected // 2 + 2


@dataclass(frozen=True)
class PrefillConfig:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    queries: int
    tokens: int
    block: int
    topk: int
    seed: int = 1234

    @property
    def g(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def q_pos0(self) -> int:
        """Position of the chunk's first query: the last chunk of the prefill."""
        return self.tokens - self.queries

    @property
    def n_blocks(self) -> int:
        return -(-self.tokens // self.block)

    def visible_keys(self) -> int:
        """Sum over query rows of one head of the keys each one sees (causal)."""
        return sum(min(self.tokens, self.q_pos0 + i + 1) for i in range(self.queries))

    def int_ops(self) -> int:
        """Algorithmic int8 ops of one scoring pass: 2 * D per visible (query
        head, key) pair."""
        return 2 * self.head_dim * self.batch * self.q_heads * self.visible_keys()


CONFIGS = {
    "cfg1": DecodeConfig("qwen3-0.6b-1layer-b1-t4096", 1, 16, 8, 128, 4096, 32, 32, 1, 256, 1, False),
    "cfg2": DecodeConfig("qwen3-0.6b-28layer-b8-t32768", 8, 16, 8, 128, 32768, 32, 32, 16, 128, 28, False),
    "cfg3": DecodeConfig("qwen3-8b-36layer-b32-t32768", 32, 32, 8, 128, 32768, 128, 64, 16, 256, 36, True),
    "cfg4": DecodeConfig("qwen3-8b-1layer-b1-t131072-planted", 1, 32, 8, 128, 131072, 128, 64, 1, 1024, 1,
                         True, planted=True),
}
PREFILL = PrefillConfig("qwen3-8b-prefill-2048x65536", 1, 32, 8, 128, 2048, 65536, 64, 64)


def outlier_channels(head_dim: int, seed: int, count: int = 4) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(head_dim, generator=g)[:count].sort().values


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float = 1.0e6):
    """cos/sin tables fp32 [P, head_dim], computed in fp64 on the CPU."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    ang = positions.cpu().to(torch.float64)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().float(), ang.sin().float()


def apply_rope(x: torch.Tensor, positions: torch.Tensor, theta: float = 1.0e6) -> torch.Tensor:
    """x [..., T, D] fp32; rotate-half RoPE as in HF Qwen3."""
    d = x.size(-1)
    cos, sin = rope_tables(positions, d, theta)
    cos, sin = cos.to(x.device), sin.to(x.device)
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    rot = torch.cat([-x2, x1], dim=-1)
    return x * cos + rot * sin


def make_layer(cfg: DecodeConfig, layer: int = 0, device: str | torch.device = "cpu",
               tokens: int | None = None, batch: int | None = None):
    """Seeded (q [B,Hq,D], k, v [B,Hkv,T,D]) in bf16 for one layer, plus the
    planted positions (int64 [B,Hkv]) for planted configs (else None).

    ``tokens``/``batch`` shrink the shape for tests while keeping the
    distribution."""
    t = cfg.tokens if tokens is None else int(tokens)
    b = cfg.batch if batch is None else int(batch)
    seed = cfg.seed + layer
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    d = cfg.head_dim
    k = torch.randn((b, cfg.kv_heads, t, d), generator=gen, device=dev, dtype=torch.float32)
    v = torch.randn((b, cfg.kv_heads, t, d), generator=gen, device=dev, dtype=torch.float32)
    q = torch.randn((b, cfg.q_heads, d), generator=gen, device=dev, dtype=torch.float32)
    out_ch = outlier_channels(d, cfg.seed).to(dev)
    k[..., out_ch] *= 8.0
    v[..., out_ch] *= 8.0
    if cfg.rope:
        k = apply_rope(k, torch.arange(t, device=dev))
        q = apply_rope(q[:, :, None, :], torch.tensor([t], device=dev))[:, :, 0, :]
    planted = None
    if cfg.planted:
        planted = torch.randint(0, t, (b, cfg.kv_heads), generator=gen, device=dev)
        qmean = q.view(b, cfg.kv_heads, cfg.g, d).mean(dim=2)
        u = qmean / qmean.norm(dim=-1, keepdim=True)
        w = torch.randn((b, cfg.kv_heads, d), generator=gen, device=dev, dtype=torch.float32)
        w = w - (w * u).sum(-1, keepdim=True) * u
        w = w / w.norm(dim=-1, keepdim=True)
        bi = torch.arange(b, device=dev)[:, None].expand(b, cfg.kv_heads)
        hi = torch.arange(cfg.kv_heads, device=dev)[None, :].expand(b, cfg.kv_heads)
        norm = k[bi, hi, planted].norm(dim=-1, keepdim=True)
        k[bi, hi, planted] = norm * (0.9 * u + math.sqrt(1.0 - 0.81) * w)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16), planted


def make_prefill(cfg: PrefillConfig, device: str | torch.device = "cpu", tokens: int | None = None,
                 queries: int | None = None):
    """Seeded (q bf16 [B, Hq, Nq, D], k bf16 [B, Hkv, T, D]) of a prefill
    chunk: N(0, 1) with the 4 outlier channels of ``outlier_channels`` scaled
    x8 in both.  ``tokens``/``queries`` shrink the shape for tests."""
    t = cfg.tokens if tokens is None else int(tokens)
    nq = cfg.queries if queries is None else int(queries)
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(cfg.seed)
    d = cfg.head_dim
    k = torch.randn((cfg.batch, cfg.kv_heads, t, d), generator=gen, device=dev, dtype=torch.float32)
    q = torch.randn((cfg.batch, cfg.q_heads, nq, d), generator=gen, device=dev, dtype=torch.float32)
    out_ch = outlier_channels(d, cfg.seed).to(dev)
    k[..., out_ch] *= 8.0
    q[..., out_ch] *= 8.0
    return q.to(torch.bfloat16), k.to(torch.bfloat16)
