"""Writes golden vectors for the stateful candidate-reuse decode step.

The reference's ``qabs{S}cand{pct}reuse[final|2set]`` driver
(``_qabs_reuse_fast_attention_forward``,
evaluate_qwen3_top2_head_limit3_ppl.py:3991-4397) keeps per-layer candidate
and final masks between decode steps (``ReuseCandidateState``, EV:1596-1759)
and mixes several module-level flags (EV:4147-4198); no closed form or
reference test pins that interplay.  This script imports the reference
module on the CPU (no GPU, no weights), runs a few consecutive decode steps
through the attention hook the model calls (``_limited_eager_attention_forward``,
EV:6236) on seeded synthetic q/K/V, and saves inputs and outputs:

* per step: the attention output [B, 1, Hq, D], and the reuse state the step
  leaves behind (current candidate mask and final mask, bool [B, Hq, hist]);
* the inputs: q for every step, K/V of the longest step (each step uses the
  prefix of the first T0 + step + 1 tokens).

Run from the repository root with the reference checked out at
/root/reference:

    python tests/golden/make_reuse_vectors.py

Outputs ``tests/golden/reuse_<name>.npz`` (a few hundred KB in all).
"""

from __future__ import annotations

import sys
import types
from pathlib import Path

import numpy as np
import torch

REF_SRC = Path("/root/reference/ymluo/projects/qwen3_top2_head_limit3_ppl/src")
OUT = Path(__file__).resolve().parent

# name: (mode, dtype, Hq, Hkv, T0, steps, top_fraction, sink, recent, keep_self, seed)
SCENARIOS = {
    "s8c5_fp32": ("qabs8cand5reuse", torch.float32, 4, 2, 240, 5, 0.05, 4, 4, True, 1),
    "s16c10_final_fp32": ("qabs16cand10reusefinal", torch.float32, 4, 2, 193, 4, 0.03, 0, 0, True, 2),
    "s8c3_2set_fp32": ("qabs8cand3reuse2set", torch.float32, 2, 1, 300, 4, 0.02, 2, 0, False, 3),
    "s8c5_bf16": ("qabs8cand5reuse", torch.bfloat16, 4, 2, 240, 4, 0.05, 3, 5, True, 4),
}


def run(ev, name, mode, dtype, hq, hkv, t0, steps, top_fraction, sink, recent, keep_self, seed):
    g = torch.Generator().manual_seed(seed)
    d = 128
    t_max = t0 + steps
    q = torch.randn((steps, 1, hq, 1, d), generator=g).to(dtype)
    # K/V values are bf16-representable (stored as bf16 bits); the fp32
    # scenarios still compute in fp32
    k = (torch.randn((1, hkv, t_max, d), generator=g) * 1.5).to(torch.bfloat16).to(dtype)
    v = torch.randn((1, hkv, t_max, d), generator=g).to(torch.bfloat16).to(dtype)
    scaling = d ** -0.5
    state = ev.ReuseCandidateState()
    module = types.SimpleNamespace(layer_idx=0, scaling=scaling)
    outs, cands, finals = [], [], []
    with ev.attention_mode(mode=mode, top_fraction=top_fraction, max_heads_per_token=3,
                           always_keep_self=keep_self, protect_sink_tokens=sink,
                           protect_recent_tokens=recent, load_stats=None, reuse_state=state,
                           qabs_fast_path=True):
        for s in range(steps):
            n = t0 + s + 1
            out, _ = ev._limited_eager_attention_forward(module, q[s], k[:, :, :n], v[:, :, :n], None,
                                                         scaling=scaling)
            rec = state.previous_layer[0]
            outs.append(out.float().numpy())
            hist = n - 1
            cand = np.zeros((1, hq, t_max), dtype=bool)
            fin = np.zeros((1, hq, t_max), dtype=bool)
            cand[..., :hist] = rec["candidate"].numpy()
            fin[..., :hist] = rec["final"].numpy()
            cands.append(cand)
            finals.append(fin)
    np.savez_compressed(
        OUT / f"reuse_{name}.npz", mode=np.array(mode), dtype=np.array(str(dtype).split(".")[-1]),
        q=q.float().numpy(), k_bf16=k.to(torch.bfloat16).view(torch.int16).numpy(),
        v_bf16=v.to(torch.bfloat16).view(torch.int16).numpy(), t0=t0, steps=steps,
        top_fraction=top_fraction, sink=sink, recent=recent, keep_self=keep_self, scaling=scaling,
        out=np.stack(outs), candidate=np.packbits(np.stack(cands), axis=-1),
        final=np.packbits(np.stack(finals), axis=-1), t_max=t_max)
    print(f"{name}: {mode} {dtype} Hq={hq} T0={t0} steps={steps} -> reuse_{name}.npz")


def main():
    sys.path.insert(0, str(REF_SRC))
    import evaluate_qwen3_top2_head_limit3_ppl as ev   # the reference module, CPU only

    torch.set_num_threads(1)
    for name, args in SCENARIOS.items():
        run(ev, name, *args)


if __name__ == "__main__":
    main()
