"""Writes golden vectors for the stateful candidate-reuse decode step and the
block-metadata selectors (qbb, brep).

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
  leaves behind (current candidate mask and final mask, bool [B, Hq, hist];
  the candidate thresholds, NaN where the step kept none; the top-|q| dims and
  their q values; the state's running count of refreshed heads);
* the inputs: q for every step, K/V of the longest step (each step uses the
  prefix of the first T0 + step + 1 tokens).

Run from the repository root with the reference checked out at
/root/reference:

    python tests/golden/make_reuse_vectors.py [scenario ...]

Outputs ``tests/golden/reuse_<name>.npz`` and ``tests/golden/block_<name>.npz``
(the stateless modes: qbb, brep, qboracle and qabs{S}cand{pct}attn).
"""

from __future__ import annotations

import re
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
    # block-expanded final selections (reuse…blk{bs}, EV:757-761, 4314-4316);
    # the histories run across block boundaries.  EV:955-960 test the mode's
    # suffix, so a "finalblk" or "2setblk" mode keeps both previous masks.
    # The bf16 seed is one where no tie decides a selection: neither a bf16
    # |q| tie at the S-th channel (torch.topk's order among ties is
    # unspecified, the reference's kernels take the lower channel,
    # QK:123-145) nor a tie of bf16-rounded rerank scores at the keep-th
    # place (the CPU fallback ranks bf16 products, EV:4290-4296; its kernel
    # ranks fp32 ones)
    "s8c5_blk16_fp32": ("qabs8cand5reuseblk16", torch.float32, 4, 2, 240, 5, 0.05, 4, 4, True, 5),
    "s16c10_finalblk8_bf16": ("qabs16cand10reusefinalblk8", torch.bfloat16, 4, 2, 203, 4, 0.03, 0, 6, True, 15),
    "s8c3_2setblk32_fp32": ("qabs8cand3reuse2setblk32", torch.float32, 2, 1, 300, 4, 0.02, 3, 0, False, 7),
    # the other candidate selections (--qabs_candidate_selection, EV:3958-3989):
    # + (selection, threshold sample size)
    "s8c5_sample64_fp32": ("qabs8cand5reuse", torch.float32, 4, 2, 600, 4, 0.05, 4, 4, True, 21,
                           "sample_quantile", 64),
    "s8c5_samplecover_fp32": ("qabs8cand5reusefinal", torch.float32, 2, 1, 100, 3, 0.05, 2, 2, False, 23,
                              "sample_quantile", 256),
    "s8c10_prevthr_fp32": ("qabs8cand10reuse", torch.float32, 4, 2, 400, 4, 0.03, 0, 6, True, 22,
                           "previous_threshold", 256),
}


# The lagged reuse modes (EV:4020-4198): lagtop2 (reuse the previous final
# selection), lagrefresh{N} (refresh every N-th query token), qdrift* (refresh
# when the top-|q| dims drift: any / majority / per head / shared across heads /
# with the cosine test) and pconf{T} (refresh heads whose previous final
# attention has an effective-sample fraction above T).  Their queries drift
# slowly on some heads and jump on others, so refreshes are mixed: q of head h
# at step s is scale_h * (base_h + eps_h * noise_{s,h}) / sqrt(1 + eps_h^2).  The bf16 seeds are
# ones with no |q| tie at the S-th dim in any step (torch.topk's order among
# ties is unspecified); scales stay at or below 1 so that the reference's bf16
# attention scores (rounded to bf16 before the softmax) stay within the bf16
# tolerance of an fp32 attention.
# name: (mode, dtype, Hq, Hkv, T0, steps, top_fraction, sink, recent, keep_self, seed)
LAG_EPS = (0.02, 3.0, 0.05, 0.3, 0.01, 2.0, 0.1, 1.0)
LAG_SCALE = (1.0, 0.3, 0.7, 1.0, 0.5, 0.9, 0.6, 0.8)
LAG_SCENARIOS = {
    "lagtop2_s8c5_bf16": ("lagtop2qabs8cand5", torch.bfloat16, 4, 2, 240, 4, 0.05, 4, 4, True, 641),
    "lagrefresh3_s8c5_bf16": ("lagrefresh3qabs8cand5", torch.bfloat16, 4, 2, 238, 5, 0.05, 3, 5, True, 142),
    "qdrift_s8c5_bf16": ("qdriftqabs8cand5", torch.bfloat16, 8, 2, 260, 5, 0.04, 4, 4, True, 7943),
    "qdriftmaj_s8c5_bf16": ("qdriftmajqabs8cand5", torch.bfloat16, 8, 2, 260, 5, 0.04, 4, 4, True, 6744),
    "qdrifthead_s8c5_bf16": ("qdriftheadqabs8cand5", torch.bfloat16, 8, 2, 260, 5, 0.04, 2, 6, True, 4845),
    "qdriftshare_s8c5_bf16": ("qdriftshareqabs8cand5", torch.bfloat16, 8, 2, 260, 5, 0.04, 4, 0, False, 4546),
    "qdriftcos_s16c10_bf16": ("qdriftcosqabs16cand10", torch.bfloat16, 8, 4, 230, 5, 0.03, 4, 4, True, 188247),
    "qdriftcoshead_s8c5_bf16": ("qdriftcosheadqabs8cand5", torch.bfloat16, 8, 2, 260, 5, 0.04, 0, 4, True, 2448),
    "pconf50_s8c5_bf16": ("pconf50qabs8cand5", torch.bfloat16, 8, 2, 260, 5, 0.04, 4, 4, True, 5349),
    "pconf37p5_s16c10_fp32": ("pconf37p5qabs16cand10", torch.float32, 8, 4, 230, 4, 0.03, 2, 3, True, 50),
    "qdrifthead_s8c5_fp32": ("qdriftheadqabs8cand5", torch.float32, 8, 2, 260, 4, 0.04, 2, 6, True, 51),
    # the other candidate selections on the lagged modes: they apply where every
    # head thresholds (a first step, a step-wide refresh, lagrefresh; EV:4116-4145)
    # + (selection, threshold sample size)
    "qdrift_sample64_s8c5_bf16": ("qdriftqabs8cand5", torch.bfloat16, 8, 2, 600, 5, 0.04, 4, 4, True, 3273,
                                  "sample_quantile", 64),
    "qdrifthead_sample64_s8c5_bf16": ("qdriftheadqabs8cand5", torch.bfloat16, 8, 2, 600, 5, 0.04, 2, 6, True, 3085,
                                      "sample_quantile", 64),
    "lagrefresh1_prevthr_s8c5_bf16": ("lagrefresh1qabs8cand5", torch.bfloat16, 4, 2, 300, 5, 0.05, 2, 3, True, 402,
                                      "previous_threshold", 256),
    "qdriftmaj_prevthr_s8c5_bf16": ("qdriftmajqabs8cand5", torch.bfloat16, 8, 2, 400, 5, 0.04, 4, 4, True, 803,
                                    "previous_threshold", 256),
    "qdriftcos_prevthr_s8c5_bf16": ("qdriftcosqabs8cand5", torch.bfloat16, 8, 2, 400, 5, 0.04, 4, 4, True, 803,
                                    "previous_threshold", 256),
}


def run(ev, name, mode, dtype, hq, hkv, t0, steps, top_fraction, sink, recent, keep_self, seed, selection="topk",
        sample_size=256, lagged=False):
    g = torch.Generator().manual_seed(seed)
    d = 128
    t_max = t0 + steps
    if lagged:
        eps = torch.tensor([LAG_EPS[h % len(LAG_EPS)] for h in range(hq)]).view(1, 1, hq, 1, 1)
        scale = torch.tensor([LAG_SCALE[h % len(LAG_SCALE)] for h in range(hq)]).view(1, 1, hq, 1, 1)
        base = torch.randn((1, 1, hq, 1, d), generator=g)
        noise = torch.randn((steps, 1, hq, 1, d), generator=g)
        q = (scale * (base + eps * noise) / torch.sqrt(1 + eps * eps)).to(dtype)
    else:
        q = torch.randn((steps, 1, hq, 1, d), generator=g).to(dtype)
    # K/V values are bf16-representable (stored as bf16 bits); the fp32
    # scenarios still compute in fp32
    k = (torch.randn((1, hkv, t_max, d), generator=g) * 1.5).to(torch.bfloat16).to(dtype)
    v = torch.randn((1, hkv, t_max, d), generator=g).to(torch.bfloat16).to(dtype)
    scaling = d ** -0.5
    state = ev.ReuseCandidateState()
    module = types.SimpleNamespace(layer_idx=0, scaling=scaling)
    outs, cands, finals, thresholds, qdims, qvals, refreshed = [], [], [], [], [], [], []
    with ev.attention_mode(mode=mode, top_fraction=top_fraction, max_heads_per_token=3,
                           always_keep_self=keep_self, protect_sink_tokens=sink,
                           protect_recent_tokens=recent, load_stats=None, reuse_state=state,
                           qabs_fast_path=True, qabs_candidate_selection=selection,
                           qabs_threshold_sample_size=sample_size):
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
            thr = rec.get("candidate_thresholds")   # None on the lagged modes' reuse steps
            thresholds.append(np.full((1, hq), np.nan, np.float32) if thr is None
                              else thr.float().numpy().reshape(1, hq))
            qdims.append(rec["qdim_indices"].numpy().astype(np.int32))
            qvals.append(rec["qdim_values"].float().numpy())
            refreshed.append(state.refresh_head_count)
    np.savez_compressed(
        OUT / f"reuse_{name}.npz", mode=np.array(mode), dtype=np.array(str(dtype).split(".")[-1]),
        q=q.float().numpy(), k_bf16=k.to(torch.bfloat16).view(torch.int16).numpy(),
        v_bf16=v.to(torch.bfloat16).view(torch.int16).numpy(), t0=t0, steps=steps,
        top_fraction=top_fraction, sink=sink, recent=recent, keep_self=keep_self, scaling=scaling,
        out=np.stack(outs), candidate=np.packbits(np.stack(cands), axis=-1),
        final=np.packbits(np.stack(finals), axis=-1), t_max=t_max, selection=np.array(selection),
        sample_size=sample_size, thresholds=np.stack(thresholds), qdim_indices=np.stack(qdims),
        qdim_values=np.stack(qvals), refresh_head_count=np.array(refreshed, dtype=np.int64))
    print(f"{name}: {mode} {dtype} {selection} Hq={hq} T0={t0} steps={steps} -> reuse_{name}.npz")


# Block-metadata selectors (qbb: Quest-style channel bounds, EV:5508-5617;
# brep: block representatives with their BlockRepState, EV:5361-5505, 1853-1918)
# and the other stateless decode modes whose final index list goes through
# _maybe_cuda_final_attention (qboracle, qabs{S}cand{pct}attn).
# name: (mode, dtype, Hq, Hkv, T0, steps, top_fraction, sink, recent, keep_self, seed)
BLOCK_SCENARIOS = {
    "qbb16q8s12cand4_fp32": ("qbb16q8s12cand4", torch.float32, 4, 2, 300, 3, 0.02, 3, 5, True, 11),
    "qbb8q16s25cand6p25_fp32": ("qbb8q16s25cand6p25", torch.float32, 4, 4, 201, 3, 0.03, 0, 0, False, 12),
    "brep16r2q8s12cand4_fp32": ("brep16r2q8s12cand4", torch.float32, 4, 2, 300, 3, 0.02, 3, 5, True, 13),
    "brep8r1q16s25cand6p25_fp32": ("brep8r1q16s25cand6p25", torch.float32, 2, 1, 233, 3, 0.03, 0, 4, True, 14),
    # block max-pool of the partial scores (qboracle, EV:5008-5097)
    "qboracle16q8s12cand4_fp32": ("qboracle16q8s12cand4", torch.float32, 4, 2, 300, 3, 0.02, 3, 5, True, 16),
    "qboracle8q16s25cand6p25_fp32": ("qboracle8q16s25cand6p25", torch.float32, 2, 1, 233, 3, 0.03, 0, 4, False, 17),
    # bf16 inputs, as the GPU step takes them; the seed is one where no tie of
    # bf16-rounded rerank scores decides the kept set (the CPU fallback ranks
    # bf16 matmul outputs, EV:5060-5067; kernels rank the fp32 scores)
    "qboracle16q8s12cand4_bf16": ("qboracle16q8s12cand4", torch.bfloat16, 8, 2, 400, 3, 0.02, 3, 5, True, 35),
    # the timed candidate-attention mode (qabs{S}cand{pct}attn, EV:4400-4502;
    # top_fraction is not used by it)
    "qabs8cand3attn_fp32": ("qabs8cand3attn", torch.float32, 4, 2, 300, 3, 0.02, 3, 5, True, 18),
    "qabs16cand10attn_fp32": ("qabs16cand10attn", torch.float32, 4, 4, 211, 3, 0.02, 0, 0, False, 19),
    "qabs8cand5attn_bf16": ("qabs8cand5attn", torch.bfloat16, 4, 2, 257, 3, 0.02, 4, 4, True, 20),
    # the appendattn variant keeps the selected copies of protected tokens
    # (EV:4451-4458, 2985-3022): wide protected ranges so that copies occur
    "qabs8cand5appendattn_fp32": ("qabs8cand5appendattn", torch.float32, 4, 2, 260, 3, 0.02, 12, 20, True, 24),
    "qabs16cand10appendattn_bf16": ("qabs16cand10appendattn", torch.bfloat16, 4, 2, 230, 3, 0.02, 8, 16, False,
                                    125),
    # the periodic variant reselects when the query token is a multiple of N
    # and otherwise reuses the last step's selection (EV:4505-4609; its state
    # is a ReuseCandidateState); the steps cross a multiple of N
    "qabs8cand5r3attn_fp32": ("qabs8cand5r3attn", torch.float32, 4, 2, 268, 5, 0.02, 4, 6, True, 26),
    "qabs8cand3r2attn_bf16": ("qabs8cand3r2attn", torch.bfloat16, 4, 2, 251, 5, 0.02, 2, 3, True, 727),
}


def run_block(ev, name, mode, dtype, hq, hkv, t0, steps, top_fraction, sink, recent, keep_self, seed):
    """Consecutive decode steps of a block selector; the final index list the
    step hands to its attention (its argument to _maybe_cuda_final_attention,
    which returns None on the CPU) is recorded as the final keep mask."""
    g = torch.Generator().manual_seed(seed)
    d = 128
    t_max = t0 + steps
    q = torch.randn((steps, 1, hq, 1, d), generator=g).to(dtype)
    k = (torch.randn((1, hkv, t_max, d), generator=g) * 1.5).to(torch.bfloat16).to(dtype)
    v = torch.randn((1, hkv, t_max, d), generator=g).to(torch.bfloat16).to(dtype)
    scaling = d ** -0.5
    module = types.SimpleNamespace(layer_idx=0, scaling=scaling)
    seen = []
    original = ev._maybe_cuda_final_attention

    def record(query_states, key_states, value_states, attention_mask, final_indices, final_valid, scaling_):
        seen.append((final_indices.clone(), final_valid.clone()))
        return original(query_states, key_states, value_states, attention_mask, final_indices, final_valid, scaling_)

    ev._maybe_cuda_final_attention = record
    brep_state = ev.BlockRepState() if mode.startswith("brep") else None
    periodic = re.fullmatch(r"qabs\d+cand\d+(?:p\d+)?r\d+attn", mode) is not None
    reuse_state = ev.ReuseCandidateState() if periodic else None
    outs, finals = [], []
    try:
        # qabs{S}cand{pct}attn runs its candidate path only with the fast-path
        # flag (EV:6436-6449), as the reference's timed runs set it
        with ev.attention_mode(mode=mode, top_fraction=top_fraction, max_heads_per_token=3,
                               always_keep_self=keep_self, protect_sink_tokens=sink,
                               protect_recent_tokens=recent, load_stats=None, brep_state=brep_state,
                               reuse_state=reuse_state, qabs_fast_path=mode.startswith("qabs")):
            for s in range(steps):
                n = t0 + s + 1
                seen.clear()
                out, _ = ev._limited_eager_attention_forward(module, q[s], k[:, :, :n], v[:, :, :n], None,
                                                             scaling=scaling)
                idx, val = seen[-1]
                keep = np.zeros((1, hq, t_max), dtype=bool)
                for h in range(hq):
                    keep[0, h, idx[0, h][val[0, h]].numpy()] = True
                outs.append(out.float().numpy())
                finals.append(keep)
    finally:
        ev._maybe_cuda_final_attention = original
    np.savez_compressed(
        OUT / f"block_{name}.npz", mode=np.array(mode), dtype=np.array(str(dtype).split(".")[-1]),
        q=q.float().numpy(), k_bf16=k.to(torch.bfloat16).view(torch.int16).numpy(),
        v_bf16=v.to(torch.bfloat16).view(torch.int16).numpy(), t0=t0, steps=steps,
        top_fraction=top_fraction, sink=sink, recent=recent, keep_self=keep_self, scaling=scaling,
        out=np.stack(outs), final=np.packbits(np.stack(finals), axis=-1), t_max=t_max)
    print(f"{name}: {mode} {dtype} Hq={hq} T0={t0} steps={steps} -> block_{name}.npz")


def main(names):
    """Writes the named scenarios (every scenario when none is named)."""
    sys.path.insert(0, str(REF_SRC))
    import evaluate_qwen3_top2_head_limit3_ppl as ev   # the reference module, CPU only

    torch.set_num_threads(1)
    for name, args in SCENARIOS.items():
        if not names or name in names:
            run(ev, name, *args)
    for name, args in LAG_SCENARIOS.items():
        if not names or name in names:
            run(ev, name, *args, lagged=True)
    for name, args in BLOCK_SCENARIOS.items():
        if not names or name in names:
            run_block(ev, name, *args)


if __name__ == "__main__":
    main(set(sys.argv[1:]))
