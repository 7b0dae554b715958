"""Writes tests/golden/c3_self_agreement.json — where two correct bf16
implementations of the decode step pick different greedy tokens.

The CPU oracle (``oracle.llama_ref.OracleLlama``, "mk" mode: bf16 rounding
points, fp32 accumulation) and the same oracle with fp64 accumulation (same
rounding points) run the config-3 sequence teacher-forced: seed-0 synthetic
Llama-3.2-1B weights, a 384-token prompt (``random_token_ids(384, seed=0)``)
followed by 639 more ids (``random_token_ids(639, seed=7)``), logits at the 640
positions 383..1022. Both are correct restatements of the reference's algorithm,
so every position where their argmaxes differ is a near-tie flip, not a bug.

Recorded per position: the fp64 variant's top-2 logit gap (the "baseline" gap a
validation run sees) and whether the two argmaxes agree. tests/test_validate_rule.py
checks main.py's validate pass rule against every window of these positions.
Run: ``python tests/golden/make_agreement.py`` (about 4 minutes on 8 cores).
"""

import json
import sys
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(REPO / "llama1b-megakernel_amd"), str(REPO), str(REPO / "tests")]

from mk_weights import random_token_ids, synthetic_state_dict  # noqa: E402
from oracle.llama_ref import OracleLlama  # noqa: E402
from noise_variants import FP64Accumulate as _FP64Accumulate  # noqa: E402

OUT = Path(__file__).resolve().with_name("c3_self_agreement.json")


def main():
    torch.set_num_threads(8)
    sd = synthetic_state_dict(seed=0)
    seq = torch.cat([random_token_ids(384, seed=0), random_token_ids(639, seed=7)])
    o = OracleLlama(sd, mode="mk")
    a = o.logits(o.forward(seq, 0, o.new_cache(1024), want_logits=False)[1][383:]).double()
    del o
    o64 = _FP64Accumulate(sd)
    b = o64.logits(o64.forward(seq, 0, o64.new_cache(1024), want_logits=False)[1][383:])
    same = (a.argmax(-1) == b.argmax(-1)).tolist()
    top2 = b.topk(2, -1).values
    gap = (top2[:, 0] - top2[:, 1]).tolist()
    OUT.write_text(json.dumps({
        "what": "oracle (fp32 accumulation) vs the oracle with fp64 accumulation, teacher-forced, "
                "config-3 positions 383..1022",
        "weights": "synthetic_state_dict(seed=0)", "prompt": "random_token_ids(384, seed=0)",
        "continuation": "random_token_ids(639, seed=7)",
        "top2_gap": [round(g, 6) for g in gap], "agree": [bool(s) for s in same]}, indent=0))
    print(f"wrote {OUT}: {sum(same)}/{len(same)} positions agree")


if __name__ == "__main__":
    main()
