"""Writes tests/golden/c1_decode.json — the BASELINE config-1 fixture.

Config 1: Llama-3.2-1B, seed-0 synthetic weights (N(0,0.02) bf16 matrices,
unit gammas; ``mk_weights.synthetic_state_dict``), 129 uniform-random token ids
(``mk_weights.random_token_ids(129, seed=0)``): the first 128 are prefilled into
a 1024-row cache, the 129th is decoded at position 128. Computed with the CPU
oracle (``oracle.llama_ref.OracleLlama``, "mk" mode).

Recorded: the token ids; SHA-256 and first 16 values of every weight tensor;
the K and V rows written at position 128 for layers 0, 7, 15; the hidden state
after the last layer; the top-32 logits with indices, the logits' sum and L2
norm; the argmax. Run: ``python tests/golden/make_golden.py``.
"""

import json
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(REPO / "llama1b-megakernel_amd"), str(REPO)]

from mk_weights import random_token_ids, state_dict_fingerprint, synthetic_state_dict  # noqa: E402
from oracle.llama_ref import OracleLlama  # noqa: E402

OUT = Path(__file__).resolve().with_name("c1_decode.json")
LAYERS = (0, 7, 15)


def bf16_bits(t: torch.Tensor):
    return [int(v) & 0xFFFF for v in t.to(torch.bfloat16).contiguous().view(torch.int16).flatten().tolist()]


def compute():
    t0 = time.time()
    sd = synthetic_state_dict(seed=0)
    ids = random_token_ids(129, seed=0)
    fp = state_dict_fingerprint(sd)
    o = OracleLlama(sd, mode="mk")
    cache = o.new_cache(1024)
    o.forward(ids[:128], 0, cache, want_logits=False)
    logits, hidden = o.forward(ids[128:], 128, cache)
    logits = logits[0]
    top = torch.topk(logits, 32)
    res = {
        "description": __doc__.strip().splitlines()[0],
        "seed": 0, "weights": "N(0,0.02) bf16 matrices from one CPU generator per parameter "
                              "(mk_weights._param_seed), unit RMSNorm gammas",
        "token_ids": ids.tolist(),
        "decode_pos": 128,
        "weight_fingerprint": fp,
        "kv_rows": {str(l): {"k": bf16_bits(cache[l][0][:, 128]), "v": bf16_bits(cache[l][1][:, 128])}
                    for l in LAYERS},
        "hidden_final": bf16_bits(hidden[0]),
        "top32_logits": [float(v) for v in top.values],
        "top32_ids": [int(i) for i in top.indices],
        "logits_sum": float(logits.double().sum()),
        "logits_l2": float(logits.double().norm()),
        "argmax": int(logits.argmax()),
        "seconds": round(time.time() - t0, 1),
    }
    return res, sd, o


if __name__ == "__main__":
    res, _, _ = compute()
    OUT.write_text(json.dumps(res))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes) in {res['seconds']} s; argmax {res['argmax']}")
