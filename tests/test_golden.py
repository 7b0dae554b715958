"""The committed config-1 fixture (tests/golden/c1_decode.json) is reproduced
by this tree: the seed-0 weight generator matches the recorded SHA-256 of every
tensor, and the oracle's decode step at position 128 matches the recorded K/V
rows, hidden state and logits (fp32 summation order may differ between hosts
and thread counts, hence the small tolerances)."""

import json
from pathlib import Path

import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "c1_decode.json"


def test_golden_fixture_reproduces():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN.with_name("make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    g = json.loads(GOLDEN.read_text())
    res, sd, _ = mg.compute()
    assert res["token_ids"] == g["token_ids"]
    for k, v in g["weight_fingerprint"].items():
        assert res["weight_fingerprint"][k]["sha256"] == v["sha256"], k
    assert res["argmax"] == g["argmax"]
    assert max(abs(a - b) for a, b in zip(res["top32_logits"], g["top32_logits"])) < 1e-3
    for l in g["kv_rows"]:
        for kind in ("k", "v"):
            a = torch.tensor(res["kv_rows"][l][kind])
            b = torch.tensor(g["kv_rows"][l][kind])
            assert (a != b).float().mean().item() < 0.02
    assert (torch.tensor(res["hidden_final"]) != torch.tensor(g["hidden_final"])).float().mean() < 0.05
