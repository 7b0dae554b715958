"""The algorithmic-byte counts that every roofline figure divides by.

`mk_config.step_bytes` is checked against the stated per-step formula of the
benchmark's metric,
    1,946,157,056 + 525,336,576 + 135,168 + sum_b(32,768*T_b + 32,768 + 4,096 + 513,024) B
(layer weights, tied lm_head, RMSNorm gammas; per sequence: K/V rows read, the
K/V row written, the embedding row, fp32 logits), term by term from the model
dimensions, and against its worked value at T = 1024 (2,505,733,120 B). One
difference is deliberate: the kernels fold the 32 per-layer RMSNorm gammas
into the weights at load (`mk_weights.fold_gamma`), so a step reads only the
final norm's gamma (4,096 B) where the formula counts all 33 (135,168 B).
`bench.py --gpus N` with N > 1 must refuse to run.
"""

import subprocess
import sys

from conftest import REPO

from mk_config import LLAMA_3_2_1B, layer_weight_bytes, step_bytes

LAYERS_W = 1_946_157_056
LM_HEAD = 525_336_576
GAMMAS_ALL = 135_168
PER_ROW_KV = 32_768
PER_SEQ = 32_768 + 4_096 + 513_024
GAMMA_FINAL = 4_096


def baseline_formula(ts):
    return LAYERS_W + LM_HEAD + GAMMAS_ALL + sum(PER_ROW_KV * t + PER_SEQ for t in ts)


def test_formula_terms_follow_from_the_model_dimensions():
    d = LLAMA_3_2_1B
    assert 16 * layer_weight_bytes(d) == LAYERS_W
    assert d.vocab * d.hidden * 2 == LM_HEAD
    assert (2 * d.n_layers + 1) * d.hidden * 2 == GAMMAS_ALL
    assert d.n_layers * 2 * d.n_kv_heads * d.head_dim * 2 == PER_ROW_KV
    assert d.vocab * 4 + d.hidden * 2 + PER_ROW_KV == PER_SEQ


def test_bs1_step_matches_the_baseline_formula():
    assert baseline_formula([1024]) == 2_505_733_120
    for t in (0, 1, 383, 700, 1023, 1024, 4095):
        assert step_bytes(16, [t], True) == baseline_formula([t]) - GAMMAS_ALL + GAMMA_FINAL


def test_batched_step_sums_per_sequence_terms():
    ts = [538, 3178, 1486, 995, 2689, 2093, 2228, 2430]
    assert step_bytes(16, ts, True) == baseline_formula(ts) - GAMMAS_ALL + GAMMA_FINAL
    # no lm_head: no logits, no vocabulary read, no final gamma
    assert step_bytes(16, ts, False) == LAYERS_W + sum(PER_ROW_KV * t + PER_ROW_KV + 4_096 for t in ts)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr
