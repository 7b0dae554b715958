"""CPU checks of main.py's validate pass rule (no GPU calls)."""


import json
from pathlib import Path

FIXTURE = Path(__file__).resolve().parent / "golden" / "c3_self_agreement.json"


def _fixture():
    d = json.loads(FIXTURE.read_text())
    assert len(d["agree"]) == len(d["top2_gap"]) == 640
    return d["agree"], d["top2_gap"]


def test_rule_passes_every_window_of_two_correct_implementations():
    """The oracle against its own fp64-accumulation variant (both correct):
    validate_pass holds on every window of >= 24 consecutive positions."""
    from main import validate_pass
    agree, gaps = _fixture()
    assert 590 <= sum(agree) <= 600            # ~93%: near-tie flips of random-init logits
    for n in (24, 48, 96, 640):
        for i in range(0, 640 - n + 1):
            ok, st = validate_pass(agree[i:i + n], gaps[i:i + n])
            assert ok, (n, i, st)


def test_flips_are_near_ties_and_cluster():
    """Why the rule excludes near-ties instead of flooring the agreement over
    all positions: every flip has a top-2 gap < 0.1, and an all-positions floor
    three binomial deviations under the mean still fails many 48-position
    windows of two correct implementations."""
    agree, gaps = _fixture()
    assert all(g < 0.1 for a, g in zip(agree, gaps) if not a)
    p, n = 0.931, 48
    floor = p - 3 * (p * (1 - p) / n) ** 0.5
    fails = sum(sum(agree[i:i + n]) / n < floor for i in range(0, 640 - n + 1))
    assert fails >= 10


def test_rule_fails_a_planted_mistake():
    """A kernel whose greedy token differs at decided positions, or whose
    agreement outside the near-tie band drops, or whose logits move beyond the
    bounds, fails."""
    from main import validate_pass
    agree, gaps = _fixture()
    dec = [i for i, g in enumerate(gaps) if g >= 0.1]
    bad = list(agree)
    bad[dec[0]] = False                        # one decided flip in a short window
    assert not validate_pass(bad[:dec[0] + 24], gaps[:dec[0] + 24])[0]
    bad = list(agree)
    for i in dec[::40]:                        # 2.5% of the decided positions over the whole run
        bad[i] = False
    assert not validate_pass(bad, gaps)[0]
    # every 5th clear position wrong: 80% outside the near-tie band
    worse = [a and not (k % 5 == 0 and g >= 0.03) for k, (a, g) in enumerate(zip(agree, gaps))]
    assert not validate_pass(worse, gaps)[0]
    assert not validate_pass(agree, gaps, worst_max_abs=0.25)[0]
    assert not validate_pass(agree, gaps, worst_rms=0.04)[0]
    assert validate_pass(agree, gaps, worst_max_abs=0.15, worst_rms=0.025)[0]


# ---------------------------------------------------------------------------
# the reference's tol_map / divergence rules, restated (mk_validate)
# ---------------------------------------------------------------------------

def _logits(seed=0, T=3, V=2000):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(T, V, generator=g, dtype=torch.float64)


def test_tol_map_is_the_references():
    from mk_validate import REFERENCE_DIVERGENCE_TOL, REFERENCE_TOL_MAP
    # main.py:544 and main.py:51
    assert REFERENCE_TOL_MAP == {None: (1e-5, 0.05), 1000: (1e-5, 0.03), 50: (1e-5, 0.03), 5: (1e-5, 0.03)}
    assert REFERENCE_DIVERGENCE_TOL == 0.001


def test_topk_tolerance_identical_and_boundary():
    from mk_validate import topk_tolerance
    e = _logits()
    r = topk_tolerance(e.clone(), e)
    assert all(v["steps_passing"] == 1.0 and v["worst_ratio"] == 0.0 for v in r.values())
    # every entry moved by exactly its bound (atol + rtol |e|) passes; by 1.01x the bound it fails
    tol = {None: (1e-5, 0.05)}
    bound = 1e-5 + 0.05 * e.abs()
    assert topk_tolerance(e + 0.999 * bound, e, tol)["all"]["steps_passing"] == 1.0
    assert topk_tolerance(e + 1.01 * bound, e, tol)["all"]["steps_passing"] == 0.0


def test_topk_tolerance_uses_the_expected_top_k():
    import torch
    from mk_validate import topk_tolerance
    e = _logits(1)
    a = e.clone()
    # spoil every entry outside the expected top-50 of step 0 by a lot: top-5 and top-50 still
    # pass, top-1000 and "all" fail for that step only
    keep = e[0].topk(50).indices
    mask = torch.ones(e.shape[1], dtype=torch.bool)
    mask[keep] = False
    a[0, mask] += 10.0
    r = topk_tolerance(a, e)
    assert r["top5"]["steps_passing"] == 1.0 and r["top50"]["steps_passing"] == 1.0
    assert abs(r["top1000"]["steps_passing"] - 2 / 3) < 1e-12
    assert abs(r["all"]["steps_passing"] - 2 / 3) < 1e-12
    # a mistake at the expected argmax fails every k
    b = e.clone()
    b[2, e[2].argmax()] -= 1.0
    r = topk_tolerance(b, e)
    assert all(abs(v["steps_passing"] - 2 / 3) < 1e-12 for v in r.values())


def test_divergences_counts_ties_within_tolerance():
    import torch
    from mk_validate import divergences
    e = torch.zeros(3, 10, dtype=torch.float64)
    e[:, 4] = 1.0
    e[0, 7] = 1.0 - 0.0005     # a near tie at step 0
    e[2, 1] = 0.5              # a clear winner at step 2
    a = e.clone()
    a[0, 7] += 0.01            # step 0 picks 7: divergence within tolerance
    a[2, 1] += 1.0             # step 2 picks 1: divergence by 0.5
    d = divergences(a, e)
    assert d["steps"] == 2 and d["within_tol"] == 1 and d["first"] == 0
    assert abs(d["largest_expected_gap"] - 0.5) < 1e-12
    assert divergences(e, e) == {"steps": 0, "within_tol": 0, "first": None, "largest_expected_gap": 0.0}
