"""CPU checks of main.py's validate pass rule (no GPU calls)."""


def test_overall_floor_is_90_percent_for_long_runs():
    from main import overall_agreement_floor
    assert overall_agreement_floor(640) == 0.90
    assert overall_agreement_floor(10_000) == 0.90


def test_overall_floor_loosens_with_fewer_positions():
    from main import AGREEMENT_NOISE_FLOOR, overall_agreement_floor
    floors = [overall_agreement_floor(n) for n in (8, 48, 128, 256, 640)]
    assert floors == sorted(floors)
    # three binomial standard deviations below the measured noise floor
    p = AGREEMENT_NOISE_FLOOR
    assert abs(overall_agreement_floor(48) - (p - 3 * (p * (1 - p) / 48) ** 0.5)) < 1e-12
    assert 0.82 < overall_agreement_floor(48) < 0.83


# ---------------------------------------------------------------------------
# the reference's tol_map / divergence rules, restated (mk_validate)
# ---------------------------------------------------------------------------

def _logits(seed=0, T=3, V=2000):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(T, V, generator=g, dtype=torch.float64)


def test_tol_map_is_the_references():
    from mk_validate import REFERENCE_DIVERGENCE_TOL, REFERENCE_TOL_MAP
    # main.py:542 and main.py:51
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
