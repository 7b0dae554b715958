"""CPU checks of main.py's validate pass rule (no GPU calls)."""


def test_overall_floor_is_90_percent_for_long_runs():
    from main import overall_agreement_floor
    assert overall_agreement_floor(640) == 0.90
    assert overall_agreement_floor(10_000) == 0.90


def test_overall_floor_loosens_with_fewer_positions():
    from main import AGREEMENT_NOISE_FLOOR, overall_agreement_floor
    floors = [overall_agreement_floor(n) for n in (8, 48, 128, 256, 640)]
    assert floors == sorted(floors)
    # two binomial standard deviations below the measured noise floor
    p = AGREEMENT_NOISE_FLOOR
    assert abs(overall_agreement_floor(48) - (p - 2 * (p * (1 - p) / 48) ** 0.5)) < 1e-12
    assert 0.85 < overall_agreement_floor(48) < 0.86
