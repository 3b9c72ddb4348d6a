"""Statistics and telemetry parsing of the controlled timing protocol (tiles_amd/controlled.py),
on the CPU: the paired bootstrap recovers a known shift, the restart in reverse spawn order
separates a placement effect from a real difference, and amd-smi JSON flattens to numeric
leaves keyed by path."""

import numpy as np

from tiles_amd import controlled as C


def test_paired_bootstrap_recovers_a_constant_shift():
    reference = [640.0, 641.5, 639.8, 640.7, 641.1, 640.2]
    p = C.paired(reference, [r + 2.5 for r in reference], seed=1)
    assert abs(p["mean_us"] - 2.5) < 1e-9 and p["ci95_us"] == [2.5, 2.5] and p["pairs"] == 6
    assert abs(p["mean_percent"] - 100 * 2.5 / np.mean(reference)) < 1e-9


def test_paired_bootstrap_interval_covers_zero_for_noise():
    rng = np.random.default_rng(3)
    reference = list(640 + rng.normal(0, 0.5, 12))
    other = list(np.asarray(reference) + rng.normal(0, 0.5, 12))
    p = C.paired(reference, other, seed=2)
    assert p["ci95_us"][0] < 0 < p["ci95_us"][1]


def test_amd_smi_records_flatten_to_numeric_leaves():
    record = {"gpu": 0, "power": {"socket_power": {"value": 312, "unit": "W"}},
              "clock": {"gfx_0": {"clk": {"value": 2100, "unit": "MHz"}, "max_clk": {"value": 2400, "unit": "MHz"}}},
              "temperature": {"hotspot": {"value": 55, "unit": "C"}, "mem": "N/A"}}
    flat = C.flatten(record)
    assert flat == {"gpu": 0.0, "power.socket_power": 312.0, "clock.gfx_0.clk": 2100.0, "clock.gfx_0.max_clk": 2400.0,
                    "temperature.hotspot": 55.0}


def test_spawn_order_effect_is_separated_from_the_difference():
    """Arm B is 1.0 us slower than A; the first-started server runs 0.6 us faster, A started first
    in blocks 0-2 and B in blocks 3-5.  The paired mean over both halves is the real 1.0 us, and
    half the halves' difference is the 0.6 us placement effect."""
    base = [640.0, 640.4, 639.8, 640.2, 640.1, 639.9]
    a = [t - (0.6 if k < 3 else 0.0) for k, t in enumerate(base)]
    b = [t + 1.0 - (0.0 if k < 3 else 0.6) for k, t in enumerate(base)]
    assert abs(C.paired(a, b, seed=4)["mean_us"] - 1.0) < 1e-9
    effect = C.spawn_order_effect(a, b, 3)
    assert abs(effect["first_half_mean_us"] - 1.6) < 1e-9 and abs(effect["second_half_mean_us"] - 0.4) < 1e-9
    assert abs(effect["spawn_order_effect_us"] - 0.6) < 1e-9


def test_outlier_exclusion_never_empties_a_block():
    """Rounds further than OUTLIER_FRACTION from the arm's median are dropped, but a block with no
    round inside keeps them all: its median stays finite, and so does the paired comparison (a tiny
    package at 45 us/token put a whole 2-round block outside a 1% band)."""
    blocks = [[100.0, 100.2], [103.0, 104.0], [99.9, 150.0]]
    kept = C.kept_rounds(blocks, 100.0)
    assert kept == [[100.0, 100.2], [103.0, 104.0], [99.9]]
    medians = [float(np.median(k)) for k in kept]
    result = C.paired(medians, [m + 1.0 for m in medians], seed=0)
    assert np.isfinite(result["mean_us"]) and all(np.isfinite(result["ci95_us"]))
