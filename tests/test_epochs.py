"""Exchange epochs across requests (CPU only: the host rule, no device).

bf16 vector exchanges carry a 16-bit tag of the epoch (epoch mod 65535 + 1), so a poll cannot
tell a stale word from a fresh one when their epochs differ by a multiple of 65535.  The
runtime keeps every polled word at most one launch older than the epoch a reader waits for.
After a generation that stopped at EOS, the launches after the stop returned at once, and
ti_epoch_after_generation moves the epoch back to follow the last launch that ran (the stop
the reference resolves in tileinfer/src/runtime/sequence_context.cu:84-99).

The simulation below replays request sequences at the granularity of exchange phases and checks
every poll of a tagged vector against the previous contents of the word it reads.  The same
simulation with the epoch left where the skipped launches took it finds collisions, which shows
that the check can fail.
"""

import ctypes as C
import random

import pytest

from tiles_amd import runtime as R

STEPS = 64          # TI_MAX_LAUNCH_STEPS
PHASES = 8          # kPhases (worker_config.hpp)
ATTN, RES, Y = 1, 2, 4  # kPhaseAttn, kPhaseR, kPhaseY


def tag(epoch: int) -> int:
    return epoch % 65535 + 1


def span(layers: int) -> int:
    return STEPS * PHASES * (layers + 1)


def after_generation(lib, current, epochs, generated, layers):
    array = (C.c_uint32 * len(epochs))(*epochs)
    return lib.ti_epoch_after_generation(current, array, len(epochs), generated, layers)


def test_epoch_rule_cases():
    lib = R.library()
    s = span(16)
    assert lib.ti_epochs_per_launch(16) == s
    epochs = [1, 1 + s, 1 + 2 * s, 1 + 3 * s]
    # every launch ran
    assert after_generation(lib, 1 + 4 * s, epochs, 256, 16) == 1 + 4 * s
    # EOS at the 10th token: only the first launch ran
    assert after_generation(lib, 1 + 4 * s, epochs, 10, 16) == 1 + s
    # EOS at token 64 (the last of launch 0) and at token 65 (launch 1)
    assert after_generation(lib, 1 + 4 * s, epochs, 64, 16) == 1 + s
    assert after_generation(lib, 1 + 4 * s, epochs, 65, 16) == 1 + 2 * s
    # the epoch wrapped after the stop: the wrap cleared the polled words, the epoch stands
    wrapped = [epochs[0], epochs[1], 1, 1 + s]
    assert after_generation(lib, 1 + 2 * s, wrapped, 10, 16) == 1 + 2 * s
    # one launch: nothing to skip
    assert after_generation(lib, 1 + s, [1], 3, 16) == 1 + s


def simulate(lib, layers, requests, settle=True):
    """Replays requests; returns the polls that would accept a stale word."""
    s = span(layers)
    epoch = 1
    writes = {}  # tagged vector -> epochs of its last two writes
    bad = []

    def write(name, at):
        writes[name] = (writes.get(name, (None, None))[1], at)

    def poll(name, want):
        # The write the poll waits for comes first in program order; the poll may still see the
        # word's contents from before it (zero, tag 0, before the first write).
        old, new = writes[name]
        assert new == want
        if old is not None and tag(old) == tag(want):
            bad.append((name, old, want))

    def run_launch(base, steps):
        for step in range(steps):
            for layer in range(layers):
                at = base + step * PHASES * (layers + 1) + layer * PHASES + 1
                if layer > 0:
                    poll(f"hidden{layer % 2}", at - PHASES + Y)  # written by the previous layer
                write("attn", at + ATTN)
                poll("attn", at + ATTN)
                write("r", at + RES)
                poll("r", at + RES)
                write(f"hidden{(layer + 1) % 2}", at + Y)

    for kind, count, stop in requests:
        if kind == "prefill":
            for first in range(0, count, STEPS):
                run_launch(epoch, min(STEPS, count - first))
                epoch += s
        else:  # generate `count` tokens; the `stop`-th is EOS (step s selects token first + s)
            epochs = []
            for first in range(0, count, STEPS):
                epochs.append(epoch)
                if first < stop:  # the stopping launch ends after that step; later ones return at once
                    run_launch(epoch, min(STEPS, count - first, stop - first))
                epoch += s
            if settle:
                epoch = after_generation(lib, epoch, epochs, stop, layers)
    return bad


@pytest.mark.parametrize("layers", [1, 3, 16, 22, 28, 32, 40, 80, 120])
def test_no_stale_tag_matches_across_requests(layers):
    lib = R.library()
    rng = random.Random(layers)
    requests = [("prefill", rng.randint(1, 200), None)]
    for _ in range(12):
        count = rng.randint(1, 64 * 40)
        requests.append(("generate", count, rng.randint(1, count)))
        if rng.random() < 0.3:
            requests.append(("prefill", rng.randint(1, 70), None))
    assert simulate(lib, layers, requests) == []


def test_simulation_detects_unsettled_epochs():
    """Without the rule, a generation that stops early leaves words hundreds of launches old and
    their tags collide for some layer counts: with 80 layers, a stop in the first of 177 launches
    (11,328 requested tokens) makes the next request's first attention poll accept a stale word."""
    lib = R.library()
    layers = 80
    hits = 0
    for launches in range(170, 185):
        requests = [("prefill", 1, None), ("generate", 64 * launches, 1), ("prefill", 64, None)]
        assert simulate(lib, layers, requests, settle=True) == []
        hits += bool(simulate(lib, layers, requests, settle=False))
    assert hits > 0
