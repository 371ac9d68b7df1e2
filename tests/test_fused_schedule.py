"""CPU check of the fused decode kernel's static schedule.

uocr_hip_fused_schedule_check replays, on the host, the wait/publish program
that every workgroup of decode_fused.hip runs, using the same FusedSchedule
code the kernel compiles (csrc/fused_schedule.hpp). It fails if any workgroup
is left waiting (a cycle, or a wait for a step its owner never publishes), if
an item is published by another workgroup or at another step than the
schedule's owner/step formulas say, or if the slot mapping is not a bijection.
No device work: this runs without a GPU.
"""
import ctypes as C

import numpy as np
import pytest

from uocr_hip import _lib

RBG, RBD = 14, 10  # inter 896 in 64-row gate/up items, hidden 1280 in 128-row down items


def check(seq, grid, n_groups, live):
    lib = _lib.load()
    arr = (C.c_int * max(1, len(live)))(*live)
    rc = lib.uocr_hip_fused_schedule_check(seq, grid, n_groups, RBG, RBD, arr, len(live))
    return rc, lib.uocr_hip_last_error().decode()


def live_groups(rng, n_experts, n_virtual, p):
    """Live routed groups ascending, then the shared groups (the kernel's order)."""
    routed = [e for e in range(n_experts) if rng.random() < p]
    return routed + [n_experts + v for v in range(n_virtual)]


@pytest.mark.parametrize("seq", [12, 14, 16])
@pytest.mark.parametrize("grid", [18, 64, 257, 496, 512, 768, 1024])
def test_schedule_completes(seq, grid):
    if grid <= seq + 1:
        pytest.skip("the launcher refuses grid <= seq + 1")
    rng = np.random.default_rng(seq * 7919 + grid)
    for p in (0.0, 0.3, 0.8, 1.0):
        live = live_groups(rng, 64, 2, p)
        rc, err = check(seq, grid, 66, live)
        assert rc == 0, (seq, grid, p, err)


def test_schedule_without_shared_groups():
    rng = np.random.default_rng(5)
    live = live_groups(rng, 64, 0, 0.5) or [0]
    rc, err = check(16, 512, 64, live)
    assert rc == 0, err


def test_checker_detects_unreachable_wait():
    # a live "group" past the last one makes its down items wait for gate/up
    # items nobody publishes: the replay must report a workgroup left waiting
    rc, err = check(16, 512, 66, [0, 1, 70])
    assert rc != 0 and "left waiting" in err


def test_checker_rejects_bad_shape():
    rc, _ = check(16, 17, 66, [0])
    assert rc != 0
