"""The stack's capacity rule (host arithmetic in the library, no GPU) and the benchmark's plan of
stack calls checked against it: every call that launches steps must fit the rows of input and the
token slots the stack was bound with, so a plan that would read past an input buffer is refused on
the host before anything runs on the device."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_capacity_rule(lib):
    L = lib.load()
    cap = L.ds_hip_stack_capacity_for
    assert cap(25, 1280, 25, -1) == 25
    assert cap(25, 1280, 45, -1) == 25          # rows read per step limit it
    assert cap(1, 0, 45, -1) == 45              # stride 0: one row serves every step
    assert cap(100, 1280, 30, -1) == 30         # token slots limit it
    assert cap(100, 1280, 100, 41) == 41        # KV positions left limit it
    assert cap(100, 1280, 100, 0) == 0
    for bad in [(0, 1280, 10, -1), (10, 1280, 0, -1), (10, -1, 10, -1)]:
        assert cap(*bad) == -1
    fit = L.ds_hip_steps_fit
    assert fit(25, 0, 25) and fit(25, 5, 20) and fit(25, 25, 0)
    assert not fit(25, 5, 21) and not fit(25, 26, 0) and not fit(25, 0, -1) and not fit(-1, 0, 0)
    assert not fit(2**31 - 1, 2**31 - 1, 2**31 - 1)  # no overflow in the sum


@pytest.mark.parametrize("steps,warmup", [(20, 5), (226, 20), (1, 0), (500, 50), (5, 300)])
def test_bench_plan_fits_its_buffers(lib, steps, warmup):
    b = load_bench()
    L = lib.load()
    rows, phases = b.bench_plan(steps, warmup, 200, 100, 20)
    assert rows >= warmup + steps and rows >= 200
    assert b.check_plan(L, rows, 1280, rows, -1, phases) == rows
    # whole decoder steps (attention): the KV positions of the cache bound the same plan
    assert b.check_plan(L, rows, 1280, rows, rows + 1, phases) == rows
    with pytest.raises(ValueError):
        b.check_plan(L, rows, 1280, rows, rows - 1, phases)


def test_decoder_leg_has_its_own_rows(lib):
    """The driver's command (--steps 20 --warmup 5) once bound the 45-step decoder leg to the main
    leg's 25 input rows; that plan must be refused, and the decoder leg's own plan must fit."""
    b = load_bench()
    L = lib.load()
    dec_rows, dec_phases = b.decoder_plan(5, 40)
    assert dec_rows == 45
    assert b.check_plan(L, dec_rows, 1280, dec_rows, dec_rows + 1, dec_phases) == 45
    main_rows = 5 + 20
    with pytest.raises(ValueError):
        b.check_plan(L, main_rows, 1280, main_rows, dec_rows + 1, dec_phases)
