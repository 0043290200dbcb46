"""Runs the CPU checks of the kernels' integer work schedules (tests/cpp/test_schedule.cpp):
the prefill grid mapping (pairing, XCD grouping, heaviest-first ranks) visits every
(sequence, head, query block) exactly once, and the decode split covers every tile once
with exact merge ranges and distinct partial slots. The header holding the schedules
(engine-mlx_amd/csrc/ema_schedule.hpp) is the one the kernels compile. Built twice: plain
and under -fsanitize=address,undefined. Also runs the CPU oracle under the same sanitizers
(tests/cpp/test_oracle_san.c: every exported function on exactly-sized buffers, with
identities between them)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CPP = os.path.join(HERE, "cpp")


@pytest.mark.parametrize("target", ["test_schedule", "test_schedule_san", "test_oracle_san"])
def test_work_schedules_cover_every_item_once(target):
    subprocess.run(["make", "-s", "-C", CPP, target], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(CPP, target)], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checks passed" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr
