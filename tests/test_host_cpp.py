"""Runs the C++ host-API tests (tests/cpp/test_host_api.cpp): the KvCache
trait contract, StaticCache and gqa_attention, in the shape of the reference's
crates/kvcache/tests and crates/attention/tests."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "test_host_api")


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)
    return BIN


def _run(mode):
    r = subprocess.run([_binary(), mode], capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_host_api_cpu():
    _run("cpu")


@pytest.mark.gpu
def test_host_api_gpu():
    _run("gpu")
