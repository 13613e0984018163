"""Copy-to-copy ordering of the SDMA link, and the engine's deferred host work, on the host.

The SDMA link may run two copies of one direction on different DMA engines (or as halves split
across two engines), so a copy into a slot must name the earlier copies through the slot's
gate that it waits for. ``mo::GateOrder`` (``csrc/mo_gate_order.h``) holds that rule, and
``SdmaLink`` takes every copy's dependency from it. This test compiles a small C++ driver
against the same header with g++ and runs it.

``mo::DeferredHost`` (``csrc/mo_deferred.h``) holds the engine's host ranges that copies may
still touch and the coded byte counts read from them: copies finish out of order, and a count
must never read a range that went back to the pool. ``native/deferred_test.cpp`` drives it
with fake copies finishing in every order, including between its two loops.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "moss-image_amd" / "csrc"
NATIVE = Path(__file__).resolve().parent / "native"


def _run_driver(tmp_path, name: str) -> None:
    exe = tmp_path / name
    subprocess.run(
        ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{CSRC}", str(NATIVE / f"{name}.cpp"), "-o", str(exe)],
        check=True,
        capture_output=True,
    )
    run = subprocess.run([str(exe)], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip() == "ok"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_gate_order_rules(tmp_path):
    _run_driver(tmp_path, "gate_order_test")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_deferred_host_counts_never_read_freed_ranges(tmp_path):
    _run_driver(tmp_path, "deferred_test")
