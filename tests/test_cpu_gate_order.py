"""Copy-to-copy ordering of the SDMA link, on the host.

The SDMA link may run two copies of one direction on different DMA engines (or as halves split
across two engines), so a copy into a slot must name the earlier copies through the slot's
gate that it waits for. ``mo::GateOrder`` (``csrc/mo_gate_order.h``) holds that rule, and
``SdmaLink`` takes every copy's dependency from it. This test compiles a small C++ driver
against the same header with g++ and runs it.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "moss-image_amd" / "csrc"
DRIVER = Path(__file__).resolve().parent / "native" / "gate_order_test.cpp"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_gate_order_rules(tmp_path):
    exe = tmp_path / "gate_order_test"
    subprocess.run(
        ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{CSRC}", str(DRIVER), "-o", str(exe)],
        check=True,
        capture_output=True,
    )
    run = subprocess.run([str(exe)], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip() == "ok"
