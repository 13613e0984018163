"""The int8 GEMMs' launch plan (``mo_int8_launch_plan``, host only, no GPU): which rows take the
large tile, the small tile or a split reduction, checked against the rules stated in
``csrc/mo_gemm.cpp`` and against invariants every plan must keep (rows covered once and in
order, a split launch fitting one round, its reduction covered exactly)."""

from __future__ import annotations

import random

import pytest

from moss_offload import quant_kernels as qk

CUS = 256  # MI355X


def _tiles(n: int, edge: int = 256) -> int:
    return -(-n // edge)


@pytest.mark.parametrize("direction,cols,reduction,expect", [
    # config 5 at 17 792 rows (the packed tokens of one batch)
    ("qkvo forward", 3072, 3072, [("large", 0, 16384), ("split", 16384, 1408, 3, 18)]),
    ("up_gate forward", 24576, 3072, [("large", 0, 17664), ("small", 17664, 128)]),
    ("up_gate input gradient", 3072, 24576, [("large", 0, 16384), ("split", 16384, 1408, 3, 132)]),
    ("down forward", 3072, 12288, [("large", 0, 16384), ("split", 16384, 1408, 3, 66)]),
    ("down input gradient", 12288, 3072, [("large", 0, 17664), ("small", 17664, 128)]),
])
def test_config5_plans(direction, cols, reduction, expect) -> None:
    parts = qk.launch_plan(17792, cols, reduction, CUS)
    got = [(p["tile"], p["row0"], p["rows"]) + ((p["splits"], p["split_steps"]) if p["tile"] == "split" else ())
           for p in parts]
    assert got == expect, direction


def test_small_and_ragged_calls() -> None:
    # under one round: split when the rows fill three quarters of their large tiles and two
    # splits of at least 12 steps fit; small tile otherwise
    assert qk.launch_plan(1024, 3072, 3072, CUS) == [
        {"tile": "split", "row0": 0, "rows": 1024, "splits": 4, "split_steps": 12}]
    assert qk.launch_plan(128, 24576, 3072, CUS)[0]["tile"] == "small"      # half-empty large tiles
    assert qk.launch_plan(4096, 3072, 3072, CUS)[0]["tile"] == "small"      # 192 tiles: no room to split
    assert qk.launch_plan(1024, 3072, 1040, CUS)[0]["tile"] == "small"      # reduction not a multiple of 64
    assert qk.launch_plan(1024, 3072, 704, CUS)[0]["tile"] == "small"       # 11 steps: under two splits of 12
    # the LDS-decode kernel never splits
    assert [p["tile"] for p in qk.launch_plan(17792, 3072, 3072, CUS, kernel="lds")] == ["large", "small"]
    # a grid that fills its last round at least half: large tiles only
    assert qk.launch_plan(8192, 12288, 3072, CUS) == [
        {"tile": "large", "row0": 0, "rows": 8192, "splits": 1, "split_steps": 0}]


def test_every_plan_keeps_its_invariants() -> None:
    rng = random.Random(7)
    for _ in range(3000):
        rows = rng.choice([rng.randrange(1, 600), rng.randrange(1, 40000)])
        cols = 16 * rng.randrange(1, 2048)
        reduction = rng.choice([64 * rng.randrange(1, 500), 16 * rng.randrange(1, 2000)])
        cus = rng.choice([256, 304, 80, 120])
        parts = qk.launch_plan(rows, cols, reduction, cus)
        assert 1 <= len(parts) <= 2
        row = 0
        for i, p in enumerate(parts):
            assert p["row0"] == row and p["rows"] > 0
            row += p["rows"]
            if i == 0 and len(parts) == 2:
                assert p["tile"] == "large" and p["rows"] % 256 == 0
            if p["tile"] == "split":
                steps = reduction // 64
                assert reduction % 64 == 0 and p["splits"] >= 2 and p["split_steps"] >= 12
                assert (p["splits"] - 1) * p["split_steps"] < steps <= p["splits"] * p["split_steps"]
                tiles = _tiles(p["rows"]) * _tiles(cols)
                assert tiles * p["splits"] <= cus
                assert 4 * p["rows"] >= 3 * 256 * _tiles(p["rows"])
        assert row == rows
