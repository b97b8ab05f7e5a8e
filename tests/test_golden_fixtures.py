"""The committed fixtures under tests/golden/ (written by tests/golden/make_fixtures.py).

They must be exactly what the script produces (data and generator agree), and the oracle's
paged attention, the reference's tiled recurrence restated, must reproduce their float64
closed-form expectations to the north star's 1e-5 for every case.
"""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest

from oracle.attention import paged_attention

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name: str):
    with np.load(GOLDEN / name) as data:  # allow_pickle stays False
        return {key: data[key] for key in data.files}


def _generator():
    spec = importlib.util.spec_from_file_location("make_fixtures", GOLDEN / "make_fixtures.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


@pytest.mark.parametrize(("name", "builder"), [("attention_cases.npz", "attention_cases"), ("rope_cases.npz", "rope_cases")])
def test_fixtures_are_what_the_generator_writes(name, builder) -> None:
    stored = _load(name)
    fresh = getattr(_generator(), builder)()
    assert set(stored) == set(fresh)
    for key in stored:
        assert np.array_equal(stored[key], fresh[key]), key


def test_the_oracle_meets_the_closed_form_on_every_case() -> None:
    data = _load("attention_cases.npz")
    for i in range(int(data["count"])):
        case = {k[len(f"c{i}_"):]: v for k, v in data.items() if k.startswith(f"c{i}_")}
        got = np.zeros_like(case["queries"])
        for s, ctx in enumerate(case["contexts"].tolist()):
            rows = np.flatnonzero(case["seq"] == s)
            table = case["tables"][s, : -(-ctx // case["keys"].shape[1])]
            got[rows] = paged_attention(case["queries"][rows], case["positions"][rows], case["keys"],
                                        case["values"], table, ctx, float(case["scale"]))  # fmt: skip
        assert np.max(np.abs(got - case["expected"])) < 1e-5, i


def test_the_oracle_rotation_equals_the_elementwise_fixture() -> None:
    """The RoPE expectations are evaluated one element at a time in float32 scalars (not by the
    oracle); the vectorised oracle must give the same bits."""
    from oracle.model import apply_rope

    data = _load("rope_cases.npz")
    for i in range(int(data["count"])):
        case = {k[len(f"r{i}_"):]: v for k, v in data.items() if k.startswith(f"r{i}_")}
        for which, index in (("q", 0), ("k", 1)):
            got = apply_rope(case["fused"][:, index], case["positions"], case["cos"], case["sin"])
            assert np.array_equal(got, case[which]), (i, which)
