"""The device-side cache-free recompute (paged_kv_serving_amd.equivalence.dense_logits), run by
torch on the CPU here, against the oracle's reference_forward, which the recorded reference
logits pin (tests/test_host_replay.py)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle.model import OracleModel
from paged_kv_serving_amd.equivalence import dense_logits, split_sizes
from paged_kv_serving_amd.replay import Trace

TRACES = Path(__file__).resolve().parent / "golden" / "traces"


@pytest.mark.parametrize("name", ["config1", "sharing_b16"])
def test_dense_logits_match_the_oracle_recompute(name) -> None:
    trace = Trace.load(TRACES / f"{name}.json")
    model = trace.language_model()
    oracle = OracleModel(model.config, model.weights)
    for seq_id in list(trace.tokens)[:3]:
        tokens = trace.tokens[seq_id]
        got = dense_logits(model, tokens, "cpu")
        want = oracle.reference_forward(tokens)
        assert got.shape == want.shape
        assert float(np.max(np.abs(got - want))) < 1e-5


def test_dense_logits_row_is_the_recorded_reference_row() -> None:
    """The last row the reference engine produced for a sequence is the dense pass's row at that
    context (to 1e-4): this ties the torch recompute to the reference's own numbers."""
    trace = Trace.load(TRACES / "config1.json")
    model = trace.language_model()
    seq_id = "req3#0"
    tokens = trace.tokens[seq_id]
    dense = dense_logits(model, tokens, "cpu")
    row, checked = 0, 0
    for it in trace.iterations:
        for seq, start, _, index, _ in it["entries"]:
            if index < 0:
                continue
            if seq == seq_id:
                assert float(np.max(np.abs(trace.logits[row] - dense[start + index]))) < 1e-4
                checked += 1
            row += 1
    assert checked == 32


def test_split_sizes() -> None:
    assert split_sizes(10, 4) == [4, 4, 2]
    assert split_sizes(8, 4) == [4, 4]
    with pytest.raises(ValueError):
        split_sizes(0, 4)
