"""The batch types of the runner's interface (reference engine/runner.py:33-87), on the CPU."""

from __future__ import annotations

import pytest

from paged_kv_serving_amd.runner import BatchEntry


def test_batch_entry_and_execution_batch_keep_the_reference_interface() -> None:
    """BatchEntry and ExecutionBatch as the reference declares them (runner.py:33-87): frozen,
    slotted dataclasses with the same fields, defaults, validation messages and properties; they
    compare, hash, copy and pickle as such dataclasses do."""
    import copy
    import dataclasses
    import pickle

    from paged_kv_serving_amd.runner import ExecutionBatch

    assert [f.name for f in dataclasses.fields(BatchEntry)] == ["seq_id", "token_ids", "positions", "block_table",
                                                             "logits_index"]  # fmt: skip
    assert BatchEntry.__slots__ == ("seq_id", "token_ids", "positions", "block_table", "logits_index")
    assert ExecutionBatch.__slots__ == ("entries",)
    for bad, message in (
        (dict(token_ids=(), positions=()), "a batch entry must run at least one token"),
        (dict(token_ids=(1, 2), positions=(0,)), "token_ids and positions must have the same length"),
        (dict(token_ids=(1,), positions=(0,), logits_index=1), "logits_index must point inside the slice"),
        (dict(token_ids=(1,), positions=(0,), logits_index=-1), "logits_index must point inside the slice"),
    ):
        with pytest.raises(ValueError, match=message):
            BatchEntry("s", block_table=(0,), **bad)
    prefill = BatchEntry("p", (5, 6, 7), (0, 1, 2), (3,), 2)
    decode = BatchEntry("d", (9,), (40,), (1, 2, 4))
    assert (prefill.num_tokens, prefill.context_len, prefill.needs_logits) == (3, 3, True)
    assert (decode.num_tokens, decode.context_len, decode.needs_logits) == (1, 41, False)
    with pytest.raises(dataclasses.FrozenInstanceError):
        decode.seq_id = "x"
    batch = ExecutionBatch((prefill, decode))
    assert (batch.num_tokens, batch.num_sequences, batch.num_prefill_tokens) == (4, 2, 3)
    for twin in (pickle.loads(pickle.dumps(batch)), copy.deepcopy(batch), copy.copy(batch)):
        assert twin == batch and hash(twin) == hash(batch)
    assert dataclasses.replace(decode, positions=(41,)).context_len == 42
