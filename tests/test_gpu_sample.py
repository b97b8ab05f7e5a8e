"""Greedy sampling on the device (pkv_greedy_tokens) against NumPy's argmax, which is the
reference's greedy_token (sampling.py:28-30): bit-exact token ids, including ties (lowest id),
NaN (first NaN wins), -inf rows, signed zeros, odd vocabulary sizes and strided rows. The
whole config-1 run sampled on the device is in test_gpu_replay.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from paged_kv_serving_amd import ops

pytestmark = pytest.mark.gpu


def _argmax_rows(logits: np.ndarray) -> np.ndarray:
    return np.asarray([int(np.argmax(row)) for row in logits], dtype=np.int32)


@pytest.mark.parametrize("vocab", [1, 3, 4, 255, 256, 1000, 32_000, 128_256])
def test_random_rows_match_numpy(device, vocab) -> None:
    rng = np.random.default_rng(vocab)
    logits = rng.standard_normal((37, vocab)).astype(np.float32)
    got = ops.greedy_tokens(torch.from_numpy(logits).to(device)).cpu().numpy()
    assert np.array_equal(got, _argmax_rows(logits))


def test_ties_nan_infinities_and_signed_zeros(device) -> None:
    vocab = 1031  # not a multiple of 4: exercises the tail of the vector path
    rows = np.zeros((10, vocab), dtype=np.float32)
    rows[0, [5, 700, 1030]] = 2.0  # tie -> lowest id
    rows[1, :] = -np.inf  # all -inf -> 0
    rows[2, [9, 400]] = np.nan  # first NaN wins over everything
    rows[2, 3] = np.inf
    rows[3, 1030] = np.nan  # a NaN in the tail
    rows[3, 2] = 1e30
    rows[4, :] = -0.0
    rows[4, 600] = 0.0  # -0.0 and +0.0 tie -> 0
    rows[5, 1029] = np.inf
    rows[5, 1030] = np.inf  # tie of infinities in the tail
    rows[6, :] = np.float32(-3.0)
    rows[6, 1027] = np.float32(-2.9999998)  # one ulp above
    rows[7, 256 * 3 + 1] = 1.0  # one element, in another thread's stretch
    rows[8, :] = np.arange(vocab, dtype=np.float32)[::-1]  # maximum at 0
    rows[9, :] = np.arange(vocab, dtype=np.float32)  # maximum at the last id
    with np.errstate(invalid="ignore"):
        want = _argmax_rows(rows)
    got = ops.greedy_tokens(torch.from_numpy(rows).to(device)).cpu().numpy()
    assert np.array_equal(got, want), (got, want)


def test_strided_and_misaligned_rows(device) -> None:
    rng = np.random.default_rng(1)
    big = torch.from_numpy(rng.standard_normal((16, 300)).astype(np.float32)).to(device)
    view = big[:, 1:258]  # stride 300, base one float past 16-byte alignment
    got = ops.greedy_tokens(view).cpu().numpy()
    assert np.array_equal(got, _argmax_rows(big[:, 1:258].cpu().numpy()))
    aligned = big[::2, :256]  # stride 600, aligned: the vector path
    assert np.array_equal(ops.greedy_tokens(aligned).cpu().numpy(), _argmax_rows(aligned.cpu().numpy()))
