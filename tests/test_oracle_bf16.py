"""Pin the oracle's float32 -> bfloat16 rounding (used for the bf16-KV tolerance oracle).

Checked against torch's CPU conversion (an independent implementation) on random and special
values, and against hand-computed round-to-nearest-even cases.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle.bf16 import bf16_bits, bf16_round, bits_to_f32


def test_matches_torch_on_random_and_special_values() -> None:
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100_000),
        np.asarray([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38], dtype=np.float32),
    ]).astype(np.float32)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16_bits(x), theirs)


def test_ties_round_to_even_and_nan_is_quiet() -> None:
    one = np.float32(1.0)
    ulp = 2.0**-7  # bfloat16 spacing at 1.0
    cases = {
        1.0 + ulp / 2: 1.0,  # tie, 1.0 is even -> down
        1.0 + 3 * ulp / 2: 1.0 + 2 * ulp,  # tie, odd below -> up
        1.0 + ulp / 2 + 2.0**-20: 1.0 + ulp,  # just above the tie -> up
    }
    for value, expected in cases.items():
        assert bf16_round(np.asarray([value], dtype=np.float32))[0] == np.float32(expected)
    assert bf16_bits(np.asarray([np.nan], dtype=np.float32))[0] == 0x7FC0
    assert np.isnan(bits_to_f32(np.asarray([0x7FC0], dtype=np.uint16))[0])
    assert bf16_round(np.asarray([one]))[0] == one
