"""The forward pass's fused RMSNorm (optionally after its residual add) and SwiGLU gate product
(csrc/pkv_model.hip) against the oracle's float32 NumPy restatement of the reference model
(oracle/model.py rms_norm and silu, reference model.py:43-51) and its closed forms.

Tolerances: every operation is the same correctly rounded float32 operation as NumPy's; only the
sum of squares of the norm is added in another order, so the norm agrees within a few float32
ulps (rtol 2e-6) and the gate product within one or two (rtol 1e-6)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.model import rms_norm as oracle_rms_norm
from oracle.model import silu as oracle_silu

pytestmark = pytest.mark.gpu


def _to(device, array):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


@pytest.mark.parametrize("rows,dim", [(1, 1), (3, 7), (5, 64), (17, 128), (256, 320), (9, 4096), (2, 5000)])
def test_rms_norm_matches_the_oracle(device, rows, dim) -> None:
    from paged_kv_serving_amd import ops

    rng = np.random.default_rng(rows * 1000 + dim)
    x = (rng.standard_normal((rows, dim)) * rng.uniform(0.01, 30, (rows, 1))).astype(np.float32)
    w = rng.standard_normal(dim).astype(np.float32)
    got = ops.rms_norm(_to(device, x), _to(device, w), 1e-5).cpu().numpy()
    np.testing.assert_allclose(got, oracle_rms_norm(x, w, 1e-5), rtol=2e-6, atol=1e-7)


def test_rms_norm_with_the_residual_add_updates_hidden_in_place(device) -> None:
    from paged_kv_serving_amd import ops

    rng = np.random.default_rng(7)
    h = rng.standard_normal((33, 128)).astype(np.float32)
    d = rng.standard_normal((33, 128)).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    hidden = _to(device, h)
    got = ops.rms_norm(hidden, _to(device, w), 1e-5, delta=_to(device, d)).cpu().numpy()
    summed = (h + d).astype(np.float32)
    assert np.array_equal(hidden.cpu().numpy(), summed)  # the add is one float32 add per element
    np.testing.assert_allclose(got, oracle_rms_norm(summed, w, 1e-5), rtol=2e-6, atol=1e-7)


def test_rms_norm_closed_forms_and_strided_rows(device) -> None:
    """A constant row c normalises to c / sqrt(c^2 + eps) * w; rows of a wider buffer (a column
    slice) are read and written at their stride; out may be hidden itself."""
    import torch

    from paged_kv_serving_amd import ops

    base = torch.full((4, 48), 3.0, device=device)
    view = base[:, 8:40]  # rows of 32 at stride 48
    w = torch.arange(32, dtype=torch.float32, device=device)
    out = torch.zeros((4, 32), device=device)
    ops.rms_norm(view, w, 0.0, out=out)
    expect = (np.float32(3.0) / np.sqrt(np.float32(9.0))) * np.arange(32, dtype=np.float32)
    assert np.array_equal(out.cpu().numpy(), np.broadcast_to(expect, (4, 32)))
    assert torch.all(base[:, :8] == 3.0) and torch.all(base[:, 40:] == 3.0)
    h = torch.randn((5, 64), device=device)
    w2 = torch.randn(64, device=device)
    want = oracle_rms_norm(h.cpu().numpy(), w2.cpu().numpy(), 1e-5)
    ops.rms_norm(h, w2, 1e-5, out=h)
    np.testing.assert_allclose(h.cpu().numpy(), want, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("rows,width", [(1, 1), (4, 320), (129, 17), (300, 1024)])
def test_silu_mul_matches_the_oracle(device, rows, width) -> None:
    from paged_kv_serving_amd import ops

    rng = np.random.default_rng(rows + width)
    gate_up = (rng.standard_normal((rows, 2 * width)) * 8).astype(np.float32)
    got = ops.silu_mul(_to(device, gate_up), width).cpu().numpy()
    want = (oracle_silu(gate_up[:, :width]) * gate_up[:, width:]).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-30)


def test_silu_mul_edge_values(device) -> None:
    """silu(0) = 0, silu(x) = x past the clip (the exponential underflows to 0 at -60: 1 / (1 +
    e^-60) rounds to 1 in float32), silu(-x) -> -x e^-60 at the negative clip (no overflow), and
    a NaN gate propagates."""
    from paged_kv_serving_amd import ops

    gate = np.asarray([0.0, 100.0, 60.0, -100.0, -1e30, np.nan, 1.0, -1.0], np.float32)
    up = np.asarray([5.0, 2.0, 1.0, 1.0, 1.0, 1.0, 3.0, 3.0], np.float32)
    got = ops.silu_mul(_to(device, np.concatenate([gate, up])[None, :]), gate.size).cpu().numpy()[0]
    want = (oracle_silu(gate) * up).astype(np.float32)
    assert got[0] == 0.0 and got[1] == 200.0 and got[2] == 60.0
    assert np.isfinite(got[3]) and np.isfinite(got[4]) and got[3] < 0 and got[4] < 0
    assert np.isnan(got[5])
    np.testing.assert_allclose(got[[0, 1, 2, 3, 4, 6, 7]], want[[0, 1, 2, 3, 4, 6, 7]], rtol=1e-6)


@pytest.mark.parametrize("width,stride", [(128, 128), (30, 33), (64, 96)])
def test_gather_rows_picks_rows_and_zeroes_ids_outside_the_table(device, width, stride) -> None:
    """pkv_gather_rows: out[r] = src[index[r]] (the embedding lookup and the logits rows of the
    forward pass, model.py:262-263 and runner.py:215-227), zeros for an index outside the table;
    16-byte accesses when aligned, scalar otherwise."""
    import torch

    from paged_kv_serving_amd import _native

    rng = np.random.default_rng(width + stride)
    src = rng.standard_normal((50, stride)).astype(np.float32)
    index = np.asarray([3, 0, 49, 7, 7, -1, 50, 12], dtype=np.int64)
    d_src, d_index = _to(device, src), torch.from_numpy(index).to(device)
    out = torch.full((index.size, width + 3), 5.0, device=device)
    rc = _native.library().pkv_gather_rows(out.data_ptr(), width + 3, d_src.data_ptr(), stride, 50,
                                           d_index.data_ptr(), index.size, width, device.index, None)  # fmt: skip
    assert rc == 0
    got = out.cpu().numpy()
    for r, i in enumerate(index):
        want = src[i, :width] if 0 <= i < 50 else np.zeros(width, np.float32)
        assert np.array_equal(got[r, :width], want), r
        assert np.all(got[r, width:] == 5.0)  # nothing past the row's width is written
