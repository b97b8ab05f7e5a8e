"""The kernels against the committed fixtures (tests/golden/*.npz): ragged attention within the
north star's 1e-5 of the float64 closed form, through both passes; the fused RoPE + append bit
for bit equal to the reference's float32 NumPy rotation. Reads only the fixture files."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from paged_kv_serving_amd import ops

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cases(name: str, prefix: str):
    with np.load(GOLDEN / name) as data:
        arrays = {key: data[key] for key in data.files}
    return [
        {k[len(f"{prefix}{i}_"):]: v for k, v in arrays.items() if k.startswith(f"{prefix}{i}_")}
        for i in range(int(arrays["count"]))
    ]


@pytest.mark.parametrize("tiles", [False, True], ids=["rows", "tiles"])
def test_attention_meets_the_golden_closed_form(device, tiles) -> None:
    for i, case in enumerate(_cases("attention_cases.npz", "c")):
        print("golden attention case", i, "tiles", tiles, flush=True)
        to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        plan = None
        if tiles:
            rows, tiles_ = ops.plan_rows(case["seq"], case["queries"].shape[2], min_tile_rows=2)
            visible = np.minimum(case["contexts"][case["seq"]], case["positions"] + 1)
            plan = ops.upload_plan(ops.expand_rows(rows, visible, 0), tiles_, device)
        out = ops.paged_attention_ragged(
            to(case["queries"]), to(case["positions"]), to(case["seq"]), to(case["keys"]),
            to(case["values"]), to(case["tables"]), to(case["contexts"]), float(case["scale"]),
            max_context_len=int(case["contexts"].max()), plan=plan,
        )  # fmt: skip
        worst = float(np.max(np.abs(out.cpu().numpy() - case["expected"])))
        assert worst < 1e-5, (i, worst)


def test_rope_append_matches_the_golden_rotation_bit_for_bit(device) -> None:
    for i, case in enumerate(_cases("rope_cases.npz", "r")):
        print("golden rope case", i, flush=True)
        fused = torch.from_numpy(case["fused"]).to(device)
        tokens, _, heads, dim = case["fused"].shape
        pool_k = torch.zeros((tokens, heads, dim), device=device)
        pool_v = torch.zeros_like(pool_k)
        slots = torch.arange(tokens, device=device)
        q = ops.rope_append(
            pool_k, pool_v, fused[:, 0], fused[:, 1], fused[:, 2], torch.from_numpy(case["positions"]).to(device),
            torch.from_numpy(case["cos"]).to(device), torch.from_numpy(case["sin"]).to(device), slots,
        )  # fmt: skip
        assert np.array_equal(q.cpu().numpy().view(np.uint32), case["q"].view(np.uint32)), i
        assert np.array_equal(pool_k.cpu().numpy().view(np.uint32), case["k"].view(np.uint32)), i
        assert np.array_equal(pool_v.cpu().numpy(), case["fused"][:, 2]), i
