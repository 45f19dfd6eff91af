"""The committed golden vectors of the tiny configuration (tests/golden/c1.npz, written by
tests/golden/make_c1.py from the fp64 oracle): the regenerated inputs must hash to the recorded
digests, and the oracle must reproduce the recorded outputs (CPU)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_c1  # noqa: E402

import oracle as O  # noqa: E402


def load():
    return dict(np.load(make_c1.OUT, allow_pickle=False))


def test_inputs_regenerate_bit_identically():
    z = load()
    x = make_c1.inputs()
    for k, v in x.items():
        assert make_c1.digest(v) == str(z["sha256_" + k]), k
    assert z["nvalid"].tolist() == x["M"].sum(-1).tolist()


def test_oracle_reproduces_golden_outputs():
    z = load()
    e = make_c1.expected(make_c1.inputs())
    assert np.array_equal(e["idx"].numpy(), z["idx"])
    for k in ("q", "w", "r", "delta", "dq", "gamma"):
        np.testing.assert_allclose(e[k].float().numpy(), z[k], rtol=0, atol=1e-6, err_msg=k)


def test_fp32_reference_order_is_within_fp32_error_of_golden():
    """The reference computes in fp32: its route/read order on fp32 inputs lands within 1e-5 of
    the fp64 golden vectors, and picks the same chunks (every top-k gap exceeds 1e-4)."""
    z = load()
    x = make_c1.inputs()
    q = torch.from_numpy(z["q"]).view(1, -1, make_c1.D_S)
    assert float(z["gap"].min()) > 1e-5
    r, w = O.branch_read(q, x["K"], x["M"], x["S"], make_c1.READ_TEMP, make_c1.ROUTE_TEMP, make_c1.TOP_K)
    assert torch.equal((w[0] > 0), torch.from_numpy(z["w"]) > 0)
    np.testing.assert_allclose(r[0].numpy(), z["r"], atol=1e-5)
