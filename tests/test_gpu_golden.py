"""GPU: the HIP route / read / dQ paths against the committed golden vectors of the tiny
configuration (tests/golden/c1.npz).  Routed indices bit-exact (every top-k gap there is > 1e-4);
r, delta and dq within the fp16 bar (max-abs 2e-3, relative 1e-2)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_c1  # noqa: E402

from kv_skill_v2_amd import ops  # noqa: E402

pytestmark = pytest.mark.gpu


def _check(a, ref, what, rel=1e-2, atol=2e-3):
    a, ref = a.detach().double().cpu(), torch.from_numpy(ref).double()
    err = (a - ref).abs().max().item()
    rn = ((a - ref).norm() / ref.norm()).item()
    assert err <= atol and rn <= rel, (what, err, rn)


def test_golden_c1_on_gpu(dev):
    print("[case] golden c1", flush=True)
    z = dict(np.load(make_c1.OUT, allow_pickle=False))
    x = make_c1.inputs()
    lib = ops.PagedLibrary.from_padded(x["K"], x["M"], x["S"], device=dev)
    q = torch.from_numpy(z["q"]).to(dev)
    w, idx, wsel = ops.route_topk(q, lib, None, make_c1.TOP_K, make_c1.ROUTE_TEMP)
    assert np.array_equal(idx.cpu().numpy(), z["idx"])
    np.testing.assert_allclose(w.cpu().numpy(), z["w"], atol=1e-6)
    r = ops.library_read_decode(q, lib, idx, wsel, None, make_c1.READ_TEMP)
    _check(r, z["r"], "r (decode)")
    qd = q.clone().requires_grad_(True)
    r2, w2 = ops.library_read(qd, lib, lib.plan([make_c1.T]), make_c1.TOP_K, make_c1.READ_TEMP, make_c1.ROUTE_TEMP)
    _check(r2, z["r"], "r (mfma)")
    (r2 * x["g_up"].to(dev)).sum().backward()
    _check(qd.grad, z["dq"], "dq", atol=2e-3 * max(1.0, float(np.abs(z["dq"]).max())))
    hn = x["h"].to(dev) * torch.rsqrt(x["h"].to(dev).pow(2).mean(-1, keepdim=True) + 1e-6)
    g = torch.sigmoid(hn @ x["gate_w"].to(dev) + x["gate_b"].to(dev)).unsqueeze(-1)
    delta = torch.exp(x["log_gain"].to(dev)) * g * (r @ x["B_w"].to(dev).t())
    _check(delta, z["delta"], "delta")
