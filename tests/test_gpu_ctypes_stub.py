"""GPU: the reference-side ctypes binding printed in INTEGRATION.md runs as written (its library
path pointed at the built library) and its route + read equal the oracle's Library branch read
(xenc/injector.py:220-265) on a seeded library.  Keeps the documented argtypes in step with the
ABI."""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import _lib
from kv_skill_v2_amd.depth import unit_rows

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _stub() -> dict:
    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text[text.index("## 3. Binding the C ABI"):]
    code = re.search(r"```python\n(.*?)```", sec, re.S).group(1)
    code = code.replace("/path/to/kv_skill_v2_amd/_lib/libxenc_hip.so", str(_lib.LIB_PATH))
    ns: dict = {}
    exec(compile(code, "INTEGRATION.md:_mi355x.py", "exec"), ns)
    return ns


def test_documented_ctypes_binding_matches_oracle(dev):
    print("[case] INTEGRATION.md ctypes stub", flush=True)
    _lib.lib()   # the built library must exist (and load) before the stub binds it
    ns = _stub()
    g = torch.Generator().manual_seed(3)
    d, n = 128, [64, 17, 64, 1, 40, 64]
    rows = [unit_rows(k, d, g) for k in n]
    K, M, S = O.library_tensors(rows)
    q = unit_rows(5, d, g)
    top_k = 3
    w, idx, ws = ns["route"](q.to(dev), S.to(dev), top_k, 10.0)
    reader = ns["Reader"](K.half().to(dev).contiguous(), M.sum(-1), max_rows=8, kk=top_k, nsplit=2)
    r = reader(q.to(dev), idx, ws).cpu().double()
    r2 = reader(q[:2].to(dev), idx[:2], ws[:2]).cpu().double()     # smaller call, same workspace
    for m in range(q.shape[0]):
        qm = q[m].view(1, 1, -1).double()
        assert float(O.boundary_gap(qm, S, top_k).min()) > 2e-5
        ref, wref = O.branch_read(qm, K.double(), M, S.double(), top_k=top_k)
        assert float((w[m].cpu().double() - wref.view(-1)).abs().max()) < 1e-5
        assert float((r[m] - ref.view(-1)).abs().max()) < 2e-3
    assert torch.equal(r2, r[:2])
