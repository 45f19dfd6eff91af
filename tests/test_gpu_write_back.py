"""GPU: the decode path's write-back (xenc_write_back) against the fp64 oracle epilogue
(xenc/injector.py:61-77, 266-267: delta = gain_scale * exp(log_gain[p]) * gate * B(r)): one
shared B, per-depth Bs selected by row group (the multi-depth shape, with an unused depth and
depths serving more than one batch of 8 rows), odd output counts, shared and per-group bias,
no bias / scale / groups, determinism and the guards."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _ref(r, W, groups, bias, scale):
    r64, W64 = r.double(), W.double()
    if W64.dim() == 2:
        W64 = W64.unsqueeze(0)
    out = torch.empty(r.shape[0], W64.shape[1], dtype=torch.float64)
    for m in range(r.shape[0]):
        g = int(groups[m]) if groups is not None else 0
        y = W64[g] @ r64[m]
        if bias is not None:
            b = bias.double()
            y = y + (b[g] if b.dim() == 2 else b)
        out[m] = y * (float(scale[m]) if scale is not None else 1.0)
    return out


def _check(out, ref):
    err = (out.double().cpu() - ref).abs().max().item()
    tol = 2e-6 * max(1.0, ref.abs().max().item())
    assert err <= tol, f"max-abs {err:.3g} > {tol:.3g}"


@pytest.mark.parametrize("M,d,d_out,G,bias_kind", [
    (1, 2560, 5120, 1, "none"),
    (3, 256, 512, 1, "shared"),
    (40, 512, 1000, 1, "shared"),           # 5 batches of 8 rows, d_out not a multiple of 32
    (64, 2560, 5120, 8, "per_group"),       # the multi-depth shape
    (17, 12, 7, 3, "shared"),               # tiny d and d_out
    (300, 100, 70, 3, "per_group"),         # libraries of ~100 rows: several 32-row passes each
    (4096, 32, 20, 2, "none"),              # the row limit
])
def test_write_back_matches_oracle(dev, M, d, d_out, G, bias_kind):
    say("write-back", dict(M=M, d=d, d_out=d_out, G=G, bias=bias_kind))
    g = torch.Generator().manual_seed(M * 7 + d)
    r = torch.randn(M, d, generator=g)
    W = torch.randn(G, d_out, d, generator=g) / d ** 0.5 if G > 1 else torch.randn(d_out, d, generator=g) / d ** 0.5
    groups = None
    if G > 2:
        # depth 1 unused; depth 0 serves 20 rows (three batches); the rest spread
        pool = [0] * 20 + [2 + (m % (G - 2)) for m in range(M - 20)]
        groups = torch.tensor(pool[:M], dtype=torch.int32)[torch.randperm(M, generator=g)]
    elif G == 2:
        groups = torch.randint(0, 2, (M,), generator=g, dtype=torch.int32)
    bias = None
    if bias_kind == "shared":
        bias = torch.randn(d_out, generator=g)
    elif bias_kind == "per_group":
        bias = torch.randn(G, d_out, generator=g)
    scale = torch.rand(M, generator=g) + 0.5
    out = ops.write_back(r.to(dev), W.to(dev), groups.to(dev) if groups is not None else None,
                         bias.to(dev) if bias is not None else None, scale.to(dev))
    _check(out, _ref(r, W, groups, bias, scale))
    again = ops.write_back(r.to(dev), W.to(dev), groups.to(dev) if groups is not None else None,
                           bias.to(dev) if bias is not None else None, scale.to(dev))
    assert torch.equal(out, again)


def test_write_back_equals_oracle_epilogue(dev):
    """row_scale = gain_scale * exp(log_gain[p]) * sigmoid(hn . gate_w + gate_b[p]) reproduces the
    oracle's epilogue exactly up to fp32 rounding."""
    say("write-back epilogue")
    g = torch.Generator().manual_seed(5)
    d_m, d_s, T = 384, 256, 6
    hn = O.rms_norm(torch.randn(T, d_m, generator=g))
    r = torch.randn(T, d_s, generator=g)
    B_w, B_b = torch.randn(d_m, d_s, generator=g) / 16, torch.randn(d_m, generator=g)
    gate_w, gate_b, log_gain = torch.randn(d_m, generator=g) / 20, torch.tensor(-1.5), torch.tensor(0.3)
    ref = O.epilogue(hn.double(), r.double(), B_w.double(), B_b.double(), gate_w.double(),
                     gate_b.double(), log_gain.double(), gain_scale=0.7)
    scale = 0.7 * torch.exp(log_gain) * torch.sigmoid(hn @ gate_w + gate_b)
    out = ops.write_back(r.to(dev), B_w.to(dev), None, B_b.to(dev), scale.float().to(dev))
    _check(out, ref)


def test_write_back_no_scale_no_bias_and_guards(dev):
    say("write-back guards")
    g = torch.Generator().manual_seed(9)
    r = torch.randn(5, 64, generator=g)
    W = torch.randn(48, 64, generator=g)
    _check(ops.write_back(r.to(dev), W.to(dev)), (W.double() @ r.double().T).T)
    with pytest.raises(ValueError):
        ops.write_back(torch.randn(2, 62, device=dev), torch.randn(8, 62, device=dev))   # d % 4
    with pytest.raises(ValueError):
        ops.write_back(torch.randn(4097, 64, device=dev), W.to(dev))                     # M > 4096
    with pytest.raises(ValueError):
        ops.write_back(r.to(dev).half(), W.to(dev))
    with pytest.raises(ValueError):
        ops.write_back(r.to(dev), W.to(dev), torch.zeros(4, dtype=torch.int32, device=dev))
    assert ops.write_back(r[:0].to(dev), W.to(dev)).shape == (0, 48)
