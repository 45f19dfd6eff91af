"""Small models and skills for the API tests, and a CPU fp64 re-run of a hooked forward through
the oracle (the reference path of each injection layer restated with oracle functions)."""

from __future__ import annotations

import copy

import torch
import torch.nn as nn

import oracle as O
from kv_skill_v2_amd.depth import KVSkill, unit_rows


class _Config:
    def __init__(self, n_layers: int, hidden: int):
        self.num_hidden_layers = n_layers
        self.hidden_size = hidden


class _Stack(nn.Module):
    def __init__(self, d: int, n_layers: int):
        super().__init__()
        self.layers = nn.ModuleList(nn.Linear(d, d) for _ in range(n_layers))


class TinyLM(nn.Module):
    """A decoder-shaped stack: model.layers, config, device; forward(x) = tanh-linear layers."""

    def __init__(self, d: int = 32, n_layers: int = 8, seed: int = 0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.model = _Stack(d, n_layers)
        with torch.no_grad():
            for p in self.model.parameters():
                p.copy_(torch.randn(p.shape, generator=g) / d ** 0.5)
        self.config = _Config(n_layers, d)

    @property
    def device(self):
        return next(self.parameters()).device

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.model.layers:
            x = torch.tanh(layer(x))
        return x


def skill_rho(d_s: int, depths, n: int = 16, seed: int = 0) -> KVSkill:
    """A rho-keyed skill with tied K = V unit rows."""
    g = torch.Generator().manual_seed(seed)
    K = {float(r): unit_rows(n, d_s, g) for r in depths}
    return KVSkill(K=K, V=K, d_s=d_s, text=f"doc{seed}", model_name="tiny-enc",
                   meta={"keyed_by": "rho", "depths": sorted(float(r) for r in depths), "tied": True})


def randomize(module: nn.Module, seed: int = 0, scale: float = 0.3) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * scale)


def x_in(d: int, T: int = 7, B: int = 2, seed: int = 1) -> torch.Tensor:
    return torch.randn(B, T, d, generator=torch.Generator().manual_seed(seed))


def oracle_forward(model: nn.Module, x: torch.Tensor, itf, tensors: dict, *, top_k: int = 0,
                   read_temp: float = 12.0, route_temp: float = 10.0, read_softmax: bool = True,
                   selector=None, grad: bool = False, call=None):
    """Run a CPU fp64 copy of `model` with one hook per injection layer computing the reference
    branch with oracle functions.  tensors: {li: (K, M, S[, V])}.  selector: a LayerSelector whose
    parameters are copied (weights from its u at the first candidate layer).  call(m, x) runs the
    copy (default: m(x) on fp64 x).  Returns (output, copies) where copies = (interface copy,
    selector copy) for gradient comparisons."""
    m = copy.deepcopy(model).cpu().double()
    for mod in m.modules():          # the copy must not run hooks an injector put on `model`
        mod._forward_hooks.clear()
        mod._forward_pre_hooks.clear()
    it = copy.deepcopy(itf).cpu().double()
    sel = copy.deepcopy(selector).cpu().double() if selector is not None else None
    blocks = m.model.layers
    state = {}

    def make(li):
        def hook(mod, args, out):
            h = out
            hn = O.rms_norm(h)
            q = O.query(hn, it.A.weight, it.A.bias if hasattr(it.A, "bias") else None)
            K, M, S = (t.double() if t.is_floating_point() else t for t in tensors[li][:3])
            V = tensors[li][3].double() if len(tensors[li]) > 3 and tensors[li][3] is not None else None
            r, _ = O.branch_read(q, K, M, S, read_temp, route_temp, top_k, read_softmax, V)
            p = it._pos[li]
            delta = O.epilogue(hn, r, it.B.weight, it.B.bias, it.gate_w, it.gate_b[p], it.log_gain[p])
            if sel is not None:
                if li == sel.first_layer:
                    z = torch.nn.functional.linear(hn, sel.u.weight, sel.u.bias)
                    state["w"] = O.selector_weights(z, sel.k, sel.straight_through)
                delta = O.selector_apply(delta, h, state["w"][..., sel.pos[li]], sel.log_alpha)
            return h + delta
        return hook

    for li in it.inject_layers:
        blocks[li].register_forward_hook(make(li))
    with torch.set_grad_enabled(grad):
        y = call(m, x.cpu()) if call is not None else m(x.cpu().double())
    return y, (it, sel)


def close(a: torch.Tensor, b: torch.Tensor, rel: float = 1e-2, atol: float = 2e-3) -> tuple:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    err = (a - b).abs().max().item()
    rn = ((a - b).norm() / b.norm().clamp_min(1e-30)).item()
    ok = rn <= rel and err <= atol * max(1.0, b.abs().max().item())
    return ok, err, rn
