"""The reader-side interface of the Library read and its save / load format.

`ModelInterface` holds, per reader model, the maps around the read (the fields
xenc/injector.py:54-77 uses):
    A        d_m -> d_s query map (q = A(rms_norm(h)), then row-L2)
    B        d_s -> d_m write map without bias, zero-initialised so that an untrained branch is a
             no-op (a zero read writes exactly zero: tests/test_d6_force_attn.py:66-68 relies on it)
    gate_w   [d_m], gate_b [n_layers]: gate sigma(hn . gate_w + gate_b[pos])
    log_gain [n_layers]: gain exp(log_gain[pos])
    _pos     {reader layer: position}
The original class lives in an external package that is not part of the reference; its
initialisation is not pinned by any file here, so the choices below are documented parameters:
A is nn.Linear(d_m, d_s, bias=False) (or a rank-r factorisation when rank > 0), gate_w starts at 0,
gate_b at gate_bias_init and log_gain at gain_init.  The methods query / gate / gain / write are
the ones the reference tests call on an interface (tests/test_interface.py:28-40).

make_interface / save_interface / load_interface / interface_param_groups / count_params /
EncoderLens follow xenc/interface.py:22-119.  The saved blob holds only tensors, strings, numbers
and lists, so `load_interface` reads it with torch.load(weights_only=True).
"""

from __future__ import annotations

import os

import torch
import torch.nn as nn

from .selector import LayerSelector

FORMAT = "xenc.interface.v1"


class ModelInterface(nn.Module):
    def __init__(self, d_m: int, d_s: int, inject_layers: list[int], gate_bias_init: float = -2.0,
                 gain_init: float = 0.0, rank: int = 0):
        super().__init__()
        self.d_m, self.d_s, self.rank = int(d_m), int(d_s), int(rank or 0)
        self.inject_layers = [int(li) for li in inject_layers]
        self._pos = {li: i for i, li in enumerate(self.inject_layers)}
        if self.rank > 0:
            self.A = nn.Sequential(nn.Linear(self.d_m, self.rank, bias=False),
                                   nn.Linear(self.rank, self.d_s, bias=False))
        else:
            self.A = nn.Linear(self.d_m, self.d_s, bias=False)
        self.B = nn.Linear(self.d_s, self.d_m, bias=False)
        nn.init.zeros_(self.B.weight)
        n = len(self.inject_layers)
        self.gate_w = nn.Parameter(torch.zeros(self.d_m))
        self.gate_b = nn.Parameter(torch.full((n,), float(gate_bias_init)))
        self.log_gain = nn.Parameter(torch.full((n,), float(gain_init)))

    def query(self, hn: torch.Tensor) -> torch.Tensor:
        q = self.A(hn)
        return q / (q.norm(dim=-1, keepdim=True) + 1e-6)

    def gate(self, hn: torch.Tensor, li: int) -> torch.Tensor:
        return torch.sigmoid(hn @ self.gate_w + self.gate_b[self._pos[li]]).unsqueeze(-1)

    def gain(self, li: int) -> torch.Tensor:
        return self.log_gain[self._pos[li]].exp()

    def write(self, r: torch.Tensor) -> torch.Tensor:
        return self.B(r)


def make_interface(d_reader: int, d_encoder: int, reader_layers: list[int], rank: int = 0,
                   gate_bias_init: float = -2.0, gain_init: float = 0.0) -> ModelInterface:
    layers = [int(li) for li in reader_layers]
    if len(set(layers)) != len(layers):
        raise ValueError(f"duplicate reader layers: {layers}")
    return ModelInterface(int(d_reader), int(d_encoder), layers, gate_bias_init=gate_bias_init,
                          gain_init=gain_init, rank=int(rank or 0))


class EncoderLens(nn.Module):
    """Per-encoder linear projection d_enc -> d_core on the last dim (orthogonal init, no bias)."""

    def __init__(self, d_enc: int, d_core: int):
        super().__init__()
        self.d_enc, self.d_core = int(d_enc), int(d_core)
        self.proj = nn.Linear(self.d_enc, self.d_core, bias=False)
        nn.init.orthogonal_(self.proj.weight)

    def forward(self, K: torch.Tensor) -> torch.Tensor:
        if K.shape[-1] != self.d_enc:
            raise ValueError(f"EncoderLens expects last dim {self.d_enc}, got {K.shape[-1]}")
        return self.proj(K.to(self.proj.weight.dtype))


def interface_param_groups(itf: nn.Module, lr: float, selector: LayerSelector | None = None,
                           selector_lr: float | None = None, lr_A: float | None = None) -> list[dict]:
    """Optimizer parameter groups: the interface at lr (the query map A at lr_A when given), then
    the selector's parameters at selector_lr (default lr)."""
    trainable = [p for p in itf.parameters() if p.requires_grad]
    if lr_A is not None and hasattr(itf, "A"):
        a_ids = {id(p) for p in itf.A.parameters()}
        groups = [{"params": [p for p in trainable if id(p) not in a_ids], "lr": lr, "name": "interface"},
                  {"params": [p for p in itf.A.parameters() if p.requires_grad], "lr": float(lr_A),
                   "name": "interface_A"}]
        groups = [g for g in groups if g["params"]]
    else:
        groups = [{"params": trainable, "lr": lr, "name": "interface"}]
    if selector is not None:
        seen = {id(p) for g in groups for p in g["params"]}
        extra = [p for p in selector.parameters() if p.requires_grad and id(p) not in seen]
        if extra:
            groups.append({"params": extra, "lr": lr if selector_lr is None else selector_lr,
                           "name": "selector"})
    return groups


def _config(itf: ModelInterface) -> dict:
    return {"d_m": itf.d_m, "d_s": itf.d_s, "inject_layers": list(itf.inject_layers),
            "rank": int(getattr(itf, "rank", 0) or 0)}


def _cpu_state(m: nn.Module) -> dict:
    return {k: v.detach().cpu() for k, v in m.state_dict().items()}


def save_interface(itf: ModelInterface, path: str, selector: LayerSelector | None = None,
                   extra: dict | None = None) -> None:
    """Write {format, config, state_dict, selector, extra} atomically (tmp file + rename)."""
    blob = {"format": FORMAT, "config": _config(itf), "state_dict": _cpu_state(itf),
            "selector": None, "extra": extra}
    if selector is not None:
        blob["selector"] = {"config": selector.config(), "state_dict": _cpu_state(selector)}
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    tmp = path + ".tmp"
    torch.save(blob, tmp)
    os.replace(tmp, path)


def load_interface(path: str, d_reader: int, d_encoder: int, reader_layers: list[int],
                   map_location="cpu"):
    """-> (interface, selector or None, extra); ValueError when the saved dims / layers differ."""
    blob = torch.load(path, map_location=map_location, weights_only=True)
    cfg = blob["config"]
    want = (int(d_reader), int(d_encoder), [int(li) for li in reader_layers])
    got = (cfg["d_m"], cfg["d_s"], list(cfg["inject_layers"]))
    if want != got:
        raise ValueError(f"interface at {path} has (d_m, d_s, layers)={got}, expected {want}")
    itf = make_interface(d_reader, d_encoder, reader_layers, rank=cfg.get("rank", 0))
    itf.load_state_dict(blob["state_dict"], strict=True)
    selector = None
    if blob.get("selector") is not None:
        sc = blob["selector"]["config"]
        selector = LayerSelector(sc["d_m"], sc["cand_layers"], k=sc["k"],
                                 straight_through=sc.get("straight_through", False))
        selector.load_state_dict(blob["selector"]["state_dict"], strict=True)
    return itf, selector, blob.get("extra")


def count_params(itf: nn.Module, selector: LayerSelector | None = None) -> dict:
    n_itf = sum(p.numel() for p in itf.parameters())
    out = {"interface": n_itf}
    for name in ("A", "B"):
        m = getattr(itf, name, None)
        if isinstance(m, nn.Module):
            out[name] = sum(p.numel() for p in m.parameters())
    out["gate_gain"] = n_itf - out.get("A", 0) - out.get("B", 0)
    out["selector"] = sum(p.numel() for p in selector.parameters()) if selector is not None else 0
    out["total"] = n_itf + out["selector"]
    return out


__all__ = ["FORMAT", "ModelInterface", "make_interface", "EncoderLens", "interface_param_groups",
           "save_interface", "load_interface", "count_params"]
