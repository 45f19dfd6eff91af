"""The reader-side maps around the Library read, and their checkpoint file.

`ModelInterface` holds what the injector applies around the read (the fields and methods the
reference's branch uses, xenc/injector.py:54-77):
    A        d_m -> d_s query map; q = A(rms_norm(h)) / (|A(rms_norm(h))| + 1e-6)
    B        d_s -> d_m write map, no bias, zero at initialisation so an untrained branch adds
             exactly nothing
    gate_w   [d_m] and gate_b [n_layers]: gate sigmoid(hn . gate_w + gate_b[pos])
    log_gain [n_layers]: gain exp(log_gain[pos])
    _pos     {reader layer: position in inject_layers}
Each method brings its weights to the input's device, so a reader sharded over devices can call
it from any layer (autograd still reaches the master copy).  The reference takes this class from
an external package that is not available; its initialisation is therefore a documented choice
here: A without bias (a rank-r factorisation when rank > 0), gate_w = 0, gate_b = gate_bias_init,
log_gain = gain_init.

The checkpoint file keeps the reference's format ("xenc.interface.v1": format, config,
state_dict, selector, extra) so that files written by either side load on the other; it holds
only tensors, strings, numbers and lists, and is read with torch.load(weights_only=True).
"""

from __future__ import annotations

import os
import tempfile
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F

from .selector import LayerSelector

FORMAT = "xenc.interface.v1"
_EPS = 1e-6


def _here(t: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    return t if t.device == x.device else t.to(x.device)


def apply_map(mod: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """A bias-optional linear map (or a chain of them) applied with its weights on x's device."""
    layers = list(mod) if isinstance(mod, nn.Sequential) else [mod]
    for lin in layers:
        x = F.linear(x, _here(lin.weight, x), None if lin.bias is None else _here(lin.bias, x))
    return x


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
        q = apply_map(self.A, hn)
        return q / (torch.linalg.vector_norm(q, dim=-1, keepdim=True) + _EPS)

    def gate(self, hn: torch.Tensor, li: int) -> torch.Tensor:
        p = self._pos[li]
        z = hn @ _here(self.gate_w, hn) + _here(self.gate_b, hn)[p]
        return torch.sigmoid(z)[..., None]

    def gain(self, li: int) -> torch.Tensor:
        return torch.exp(self.log_gain[self._pos[li]])

    def write(self, r: torch.Tensor) -> torch.Tensor:
        return apply_map(self.B, r)


def make_interface(d_reader: int, d_encoder: int, reader_layers: list[int], rank: int = 0,
                   gate_bias_init: float = -2.0, gain_init: float = 0.0) -> ModelInterface:
    layers = [int(li) for li in reader_layers]
    repeated = sorted({li for li in layers if layers.count(li) > 1})
    if repeated:
        raise ValueError(f"reader layers {repeated} appear more than once in {layers}")
    return ModelInterface(int(d_reader), int(d_encoder), layers, gate_bias_init=gate_bias_init,
                          gain_init=gain_init, rank=int(rank or 0))


def _host_state(m: nn.Module) -> dict:
    return {name: t.detach().to("cpu") for name, t in m.state_dict().items()}


def save_interface(itf: ModelInterface, path: str, selector: LayerSelector | None = None,
                   extra: dict | None = None) -> None:
    """Write the checkpoint: the file appears complete or not at all (a temporary file in the same
    directory, then an atomic rename)."""
    record = {
        "format": FORMAT,
        "config": {"d_m": itf.d_m, "d_s": itf.d_s, "inject_layers": list(itf.inject_layers),
                   "rank": int(getattr(itf, "rank", 0) or 0)},
        "state_dict": _host_state(itf),
        "selector": None if selector is None else {"config": selector.config(),
                                                   "state_dict": _host_state(selector)},
        "extra": extra,
    }
    folder = Path(path).resolve().parent
    folder.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=".itf-", suffix=".part", dir=folder)
    os.close(fd)
    try:
        torch.save(record, tmp)
        os.replace(tmp, path)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)


def load_interface(path: str, d_reader: int, d_encoder: int, reader_layers: list[int],
                   map_location="cpu"):
    """-> (interface, selector or None, extra).  ValueError when the file was written for other
    dimensions or reader layers."""
    record = torch.load(path, map_location=map_location, weights_only=True)
    cfg = record["config"]
    expect = {"d_m": int(d_reader), "d_s": int(d_encoder), "inject_layers": [int(li) for li in reader_layers]}
    found = {"d_m": cfg["d_m"], "d_s": cfg["d_s"], "inject_layers": list(cfg["inject_layers"])}
    if found != expect:
        raise ValueError(f"{path} holds an interface for {found}, not for {expect}")
    itf = make_interface(d_reader, d_encoder, reader_layers, rank=cfg.get("rank", 0))
    itf.load_state_dict(record["state_dict"], strict=True)
    sel_rec = record.get("selector")
    selector = None
    if sel_rec is not None:
        sc = sel_rec["config"]
        selector = LayerSelector(sc["d_m"], sc["cand_layers"], k=sc["k"],
                                 straight_through=sc.get("straight_through", False))
        selector.load_state_dict(sel_rec["state_dict"], strict=True)
    return itf, selector, record.get("extra")


__all__ = ["FORMAT", "ModelInterface", "make_interface", "save_interface", "load_interface", "apply_map"]
