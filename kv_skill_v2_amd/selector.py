"""LayerSelector: a sparse top-k gate over candidate reader layers (xenc/selector.py:36-118).

At the first candidate layer the selector reads the RMS-normed residual once per forward and keeps
per-token weights w [B, T, n_cand] (top-k of u(hn0), softmax over the kept logits, zero
elsewhere; optionally straight-through: uniform 1/k forward, dense softmax gradient).  Each
candidate layer's update is rescaled to a matched norm, ||delta|| / ||h|| = alpha per token, then
multiplied by its weight, so after `apply` ||delta_l|| / ||h|| = w_l * alpha.

The injector resets the selector before every forward; `apply` at the first candidate layer
recomputes the weights unless `compute` was called explicitly for this forward.

`selected_rows(li)` exposes which token rows give layer li a nonzero weight: the injector reads
the Library only for those rows (every other row's update is multiplied by an exact 0).
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

_EPS = 1e-6


def rms_norm(x: torch.Tensor, eps: float = _EPS) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) over the last dim, in fp32 (no weight)."""
    x = x.float()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def _on(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if t.device == like.device else t.to(like.device)


class LayerSelector(nn.Module):
    def __init__(self, d_m: int, cand_layers: list[int], k: int = 2, alpha_init: float = 0.02,
                 straight_through: bool = False):
        super().__init__()
        cand = [int(li) for li in cand_layers]
        if len(set(cand)) != len(cand):
            raise ValueError(f"duplicate candidate layers: {cand}")
        if not 1 <= k <= len(cand):
            raise ValueError(f"k={k} must be in [1, {len(cand)}]")
        if alpha_init <= 0:
            raise ValueError("alpha_init must be > 0")
        self.d_m, self.k = int(d_m), int(k)
        self.cand_layers = sorted(cand)
        self.n_cand = len(self.cand_layers)
        self.pos = {li: i for i, li in enumerate(self.cand_layers)}
        self.first_layer = self.cand_layers[0]
        self.straight_through = bool(straight_through)
        self.u = nn.Linear(self.d_m, self.n_cand, bias=True)
        self.log_alpha = nn.Parameter(torch.tensor(math.log(alpha_init)))
        self._w: torch.Tensor | None = None
        self._explicit = False

    # ------------------------------------------------------------------ weights
    def _weights_from_logits(self, z: torch.Tensor) -> torch.Tensor:
        if (z.is_cuda and z.dtype == torch.float32 and not self.straight_through and z.shape[-1] <= 256
                and not (torch.is_grad_enabled() and z.requires_grad)):
            from .ops import selector_weights   # xenc_selector_weights: ties to the lower index
            w, _, _ = selector_weights(z.reshape(-1, z.shape[-1]).contiguous(), self.k)
            return w.view(z.shape)
        top, idx = z.topk(self.k, dim=-1)
        sparse = torch.zeros_like(z).scatter(-1, idx, torch.softmax(top, dim=-1))
        if not self.straight_through:
            return sparse
        hard = torch.zeros_like(z).scatter(-1, idx, torch.full_like(top, 1.0 / self.k))
        soft = torch.softmax(z, dim=-1)
        return hard + (soft - soft.detach())

    def compute(self, hn0: torch.Tensor) -> None:
        """hn0 [B, T, d_m]: RMS-normed residual at the first candidate layer."""
        x = hn0.to(self.u.weight.dtype)
        self._w = self._weights_from_logits(F.linear(x, _on(self.u.weight, x), _on(self.u.bias, x)))
        self._explicit = True

    def reset(self) -> None:
        self._w = None
        self._explicit = False

    def weights(self) -> torch.Tensor | None:
        return self._w

    @torch.no_grad()
    def entropy(self) -> torch.Tensor | None:
        if self._w is None:
            return None
        w = self._w.detach().float().clamp_min(0)
        return -(w * torch.log(w.clamp_min(1e-12))).sum(-1).mean()

    def alpha(self) -> torch.Tensor:
        return self.log_alpha.exp()

    # ------------------------------------------------------------------ apply
    def _ensure(self, h: torch.Tensor, li: int) -> None:
        if li == self.first_layer:
            if not self._explicit or self._w is None:
                self.compute(rms_norm(h))
            self._explicit = False           # consumed: the next first-layer call is a new forward
        elif self._w is None or self._w.shape[:-1] != h.shape[:-1]:
            self.compute(rms_norm(h))          # hooks entered past the first candidate layer
            self._explicit = False

    def selected_rows(self, h: torch.Tensor, li: int) -> torch.Tensor:
        """Bool [B, T]: rows whose weight for layer li is nonzero (computes the weights at the
        first candidate layer exactly as `apply` would; `apply` then reuses them)."""
        p = self.pos[li]
        self._ensure(h, li)
        if li == self.first_layer:
            self._explicit = True            # let the apply() of this same layer reuse them
        return self._w[..., p] != 0

    def apply(self, delta: torch.Tensor, h: torch.Tensor, li: int) -> torch.Tensor:
        """Matched-norm rescale of delta, times w[..., pos[li]]; returns delta's dtype."""
        p = self.pos[li]                     # KeyError for a non-candidate layer
        self._ensure(h, li)
        if (delta.is_cuda and not (torch.is_grad_enabled() and (delta.requires_grad or self.log_alpha.requires_grad
                                                                 or self._w.requires_grad))):
            from .ops import selector_apply      # xenc_selector_apply (k = 1)
            shp = delta.shape
            d2 = delta.float().reshape(-1, shp[-1]).contiguous()
            h2 = h.float().reshape(-1, shp[-1]).contiguous()
            w2 = _on(self._w[..., p], d2).reshape(-1).float().contiguous()
            return selector_apply(d2, h2, w2, self.log_alpha, k=1).view(shp).to(delta.dtype)
        d = delta.float()
        rel = d.norm(dim=-1, keepdim=True) / (h.float().norm(dim=-1, keepdim=True) + _EPS)
        d = d / (rel + _EPS) * _on(self.log_alpha, d).exp()
        out = _on(self._w[..., p], d).unsqueeze(-1).to(d.dtype) * d
        return out.to(delta.dtype)

    def extra_repr(self) -> str:
        return (f"d_m={self.d_m}, cand_layers={self.cand_layers}, k={self.k}, "
                f"straight_through={self.straight_through}")

    def config(self) -> dict:
        return {"d_m": self.d_m, "cand_layers": list(self.cand_layers), "k": self.k,
                "straight_through": self.straight_through}


__all__ = ["LayerSelector", "rms_norm"]
