"""LayerSelector: which candidate reader layers a token's update is written at, and how strongly
(the API of xenc/selector.py:36-118).

Per forward the selector reads the RMS-normed residual at its first candidate layer once and
keeps per-token weights w [B, T, n_cand]: the k largest logits u(hn0) keep a softmax over
themselves, every other layer gets 0 (straight_through: 1/k on the kept layers in the forward,
the dense softmax's gradient in the backward).  A layer's update delta is rescaled so that
|delta| / |h| = w_l * alpha per token (`matched_norm`), i.e. the selection decides where to
write, alpha how much.

Weights are recomputed at the first candidate layer of every forward unless `compute` set them
for it, so T = 1 decode steps never reuse stale weights.  Ties between equal logits go to the
lower layer on every path (the HIP kernel and the torch code below share that order).
`selected_rows` tells the injector which token rows give a layer a nonzero weight, so it can
skip the read of the others without a host synchronisation.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

_EPS = 1e-6


def rms_norm(x: torch.Tensor, eps: float = _EPS) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) over the last dim, in fp32 (no weight).  The reference imports
    this from an external package that is absent; eps = 1e-6 follows the reference's own copies
    (xenc/hyb_hm.py:37-38, xenc/p5_copy.py:99-101)."""
    x = x.float()
    return x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + eps)


def _here(t: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    return t if t.device == x.device else t.to(x.device)


def topk_lower_first(z: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest entries of the last dim in rank order; equal values rank by the
    lower index (a stable descending sort)."""
    return torch.sort(z, dim=-1, descending=True, stable=True).indices[..., :k]


class _HardKeptSoftGrad(torch.autograd.Function):
    """Forward: 1/k on the kept entries, 0 elsewhere.  Backward: the Jacobian of the dense
    softmax of z (the straight-through estimator of the reference's selector)."""

    @staticmethod
    def forward(ctx, z, kept):
        k = kept.shape[-1]
        soft = torch.softmax(z, dim=-1)
        ctx.save_for_backward(soft)
        return torch.zeros_like(z).scatter(-1, kept, 1.0 / k)

    @staticmethod
    def backward(ctx, g):
        (soft,) = ctx.saved_tensors
        return soft * (g - (g * soft).sum(-1, keepdim=True)), None


def sparse_weights(z: torch.Tensor, k: int, straight_through: bool = False) -> torch.Tensor:
    """Selector weights from logits z [..., n] on the torch path (differentiable in z)."""
    kept = topk_lower_first(z, k)
    if straight_through:
        return _HardKeptSoftGrad.apply(z, kept)
    return torch.zeros_like(z).scatter(-1, kept, torch.softmax(z.gather(-1, kept), dim=-1))


def matched_norm(delta: torch.Tensor, h: torch.Tensor, w_l: torch.Tensor, log_alpha: torch.Tensor) -> torch.Tensor:
    """w_l * alpha * delta / (|delta| / (|h| + 1e-6) + 1e-6) per token, in fp32."""
    d = delta.float()
    rel = torch.linalg.vector_norm(d, dim=-1, keepdim=True) / (
        torch.linalg.vector_norm(h.float(), dim=-1, keepdim=True) + _EPS)
    scale = _here(w_l, d).to(d.dtype)[..., None] * torch.exp(_here(log_alpha, d)) / (rel + _EPS)
    return scale * d


class LayerSelector(nn.Module):
    def __init__(self, d_m: int, cand_layers: list[int], k: int = 2, alpha_init: float = 0.02,
                 straight_through: bool = False):
        super().__init__()
        layers = [int(li) for li in cand_layers]
        repeated = sorted({li for li in layers if layers.count(li) > 1})
        if repeated:
            raise ValueError(f"candidate layers {repeated} appear more than once")
        if k < 1 or k > len(layers):
            raise ValueError(f"k={k} is outside 1..{len(layers)} (the number of candidate layers)")
        if not alpha_init > 0:
            raise ValueError(f"alpha_init={alpha_init} must be positive")
        self.d_m, self.k = int(d_m), int(k)
        self.cand_layers = sorted(layers)
        self.n_cand = len(self.cand_layers)
        self.pos = {li: j for j, li in enumerate(self.cand_layers)}
        self.first_layer = self.cand_layers[0]
        self.straight_through = bool(straight_through)
        self.u = nn.Linear(self.d_m, self.n_cand, bias=True)
        self.log_alpha = nn.Parameter(torch.tensor(math.log(alpha_init)))
        self._w: torch.Tensor | None = None
        self._explicit = False       # compute() ran for the forward that has not reached its first layer yet

    # ---------------------------------------------------------------- weights
    def _weights_from_logits(self, z: torch.Tensor) -> torch.Tensor:
        needs_grad = torch.is_grad_enabled() and z.requires_grad
        if (z.is_cuda and z.dtype == torch.float32 and z.shape[-1] <= 256 and not self.straight_through
                and not needs_grad):
            from .ops import selector_weights          # HIP xenc_selector_weights, same tie order
            w, _, _ = selector_weights(z.reshape(-1, z.shape[-1]).contiguous(), self.k)
            return w.view(z.shape)
        return sparse_weights(z, self.k, self.straight_through)

    def compute(self, hn0: torch.Tensor) -> None:
        """Set this forward's weights from hn0 [B, T, d_m], the RMS-normed residual at the first
        candidate layer."""
        x = hn0.to(self.u.weight.dtype)
        self._w = self._weights_from_logits(F.linear(x, _here(self.u.weight, x), _here(self.u.bias, x)))
        self._explicit = True

    def reset(self) -> None:
        self._w, self._explicit = None, False

    def weights(self) -> torch.Tensor | None:
        return self._w

    @torch.no_grad()
    def entropy(self) -> torch.Tensor | None:
        """Mean per-token entropy (nats) of the current weights; None before they exist."""
        if self._w is None:
            return None
        p = self._w.detach().float().clamp_min(0)
        return -(p * p.clamp_min(1e-12).log()).sum(-1).mean()

    def alpha(self) -> torch.Tensor:
        return self.log_alpha.exp()

    def _current(self, h: torch.Tensor, li: int) -> torch.Tensor:
        """The weights for layer li's call in this forward, computed from rms_norm(h) when the
        forward starts (first candidate layer, unless compute() already ran for it) or when none
        fit h's batch shape (hooks entered past the first candidate layer)."""
        starting = li == self.first_layer
        stale = self._w is None or (not starting and self._w.shape[:-1] != h.shape[:-1])
        if (starting and not self._explicit) or stale:
            self.compute(rms_norm(h))
        if starting or stale:
            self._explicit = False
        return self._w

    # ---------------------------------------------------------------- use
    def selected_rows(self, h: torch.Tensor, li: int) -> torch.Tensor:
        """Bool [B, T]: the token rows whose weight for layer li is nonzero.  At the first
        candidate layer this fixes the forward's weights, and the same layer's apply() reuses
        them."""
        col = self.pos[li]
        w = self._current(h, li)
        if li == self.first_layer:
            self._explicit = True
        return w[..., col] != 0

    def apply(self, delta: torch.Tensor, h: torch.Tensor, li: int) -> torch.Tensor:
        """Layer li's update rescaled to the matched norm and weighted; delta's dtype."""
        col = self.pos[li]                  # KeyError for a layer that is not a candidate
        w = self._current(h, li)
        grad = torch.is_grad_enabled() and (delta.requires_grad or self.log_alpha.requires_grad
                                            or w.requires_grad)
        if delta.is_cuda and not grad:
            from .ops import selector_apply   # HIP xenc_selector_apply
            shape = delta.shape
            out = selector_apply(delta.float().reshape(-1, shape[-1]).contiguous(),
                                 h.float().reshape(-1, shape[-1]).contiguous(),
                                 _here(w[..., col], delta).reshape(-1).float().contiguous(), self.log_alpha, k=1)
            return out.view(shape).to(delta.dtype)
        return matched_norm(delta, h, w[..., col], self.log_alpha).to(delta.dtype)

    def extra_repr(self) -> str:
        return (f"d_m={self.d_m}, cand_layers={self.cand_layers}, k={self.k}, "
                f"straight_through={self.straight_through}")

    def config(self) -> dict:
        return {"d_m": self.d_m, "cand_layers": list(self.cand_layers), "k": self.k,
                "straight_through": self.straight_through}


__all__ = ["LayerSelector", "rms_norm", "sparse_weights", "matched_norm", "topk_lower_first"]
