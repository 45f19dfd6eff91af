"""Reader-side injectors: forward hooks that add the Library read to a reader's residual stream.

LibraryInjector keeps the API of xenc/injector.py:121-273: per-token routing over the chunk
summary keys (optional top-k), the masked per-chunk read, the route-weighted merge, the
gate * gain * B write-back, an optional LayerSelector, and the bookkeeping (mag_terms, last_route,
route_terms, record_attn / last_attn, force_attn / force_norm_match, training_attn / attn_pos /
attn_terms).  The routing and the read run in the HIP kernels of kv_skill_v2_amd.ops:
    route_rows  -> route_topk_kernel (no grad) or RouteFn (route kernel + route backward)
    read_rows   -> the split-K decode kernel (few rows, no grad) or ReadFn (MFMA prefill read and
                   its dQ backward)
The query map, RMS norm, gate, gain and B projection stay in torch around them, as in the
reference.  The diagnostics that expose or replace the [C, N] slot attention (record_attn,
training_attn, force_attn) compute that one [C, N] map with torch on the device from the
Library's fp32 K.

XEncInjector is the single-skill path (xenc/injector.py:80-118): one skill is read as a one-chunk
Library (routing over one chunk gives w = 1 exactly).

The hook plumbing (`enabled`, `_handles`, `mag_terms`, `detach`, `gain_scale`, `calib`,
`_pos_mask`) is the contract of the base injector the reference subclasses from an external
package; it is restated in `SkillInjector`.  No position mask is applied (`_pos_mask` returns
None) and gain_scale defaults to 1.0.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .depth import KVSkill, decoder_layers, for_reader
from .interface import ModelInterface
from .library import PAGE_ALIGN, Library
from .selector import rms_norm


def _on(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """`t` on like's device; the same object when it is already there."""
    return t if t.device == like.device else t.to(like.device)


def _linear(mod: nn.Module, x: torch.Tensor) -> torch.Tensor:
    if isinstance(mod, nn.Sequential):
        for m in mod:
            x = _linear(m, x)
        return x
    b = None if mod.bias is None else _on(mod.bias, x)
    return F.linear(x, _on(mod.weight, x), b)


# The fused write-back kernel serves the decode path (few rows, no autograd); many rows go to
# the library GEMM, whose W reuse across rows the kernel does not have.
_FUSED_WRITE_ROWS = 64


def write_delta(itf, hn: torch.Tensor, r: torch.Tensor, li: int, gain_scale: float,
                gcal=1.0) -> torch.Tensor:
    """delta = gain_scale * gain * gcal * gate * B(r) (xenc/injector.py:266-267).  On the decode
    path (a ModelInterface with an fp32 linear B, at most 64 rows, nothing requiring grad) the
    product runs as one xenc_write_back launch: B streamed once with gate * gain folded into a
    per-row scale."""
    Bm = getattr(itf, "B", None) if isinstance(itf, ModelInterface) else None
    rows = r.numel() // r.shape[-1]
    grad = torch.is_grad_enabled() and (
        r.requires_grad or hn.requires_grad
        or (isinstance(itf, nn.Module) and any(p.requires_grad for p in itf.parameters()))
        or (isinstance(gcal, torch.Tensor) and gcal.requires_grad))
    fused = (isinstance(Bm, nn.Linear) and r.is_cuda and r.dtype == torch.float32
             and Bm.weight.dtype == torch.float32 and rows <= _FUSED_WRITE_ROWS
             and r.shape[-1] % 4 == 0 and not grad and isinstance(gcal, (int, float)))
    if not fused:
        return gain_scale * itf_gain(itf, li, hn) * gcal * itf_gate(itf, hn, li) * itf_write(itf, r)
    # gain_scale * gcal * exp(log_gain[p]) * sigmoid(hn . gate_w + gate_b[p]) per row on
    # xenc_gate_scale, then B streamed once with that scale folded in (xenc_write_back).
    p = itf._pos[li]
    scale = ops.gate_scale(hn.reshape(rows, hn.shape[-1]).float().contiguous(), _on(itf.gate_w, r),
                           _on(itf.gate_b, r)[p:p + 1], _on(itf.log_gain, r)[p:p + 1],
                           float(gain_scale) * float(gcal))
    W = _on(Bm.weight, r).contiguous()
    b = None if Bm.bias is None else _on(Bm.bias, r).float().contiguous()
    out = ops.write_back(r.reshape(rows, r.shape[-1]).contiguous(), W, None, b, scale)
    return out.view(*r.shape[:-1], W.shape[0])


def itf_query(itf, hn: torch.Tensor) -> torch.Tensor:
    if not isinstance(itf, ModelInterface):
        return itf.query(hn)
    q = _linear(itf.A, hn)
    return q / (q.norm(dim=-1, keepdim=True) + 1e-6)


def itf_gate(itf, hn: torch.Tensor, li: int) -> torch.Tensor:
    if not isinstance(itf, ModelInterface):
        return itf.gate(hn, li)
    return torch.sigmoid(hn @ _on(itf.gate_w, hn) + _on(itf.gate_b, hn)[itf._pos[li]]).unsqueeze(-1)


def itf_gain(itf, li: int, like: torch.Tensor) -> torch.Tensor:
    if not isinstance(itf, ModelInterface):
        return _on(itf.gain(li), like)
    return _on(itf.log_gain, like)[itf._pos[li]].exp()


def itf_write(itf, r: torch.Tensor) -> torch.Tensor:
    if not isinstance(itf, ModelInterface):
        return itf.write(r)
    return _linear(itf.B, r)


class SkillInjector:
    """Hook plumbing: one forward hook per injection layer adds `_branch(h, li)` to the layer's
    output hidden state and records mean ||delta|| / ||h|| in `mag_terms`."""

    def __init__(self, model: nn.Module, interface, read_fp32: bool = True, read_softmax: bool = True,
                 read_temp: float = 12.0, gain_scale: float = 1.0):
        self.model, self.itf = model, interface
        self.read_fp32, self.read_softmax, self.read_temp = bool(read_fp32), bool(read_softmax), float(read_temp)
        self.gain_scale = float(gain_scale)
        self.calib = None
        self.enabled = True
        self.skill = None
        self.mag_terms: list = []
        self._handles: list = []
        self._attach()

    def _active(self) -> bool:
        return self.enabled and self.skill is not None

    def _pos_mask(self, h: torch.Tensor):
        return None

    def _hook(self, li: int):
        def hook(mod, args, output):
            if not self._active():
                return output
            is_tuple = isinstance(output, tuple)
            h = output[0] if is_tuple else output
            delta = self._branch(h, li).to(h.dtype)
            mask = self._pos_mask(h)
            if mask is not None:
                delta = delta * mask
            rel = delta.float().norm(dim=-1) / (h.float().norm(dim=-1) + 1e-6)
            self.mag_terms.append(rel.mean())
            h = h + delta
            return (h,) + tuple(output[1:]) if is_tuple else h
        return hook

    def _attach(self) -> None:
        blocks = decoder_layers(self.model)
        for li in self.itf.inject_layers:
            self._handles.append(blocks[li].register_forward_hook(self._hook(li)))

    def detach(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles.clear()

    def load(self, skill) -> None:
        self.skill = skill

    def unload(self) -> None:
        self.skill = None
        self.mag_terms.clear()


class XEncInjector(SkillInjector):
    def load(self, skill: KVSkill) -> None:
        if skill.meta.get("keyed_by") == "rho":
            skill = for_reader(skill, self.model)
        if skill.d_s != self.itf.d_s:
            raise ValueError(f"skill d_s={skill.d_s} (encoder) != interface d_s={self.itf.d_s}")
        missing = set(self.itf.inject_layers) - set(skill.K)
        if missing:
            raise KeyError(f"skill has no operator for reader layers {sorted(missing)}")
        self._skill_pool = {}
        super().load(skill)

    def _skill_kv(self, li: int, like: torch.Tensor):
        """Skill K / V of layer li on like's device (moved once, cached in the loaded skill)."""
        K, V = self.skill.K[li], self.skill.V[li]
        if K.device != like.device:
            K = self.skill.K[li] = K.to(like.device)
        if V.device != like.device:
            V = self.skill.V[li] = V.to(like.device)
        return K, V

    def _skill_paged(self, li: int, like: torch.Tensor):
        """The skill of layer li as a one-chunk HIP read pool (all rows valid)."""
        key = (li, like.device)
        pl = self._skill_pool.get(key)
        if pl is None:
            K, V = self._skill_kv(li, like)
            K3 = K.float().unsqueeze(0)
            M = torch.ones(K3.shape[:2], dtype=torch.bool, device=K3.device)
            S = K3[0].mean(0, keepdim=True)
            pl = ops.PagedLibrary.from_padded(K3, M, S, device=like.device,
                                              V=None if V is K else V.float().unsqueeze(0), pad_to=PAGE_ALIGN)
            self._skill_pool[key] = pl
        return pl

    def _branch(self, h: torch.Tensor, li: int) -> torch.Tensor:
        """delta = gain_scale * gain * gate * B(read), the read over all skill rows."""
        hn = rms_norm(h.float())
        q = itf_query(self.itf, hn)
        B_, T_, d = q.shape
        r, _ = ops.branch_read(q.reshape(B_ * T_, d), self._skill_paged(li, hn), 0, self.read_temp,
                               1.0, self.read_softmax)
        r = r.view(B_, T_, d)
        gcal = 1.0
        if self.calib is not None and li in self.calib:
            r = r * _on(self.calib[li]["scale"], r)
            gcal = self.calib[li]["gain"]
            if isinstance(gcal, torch.Tensor):
                gcal = _on(gcal, r)
        return write_delta(self.itf, hn, r, li, self.gain_scale, gcal)


class LibraryInjector(XEncInjector):
    def __init__(self, model, interface, read_softmax: bool = True, read_temp: float = 12.0,
                 route_temp: float = 10.0, top_k: int = 0, selector=None, read_fp32: bool = True):
        self.lib: Library | None = None
        self.route_temp = float(route_temp)
        self.top_k = int(top_k)
        self.selector = selector
        self.last_route: torch.Tensor | None = None
        self.record_attn = False       # keep the [C, N] attention of the last position per layer
        self.last_attn: dict = {}
        self.force_attn = None         # a [C, N] map (or {li: [C, N]}) replacing the attention
        self.force_norm_match = False  # rescale the forced read per token to the computed read's norm
        self.training_attn = False     # keep aw[0, attn_pos] with grad per hooked layer
        self.attn_pos: int = -1
        self.attn_terms: list = []
        self.route_terms: list = []
        super().__init__(model, interface, read_fp32=read_fp32, read_softmax=read_softmax,
                         read_temp=read_temp)

    # ------------------------------------------------------------------ load / unload
    def load(self, skill: KVSkill) -> None:
        self.lib = None
        super().load(skill)

    def load_library(self, lib: Library) -> None:
        if lib.d_s != self.itf.d_s:
            raise ValueError(f"library d_s={lib.d_s} (encoder) != interface d_s={self.itf.d_s}")
        missing = set(self.itf.inject_layers) - set(lib.K)
        if missing:
            raise KeyError(f"library has no operator for reader layers {sorted(missing)}")
        dtype = torch.float32 if self.read_fp32 else next(self.model.parameters()).dtype
        self.skill = None
        self.lib = lib.to(self.model.device, dtype)

    def unload(self) -> None:
        """Unload and clear the per-forward bookkeeping."""
        self.skill = None
        self.lib = None
        self.mag_terms.clear()
        self.route_terms.clear()
        self.attn_terms.clear()
        self.last_route = None

    # ------------------------------------------------------------------ hooks
    def _active(self) -> bool:
        return self.enabled and (self.skill is not None or self.lib is not None)

    def _attach(self) -> None:
        blocks = decoder_layers(self.model)

        def pre(mod, args):          # start of every forward (each decode step included)
            if self.selector is not None:
                self.selector.reset()

        self._handles.append(blocks[self.itf.inject_layers[0]].register_forward_pre_hook(pre))
        super()._attach()

    # ------------------------------------------------------------------ library tensors
    def _lib_layer(self, li: int, like: torch.Tensor):
        """(K, mask, S) of layer li on like's device, moved once and cached in the Library."""
        lib = self.lib
        if lib.K[li].device != like.device:
            lib.K[li] = lib.K[li].to(like.device)
            lib.mask[li] = lib.mask[li].to(like.device)
            lib.S[li] = lib.S[li].to(like.device)
        return lib.K[li], lib.mask[li], lib.S[li]

    def _lib_values(self, li: int, like: torch.Tensor) -> torch.Tensor:
        lib = self.lib
        if lib.V is None:
            return self._lib_layer(li, like)[0]
        if lib.V[li].device != like.device:
            lib.V[li] = lib.V[li].to(like.device)
        return lib.V[li]

    def _pool(self, li: int, like: torch.Tensor):
        return self.lib.paged(li, like.device)

    # ------------------------------------------------------------------ route / read
    def route(self, q: torch.Tensor, li: int) -> torch.Tensor:
        """Routing weights [B, T, C] over the chunks: sum to 1, exactly top_k nonzeros if set."""
        pl = self._pool(li, q)
        B_, T_, d = q.shape
        w, _, _ = ops.route_rows(q.reshape(B_ * T_, d), pl, self.top_k, self.route_temp)
        return w.view(B_, T_, -1)

    def _attn_rows(self, q_rows: torch.Tensor, w_rows: torch.Tensor, li: int) -> torch.Tensor:
        """aw [R, C, N] = (masked softmax or linear read weights) * w for a few rows (torch)."""
        K, M, _ = self._lib_layer(li, q_rows)
        a = torch.einsum("rd,cnd->rcn", q_rows.to(K.dtype), K)
        if self.read_softmax:
            a = torch.softmax((a * self.read_temp).masked_fill(~M, float("-inf")), -1)
        else:
            n = M.sum(-1).to(a.dtype).clamp_min(1)
            a = a.masked_fill(~M, 0.0) / n.sqrt().view(1, -1, 1)
        return a * w_rows.to(a.dtype).unsqueeze(-1)

    def _forced(self, li: int, like: torch.Tensor, r: torch.Tensor) -> tuple:
        """(r, fa, scale): the read under force_attn.  fa [C, N] replaces the attention of every
        token; with force_norm_match each token's forced map is scaled by scale [B, T, 1] =
        ||computed read|| / (||forced read|| + 1e-6), both reads taken with K as values."""
        fa = self.force_attn.get(li) if isinstance(self.force_attn, dict) else self.force_attn
        K, M, _ = self._lib_layer(li, like)
        fa = _on(fa, K).to(K.dtype)
        if fa.shape != M.shape:
            raise ValueError(f"force_attn {tuple(fa.shape)} != library [C,N] {tuple(M.shape)}")
        Vt = self._lib_values(li, like)
        out = (fa.reshape(-1) @ Vt.reshape(-1, Vt.shape[-1])).expand_as(r).to(r.dtype)
        scale = None
        if self.force_norm_match:
            r0 = r
            if self.lib.V is not None:   # the computed read's norm is taken with K as values
                pl = self._pool(li, like)
                tied = ops.PagedLibrary(pl.pages, pl.chunk_page, pl.chunk_nvalid, pl.chunk_ptr, pl.S,
                                        n_chunks=pl.n_chunks, nvalid=pl.nvalid, d_valid=pl.d_valid)
                r0 = self._read_all(self._last_q, li, tied)[0]
            k1 = fa.reshape(-1) @ K.reshape(-1, K.shape[-1])
            scale = r0.norm(dim=-1, keepdim=True) / (k1.norm() + 1e-6)
            out = out * scale.to(out.dtype)
        return out, fa, scale

    def _read_all(self, q: torch.Tensor, li: int, pl, rows: torch.Tensor | None = None):
        """(r [B, T, d], w [B, T, C]); with `rows` (bool [B, T]) only those rows are read, the
        others get r = 0 (their update is multiplied by an exact 0 afterwards)."""
        B_, T_, d = q.shape
        q2 = q.reshape(B_ * T_, d)
        w, idx, wsel = ops.route_rows(q2, pl, self.top_k, self.route_temp)
        if rows is None:
            r = ops.read_rows(q2, w, idx, wsel, pl, self.read_temp, self.read_softmax)
        else:
            sel = rows.reshape(-1).nonzero().squeeze(1)
            r = torch.zeros(B_ * T_, d, dtype=torch.float32, device=q.device)
            if sel.numel():
                rs = ops.read_rows(q2.index_select(0, sel), w.index_select(0, sel), idx.index_select(0, sel),
                                   wsel.index_select(0, sel), pl, self.read_temp, self.read_softmax)
                r = r.index_copy(0, sel, rs)
        return r.view(B_, T_, d), w.view(B_, T_, -1)

    def _branch(self, h: torch.Tensor, li: int) -> torch.Tensor:
        if self.lib is None:                               # single-skill path
            delta = super()._branch(h, li)
        else:
            hn = rms_norm(h.float())
            q = itf_query(self.itf, hn)                    # [B, T, d_s]
            pl = self._pool(li, hn)
            diag = self.force_attn is not None or self.record_attn or (
                self.training_attn and torch.is_grad_enabled())
            rows = None
            if self.selector is not None and hasattr(self.selector, "selected_rows") and not diag:
                rows = self.selector.selected_rows(h, li)
            self._last_q = q
            r, w = self._read_all(q, li, pl, rows)
            fa = scale = None
            if self.force_attn is not None:
                r, fa, scale = self._forced(li, hn, r)
            if self.record_attn or (self.training_attn and torch.is_grad_enabled()):
                pos = [q.shape[1] - 1, self.attn_pos]
                if fa is None:
                    aw2 = self._attn_rows(q[0, pos], w[0, pos], li)
                else:
                    aw2 = fa.unsqueeze(0).expand(2, *fa.shape)
                    if scale is not None:
                        aw2 = aw2 * scale[0, pos].to(fa.dtype).view(2, 1, 1)
                last, at = aw2[0], aw2[1]
                if self.record_attn:
                    self.last_attn[li] = last.detach().float().cpu()
                if self.training_attn and torch.is_grad_enabled():
                    self.attn_terms.append(at.float())
            self._last_q = None
            delta = write_delta(self.itf, hn, r, li, self.gain_scale)
            self.last_route = w.detach()
            if torch.is_grad_enabled():
                self.route_terms.append((li, w))
        if self.selector is not None:
            delta = self.selector.apply(delta, h, li)
        return delta


__all__ = ["SkillInjector", "XEncInjector", "LibraryInjector", "itf_query", "itf_gate", "itf_gain",
           "itf_write", "write_delta", "rms_norm"]
