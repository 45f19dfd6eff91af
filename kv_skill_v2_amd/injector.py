"""Reader-side injectors: forward hooks that add the Library read to a reader's residual stream.

LibraryInjector keeps the API of xenc/injector.py:121-273 (constructor, load_library / unload,
route, _branch, and the bookkeeping attributes mag_terms, last_route, route_terms, record_attn /
last_attn, force_attn / force_norm_match, training_attn / attn_pos / attn_terms) and
XEncInjector the single-skill API (xenc/injector.py:80-118).  The work of one hooked layer runs
in three stages:

    query      hn = rms_norm(h), q = the interface's query map of hn                  (torch)
    read       routing over the chunk summaries, then the masked per-chunk read of the routed
               pages merged by the route weights                                       (HIP)
    update     delta = gain_scale * gain * gate * B(r), then the LayerSelector if set  (HIP on
               the decode path, torch with autograd)

The read goes through torch.ops.xenc: few rows without autograd take the split-K decode
operators (xenc::route_topk, xenc::library_read), many rows or autograd the MFMA operators
(xenc::route_rows, xenc::library_prefill_fwd, both differentiable).  With a LayerSelector the
rows a layer does not select are not read: their routed-chunk lists are emptied on the device
(index -1), so the read returns 0 for them without a host synchronisation, and their update is
multiplied by the selector's exact 0 afterwards.

The diagnostics that expose or replace the [C, N] slot attention (record_attn, training_attn,
force_attn) compute that one map with torch on the device from the Library's K.

The base class SkillInjector carries the hook contract of the external package the reference
subclasses (enabled, _handles, mag_terms, detach, gain_scale, calib, _pos_mask): no position mask
is applied (`_pos_mask` returns None) and gain_scale defaults to 1.0.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import ops
from .depth import KVSkill, decoder_layers, for_reader
from .interface import ModelInterface, apply_map
from .library import PAGE_ALIGN, Library
from .selector import rms_norm


def _here(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if t.device == like.device else t.to(like.device)


# ----------------------------------------------------------------------------- interface calls
# An interface is any object with query(hn), gate(hn, li), gain(li) and write(r); ModelInterface's
# methods bring their weights to the input's device themselves.
def itf_query(itf, hn: torch.Tensor) -> torch.Tensor:
    return itf.query(hn)


def itf_gate(itf, hn: torch.Tensor, li: int) -> torch.Tensor:
    return itf.gate(hn, li)


def itf_gain(itf, li: int, like: torch.Tensor) -> torch.Tensor:
    return _here(itf.gain(li), like)


def itf_write(itf, r: torch.Tensor) -> torch.Tensor:
    return itf.write(r)


# The fused write-back serves the decode path (few rows, no autograd); many rows go to the
# library GEMM, whose reuse of B across rows the kernel does not have.
_FUSED_WRITE_ROWS = 64


def _needs_grad(itf, *tensors) -> bool:
    if not torch.is_grad_enabled():
        return False
    if any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors):
        return True
    return isinstance(itf, nn.Module) and any(p.requires_grad for p in itf.parameters())


def write_delta(itf, hn: torch.Tensor, r: torch.Tensor, li: int, gain_scale: float,
                gcal=1.0) -> torch.Tensor:
    """delta = gain_scale * gain * gcal * gate * B(r) (xenc/injector.py:266-267).  On the decode
    path (a ModelInterface with a plain linear B in fp32, at most 64 rows, nothing requiring grad)
    it is one HIP row scale (xenc_gate_scale) and one write-back launch that streams B once with
    the scale folded in (xenc_write_back)."""
    rows = r.numel() // r.shape[-1]
    B = itf.B if isinstance(itf, ModelInterface) else None
    fused = (isinstance(B, nn.Linear) and r.is_cuda and r.dtype == torch.float32 and B.weight.dtype == torch.float32
             and rows <= _FUSED_WRITE_ROWS and r.shape[-1] % 4 == 0 and isinstance(gcal, (int, float))
             and not _needs_grad(itf, r, hn))
    if not fused:
        return gain_scale * itf_gain(itf, li, hn) * gcal * itf_gate(itf, hn, li) * itf_write(itf, r)
    p = itf._pos[li]
    scale = ops.gate_scale(hn.reshape(rows, hn.shape[-1]).float().contiguous(), _here(itf.gate_w, r),
                           _here(itf.gate_b, r)[p:p + 1], _here(itf.log_gain, r)[p:p + 1],
                           float(gain_scale) * float(gcal))
    bias = None if B.bias is None else _here(B.bias, r).float().contiguous()
    out = ops.write_back(r.reshape(rows, r.shape[-1]).contiguous(), _here(B.weight, r).contiguous(), None,
                         bias, scale)
    return out.view(*r.shape[:-1], B.weight.shape[0])


# ----------------------------------------------------------------------------- hooks
class _AddUpdate:
    """Forward hook of one injection layer: the layer's output hidden state plus the branch's
    update, recording mean |delta| / |h| in the injector's mag_terms."""

    def __init__(self, owner: "SkillInjector", li: int):
        self.owner, self.li = owner, li

    def __call__(self, module, args, output):
        inj = self.owner
        if not inj._active():
            return output
        packed = isinstance(output, tuple)
        h = output[0] if packed else output
        delta = inj._branch(h, self.li).to(h.dtype)
        mask = inj._pos_mask(h)
        if mask is not None:
            delta = delta * mask
        ratio = torch.linalg.vector_norm(delta.float(), dim=-1) / (torch.linalg.vector_norm(h.float(), dim=-1) + 1e-6)
        inj.mag_terms.append(ratio.mean())
        out = h + delta
        return (out, *output[1:]) if packed else out


class _ResetSelector:
    """Forward pre-hook on the first injection layer: a new forward starts, so the selector's
    weights of the previous one are dropped (each decode step recomputes them)."""

    def __init__(self, owner: "LibraryInjector"):
        self.owner = owner

    def __call__(self, module, args):
        if self.owner.selector is not None:
            self.owner.selector.reset()


class SkillInjector:
    """Hook contract: one forward hook per injection layer of the interface."""

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

    def _attach(self) -> None:
        blocks = decoder_layers(self.model)
        self._handles.extend(blocks[li].register_forward_hook(_AddUpdate(self, li)) for li in self.itf.inject_layers)

    def detach(self) -> None:
        while self._handles:
            self._handles.pop().remove()

    def load(self, skill) -> None:
        self.skill = skill

    def unload(self) -> None:
        self.skill = None
        self.mag_terms.clear()

    def _query(self, h: torch.Tensor):
        hn = rms_norm(h)
        return hn, itf_query(self.itf, hn)


class XEncInjector(SkillInjector):
    """One skill read as a one-chunk Library: routing over a single chunk gives w = 1 exactly, so
    the read is softmax(read_temp q K^T) V over every skill row."""

    def load(self, skill: KVSkill) -> None:
        if skill.meta.get("keyed_by") == "rho":
            skill = for_reader(skill, self.model)
        if skill.d_s != self.itf.d_s:
            raise ValueError(f"the skill has d_s={skill.d_s} (its encoder), the interface d_s={self.itf.d_s}")
        uncovered = sorted(set(self.itf.inject_layers) - set(skill.K))
        if uncovered:
            raise KeyError(f"the skill holds no operator for reader layers {uncovered}")
        self._skill_pools = {}
        super().load(skill)

    def _skill_pool(self, li: int, device) -> ops.PagedLibrary:
        """The skill of layer li as a one-chunk read pool on `device` (built once per load)."""
        key = (li, device)
        pool = self._skill_pools.get(key)
        if pool is None:
            K, V = self.skill.K[li], self.skill.V[li]
            K3 = K.float()[None]
            mask = torch.ones(K3.shape[:2], dtype=torch.bool, device=K3.device)
            pool = ops.PagedLibrary.from_padded(K3, mask, K3[0].mean(0, keepdim=True), device=device,
                                                V=None if V is K else V.float()[None], pad_to=PAGE_ALIGN)
            self._skill_pools[key] = pool
        return pool

    def _calibrated(self, r: torch.Tensor, li: int):
        """(r, gcal) after the optional per-layer calibration {li: {"scale", "gain"}}."""
        if self.calib is None or li not in self.calib:
            return r, 1.0
        cal = self.calib[li]
        g = cal["gain"]
        return r * _here(cal["scale"], r), (_here(g, r) if isinstance(g, torch.Tensor) else g)

    def _branch(self, h: torch.Tensor, li: int) -> torch.Tensor:
        hn, q = self._query(h)
        lead, d = q.shape[:-1], q.shape[-1]
        r, _ = ops.branch_read(q.reshape(-1, d), self._skill_pool(li, hn.device), 0, self.read_temp, 1.0,
                               self.read_softmax)
        r, gcal = self._calibrated(r.view(*lead, -1), li)
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
        self.training_attn = False     # keep the [C, N] attention at attn_pos with grad per hooked layer
        self.attn_pos: int = -1
        self.attn_terms: list = []
        self.route_terms: list = []
        self._dense_cache: dict = {}
        super().__init__(model, interface, read_fp32=read_fp32, read_softmax=read_softmax,
                         read_temp=read_temp)

    # ------------------------------------------------------------------ load / unload
    def load(self, skill: KVSkill) -> None:
        self.lib = None
        super().load(skill)

    def load_library(self, lib: Library) -> None:
        if lib.d_s != self.itf.d_s:
            raise ValueError(f"the library has d_s={lib.d_s} (its encoder), the interface d_s={self.itf.d_s}")
        uncovered = sorted(set(self.itf.inject_layers) - set(lib.K))
        if uncovered:
            raise KeyError(f"the library holds no operator for reader layers {uncovered}")
        dtype = torch.float32 if self.read_fp32 else next(self.model.parameters()).dtype
        self.skill = None
        self._dense_cache = {}
        self.lib = lib.to(self.model.device, dtype)

    def unload(self) -> None:
        """Unload and clear the per-forward bookkeeping."""
        self.skill = self.lib = self.last_route = None
        self._dense_cache = {}
        for log in (self.mag_terms, self.route_terms, self.attn_terms):
            log.clear()

    # ------------------------------------------------------------------ hooks
    def _active(self) -> bool:
        return self.enabled and (self.skill is not None or self.lib is not None)

    def _attach(self) -> None:
        first = decoder_layers(self.model)[self.itf.inject_layers[0]]
        self._handles.append(first.register_forward_pre_hook(_ResetSelector(self)))
        super()._attach()

    # ------------------------------------------------------------------ library tensors
    def _pool(self, li: int, like: torch.Tensor) -> ops.PagedLibrary:
        return self.lib.paged(li, like.device)

    def _dense(self, li: int, device) -> tuple:
        """(K, mask, V) of layer li on `device` for the torch diagnostics (V is K when tied)."""
        key = (li, device)
        if key not in self._dense_cache:
            K = self.lib.K[li].to(device)
            M = self.lib.mask[li].to(device)
            V = K if self.lib.V is None else self.lib.V[li].to(device)
            self._dense_cache[key] = (K, M, V)
        return self._dense_cache[key]

    # ------------------------------------------------------------------ route / read
    def route(self, q: torch.Tensor, li: int) -> torch.Tensor:
        """Routing weights [B, T, C] over the chunks: sum to 1, exactly top_k nonzeros if set."""
        w, _, _ = ops.route_rows(q.reshape(-1, q.shape[-1]), self._pool(li, q), self.top_k, self.route_temp)
        return w.view(*q.shape[:-1], -1)

    def _read(self, q: torch.Tensor, pool: ops.PagedLibrary, keep: torch.Tensor | None = None):
        """(r [B, T, d], w [B, T, C]).  keep (bool [B, T], device): rows left out read nothing and
        get r = 0 (their routed-chunk lists are emptied on the device)."""
        lead, d = q.shape[:-1], q.shape[-1]
        rows = q.reshape(-1, d)
        if keep is None or (torch.is_grad_enabled() and rows.requires_grad):
            # (with autograd every row is read: the selector's weight zeroes the left-out ones)
            r, w = ops.branch_read(rows, pool, self.top_k, self.read_temp, self.route_temp, self.read_softmax)
            return r.view(*lead, -1), w.view(*lead, -1)
        w, idx, w_sel = ops.route_rows(rows, pool, self.top_k, self.route_temp)
        idx = torch.where(keep.reshape(-1, 1), idx, torch.full_like(idx, -1))
        r = ops.read_rows(rows, w, idx, w_sel, pool, self.read_temp, self.read_softmax)
        return r.view(*lead, -1), w.view(*lead, -1)

    def _slot_attention(self, q_rows: torch.Tensor, w_rows: torch.Tensor, li: int) -> torch.Tensor:
        """Route-weighted slot attention [R, C, N] of a few query rows (torch)."""
        K, M, _ = self._dense(li, q_rows.device)
        s = torch.einsum("rd,cnd->rcn", q_rows.to(K.dtype), K)
        if self.read_softmax:
            a = torch.softmax((s * self.read_temp).masked_fill(~M, float("-inf")), dim=-1)
        else:
            n = M.sum(-1).to(s.dtype).clamp_min(1)
            a = s.masked_fill(~M, 0.0) / n.sqrt()[None, :, None]
        return a * w_rows.to(a.dtype)[..., None]

    def _forced_read(self, li: int, q: torch.Tensor, r: torch.Tensor):
        """(r, fa, scale) under force_attn: the [C, N] map fa replaces every token's attention.
        With force_norm_match each token's forced read is scaled by |computed read| /
        (|forced read| + 1e-6), both taken with K as the values."""
        fa = self.force_attn.get(li) if isinstance(self.force_attn, dict) else self.force_attn
        K, M, V = self._dense(li, q.device)
        fa = _here(fa, K).to(K.dtype)
        if fa.shape != M.shape:
            raise ValueError(f"force_attn {tuple(fa.shape)} does not match the library's [C, N] {tuple(M.shape)}")
        flat = fa.reshape(-1)
        out = (flat @ V.reshape(-1, V.shape[-1])).to(r.dtype).expand_as(r)
        if not self.force_norm_match:
            return out, fa, None
        r_keys = r
        if self.lib.V is not None:        # the computed read's norm is taken with K as the values
            pool = self._pool(li, q)
            tied = ops.PagedLibrary(pool.pages, pool.chunk_page, pool.chunk_nvalid, pool.chunk_ptr, pool.S,
                                    n_chunks=pool.n_chunks, nvalid=pool.nvalid, d_valid=pool.d_valid)
            r_keys = self._read(q, tied)[0]
        forced_keys = flat @ K.reshape(-1, K.shape[-1])
        scale = torch.linalg.vector_norm(r_keys, dim=-1, keepdim=True) / (torch.linalg.vector_norm(forced_keys) + 1e-6)
        return out * scale.to(out.dtype), fa, scale

    def _keep_diagnostics(self, li: int, q, w, fa, scale) -> None:
        """record_attn: the [C, N] attention of the last position (detached, on the host);
        training_attn: the one at attn_pos with grad (batch row 0 for both)."""
        want_train = self.training_attn and torch.is_grad_enabled()
        if not (self.record_attn or want_train):
            return
        at = [q.shape[1] - 1, self.attn_pos]
        if fa is None:
            maps = self._slot_attention(q[0, at], w[0, at], li)
        else:
            maps = fa[None].expand(2, *fa.shape)
            if scale is not None:
                maps = maps * scale[0, at].to(fa.dtype).view(2, 1, 1)
        if self.record_attn:
            self.last_attn[li] = maps[0].detach().float().cpu()
        if want_train:
            self.attn_terms.append(maps[1].float())

    def _branch(self, h: torch.Tensor, li: int) -> torch.Tensor:
        if self.lib is None:                               # single-skill path
            delta = super()._branch(h, li)
        else:
            hn, q = self._query(h)                         # q [B, T, d_s]
            pool = self._pool(li, hn)
            diagnostics = self.force_attn is not None or self.record_attn or (
                self.training_attn and torch.is_grad_enabled())
            keep = None
            if self.selector is not None and hasattr(self.selector, "selected_rows") and not diagnostics:
                keep = self.selector.selected_rows(h, li)
            r, w = self._read(q, pool, keep)
            fa = scale = None
            if self.force_attn is not None:
                r, fa, scale = self._forced_read(li, q, r)
            self._keep_diagnostics(li, q, w, fa, scale)
            delta = write_delta(self.itf, hn, r, li, self.gain_scale)
            self.last_route = w.detach()
            if torch.is_grad_enabled():
                self.route_terms.append((li, w))
        if self.selector is not None:
            delta = self.selector.apply(delta, h, li)
        return delta


__all__ = ["SkillInjector", "XEncInjector", "LibraryInjector", "itf_query", "itf_gate", "itf_gain",
           "itf_write", "write_delta", "rms_norm", "apply_map"]
