"""D8: question-dependent slot top-k selection inside the read branch (the API of xenc/topk_read.py).

Selection (once per multi-token forward): the reader's own attention queries at a selection
layer (pre-RoPE, post q_norm), at one prompt position, are scored against slot-aligned attention
keys of the library, s_i = pool_h(q_h . k_{kv(h), i}) (GQA; pool = max over heads by default),
and the top-k valid slots are kept (`last_idx` [B, k], flat into [C * N]).  The scores run on
`xenc_select_scores` and the top-k on `xenc_topk_rows` (descending, ties to the lower index).

Read (every injection layer): the read restricted to the k selected slots, one softmax over
them, q = L2(A . RMSNorm(h)).  The selected slot rows are gathered (`xenc_gather_pages`) into a
one-chunk library per selection set, which the Library-read kernels then read with route
weight 1: the decode kernel for a few rows, the MFMA prefill kernels (differentiable in q) for
many rows or under autograd.  Single-token decode forwards reuse the selected set.  k >= the
number of valid slots skips the selection and reads exactly like LibraryInjector.

The selection query comes from an injector-disabled pre-pass of the bare reader that stops at
the selection layer's attention (a forward pre-hook on the model for HF models, on decoder
block 0 for models whose logits() bypasses __call__).
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import ops
from .depth import decoder_layers, rho_key, rho_layer_map
from .injector import LibraryInjector, _on, itf_query, write_delta
from .library import Library
from .selector import rms_norm


# ============================================================================ attention geometry
def attn_geometry(att) -> dict:
    """Head layout of an attention module (xenc/topk_read.py:43-52): head dim, kv heads, GQA
    groups, query heads, and whether q_proj also emits a gate (twice the query width)."""
    hd = int(getattr(att, "head_dim"))
    n_kv = att.k_proj.out_features // hd
    groups = int(getattr(att, "num_key_value_groups", 1))
    n_q = n_kv * groups
    gated = att.q_proj.out_features == 2 * n_q * hd
    if not gated and att.q_proj.out_features != n_q * hd:
        raise ValueError(f"q_proj out {att.q_proj.out_features} inconsistent with {n_q} heads x {hd}")
    return {"hd": hd, "n_kv": n_kv, "groups": groups, "n_q": n_q, "gated": gated}


def reader_queries(att, x: torch.Tensor, geo: dict) -> torch.Tensor:
    """The attention module's own pre-RoPE queries (post q_norm) -> [B, n_q, T, hd]
    (xenc/topk_read.py:55-66)."""
    B, T, _ = x.shape
    hd = geo["hd"]
    qg = att.q_proj(x)
    if geo["gated"]:
        q = qg.view(B, T, -1, 2 * hd)[..., :hd]
    else:
        q = qg.view(B, T, -1, hd)
    if hasattr(att, "q_norm"):
        q = att.q_norm(q)
    return q.transpose(1, 2)


def attn_layer_map(model, depths) -> dict:
    """rho -> the first layer with softmax attention (q/k/v projections) at or after the rho layer,
    else the last such layer (xenc/depth_skill.py:130-141)."""
    blocks = decoder_layers(model)
    full = [i for i, b in enumerate(blocks)
            if all(hasattr(getattr(b, "self_attn", None), p) for p in ("q_proj", "k_proj", "v_proj"))]
    if not full:
        raise ValueError("the model has no self-attention module with q_proj/k_proj/v_proj")
    out = {}
    for rho, li in rho_layer_map(model, depths).items():
        after = [j for j in full if j >= li]
        out[rho] = after[0] if after else full[-1]
    return out


def sel_layer_for(model, sel_rho: float) -> int:
    return int(attn_layer_map(model, [float(sel_rho)])[float(sel_rho)])


class _StopSelect(Exception):
    pass


# ============================================================================ selection-key library
class TopKLibrary(Library):
    """A residual Library plus `sel_K` [C, N, d_k]: the slot-aligned attention keys used for
    selection (xenc/topk_read.py:74-90)."""

    sel_K: torch.Tensor

    def subset(self, idx) -> "TopKLibrary":
        new = super().subset(idx)
        idx = [int(i) for i in (idx if hasattr(idx, "__iter__") else [idx])]
        n = next(iter(new.K.values())).shape[1]
        new.__class__ = TopKLibrary
        new.sel_K = self.sel_K.index_select(0, torch.tensor(idx, device=self.sel_K.device))[:, :n].clone()
        return new

    def to(self, device=None, dtype=None) -> "TopKLibrary":
        super().to(device=device, dtype=dtype)
        self.sel_K = self.sel_K.to(device=device, dtype=dtype)
        return self


def attach_sel_keys(lib: Library, attn_cache: dict, sel_rho: float) -> TopKLibrary:
    """Turn `lib` (in place) into a TopKLibrary whose sel_K holds the attention cache's keys at
    sel_rho, zero-padded to lib's [C, N] (xenc/topk_read.py:93-112).  The two harvests must be
    slot-aligned (same chunks, same valid counts)."""
    chunks = attn_cache["chunks"]
    C, N = next(iter(lib.mask.values())).shape
    if len(chunks) != C:
        raise ValueError(f"attn cache has {len(chunks)} chunks, residual library {C}")
    rows = [c["K"][rho_key(c["K"], sel_rho)] for c in chunks]
    n_lib = next(iter(lib.mask.values())).sum(-1).tolist()
    for c, r in enumerate(rows):
        if r.shape[0] != int(n_lib[c]):
            raise ValueError(f"chunk {c}: attn cache {r.shape[0]} slots vs residual {int(n_lib[c])} (not aligned)")
    dev = next(iter(lib.K.values())).device
    S = torch.zeros(C, N, rows[0].shape[-1], dtype=torch.float32, device=dev)
    for c, r in enumerate(rows):
        S[c, : r.shape[0]] = r.to(device=dev, dtype=torch.float32)
    lib.__class__ = TopKLibrary
    lib.sel_K = S
    return lib


# ============================================================================ selector
class TopKSelector:
    """Captures the reader's queries at `sel_layer` and scores them against the loaded selection
    keys (xenc/topk_read.py:160-270).  keys [S, n_kv, hd] (flat over C * N; invalid slots masked).
    Scores per head [B, n_q, S], pooled over heads ("max" | "mean") -> [B, S]; `last_idx` = the
    top-k flat indices [B, k] in descending score order (ties to the lower index)."""

    def __init__(self, model, sel_layer: int, k: int = 64, pool: str = "max", query: str = "last",
                 kmap: dict | None = None):
        blocks = decoder_layers(model)
        att = getattr(blocks[sel_layer], "self_attn", None)
        if att is None or not hasattr(att, "q_proj"):
            raise ValueError(f"selection layer {sel_layer} has no softmax self-attention with q_proj")
        self.model, self.sel_layer, self.att = model, int(sel_layer), att
        self.geo = attn_geometry(att)
        self.k, self.pool, self.query = int(k), pool, query
        self.kmap = kmap
        self.keys: torch.Tensor | None = None
        self.valid: torch.Tensor | None = None
        self.pos: int = -1
        self.last_idx: torch.Tensor | None = None
        self.last_scores: torch.Tensor | None = None
        self.last_head_scores: torch.Tensor | None = None
        self.keep_heads = False
        self.armed = False

    # ---- keys
    def set_keys(self, sel_K: torch.Tensor, valid: torch.Tensor) -> None:
        K = sel_K.reshape(-1, sel_K.shape[-1]).float()
        if self.kmap is not None:
            K = K @ self.kmap["W"].to(K).T + self.kmap["b"].to(K)
        g = self.geo
        if K.shape[-1] != g["n_kv"] * g["hd"]:
            raise ValueError(f"selection keys d={K.shape[-1]} != reader KV dim {g['n_kv'] * g['hd']} "
                             "(cross-model selection needs a key map)")
        self.keys = K.reshape(-1, g["n_kv"], g["hd"]).contiguous()
        self.valid = valid.reshape(-1).bool()

    def clear(self) -> None:
        self.keys = self.valid = self.last_idx = self.last_scores = self.last_head_scores = None

    @property
    def n_valid(self) -> int:
        return int(self.valid.sum()) if self.valid is not None else 0

    # ---- scoring
    def head_scores(self, q: torch.Tensor) -> torch.Tensor:
        """q [B, n_q, T, hd] -> per-head scores [B, n_q, T, S] (GQA grouping, no RoPE either side)."""
        g = self.geo
        K = _on(self.keys, q)
        B, _, T, hd = q.shape
        qh = q.float().reshape(B, g["n_kv"], g["groups"], T, hd)
        s = torch.einsum("bkgtd,skd->bkgts", qh, K)
        return s.reshape(B, g["n_q"], T, -1)

    def pool_scores(self, s: torch.Tensor, query: str | None = None, pool: str | None = None) -> torch.Tensor:
        """[B, n_q, T, S] -> [B, S]: positions per `query` (last | all_max | all_mean), heads per `pool`."""
        query, pool = query or self.query, pool or self.pool
        if query == "last":
            s = s[:, :, -1]
        elif query == "all_max":
            s = s.amax(2)
        elif query == "all_mean":
            s = s.mean(2)
        else:
            raise ValueError(f"unknown selection query {query}")
        s = s.amax(1) if pool == "max" else s.mean(1)
        return s.masked_fill(~_on(self.valid, s).unsqueeze(0), float("-inf"))

    def select_from_input(self, x: torch.Tensor) -> torch.Tensor:
        """x = input of the selection layer's attention (post input_layernorm) [B, T, d].  The
        last-position scores and the top-k run on the HIP kernels."""
        T = x.shape[1]
        pos = self.pos if self.pos >= 0 else T + self.pos
        q = reader_queries(self.att, x[:, : pos + 1], self.geo)       # [B, n_q, pos+1, hd]
        if self.query == "last" and not self.keep_heads:
            self.keys = _on(self.keys, q)
            sc = ops.select_scores(q[:, :, -1].float().contiguous(), self.keys, _on(self.valid, q), self.pool)
        else:
            s = self.head_scores(q)
            if self.keep_heads:
                self.last_head_scores = s.detach()
            sc = self.pool_scores(s).contiguous()
        k = min(self.k, self.n_valid)
        self.last_scores = sc.detach()
        idx, _ = ops.topk_rows(sc.float(), k)
        self.last_idx = idx.long()
        return self.last_idx

    # ---- stats
    def gold_hit(self, gold_flat: torch.Tensor, ks=None) -> dict:
        """gold_flat [C * N] bool -> {k: {hit, n_gold_sel, chance_any, chance_frac}} for batch row 0
        (xenc/topk_read.py:245-270)."""
        sc = self.last_scores[0]
        g = _on(gold_flat.reshape(-1).bool(), sc)[: sc.numel()]
        v = _on(self.valid, sc)
        g = g & v
        n, ng = int(v.sum()), int(g.sum())
        if ng == 0:
            return {}
        order = sc.argsort(descending=True, stable=True)
        rank_of = torch.empty_like(order)
        rank_of[order] = torch.arange(order.numel(), device=order.device)
        best = int(rank_of[g].min())
        out = {"n_valid": n, "n_gold": ng, "best_rank": best, "best_rank_frac": best / max(n - 1, 1)}
        for k in (ks or [self.k]):
            k = min(int(k), n)
            hits = int(g[order[:k]].sum())
            # P(a uniformly random k-subset holds >= 1 gold slot) = 1 - C(n - ng, k) / C(n, k)
            lp = (math.lgamma(n - ng + 1) - math.lgamma(n - ng - k + 1) - math.lgamma(n + 1)
                  + math.lgamma(n - k + 1)) if n - ng >= k else float("-inf")
            out[k] = {"hit": float(hits > 0), "n_gold_sel": hits, "chance_any": 1.0 - math.exp(lp),
                      "chance_frac": k * ng / n}
        return out


def _is_hf(model: nn.Module) -> bool:
    try:
        from transformers import PreTrainedModel
    except ImportError:   # no transformers: every model is driven through block 0
        return False
    return isinstance(model, PreTrainedModel)


# ============================================================================ injector
class TopKLibraryInjector(LibraryInjector):
    """LibraryInjector whose read covers only the selected slots (xenc/topk_read.py:272-414)."""

    def __init__(self, model, interface, selector: TopKSelector, read_softmax: bool = True,
                 read_temp: float = 12.0, route_temp: float = 10.0, top_k: int = 0, layer_selector=None,
                 read_fp32: bool = True):
        self.tk = selector
        self._selecting = False
        self._sel_this_forward = False
        self.sel_pos = -1
        self.n_select_passes = 0
        super().__init__(model, interface, read_softmax=read_softmax, read_temp=read_temp,
                         route_temp=route_temp, top_k=top_k, selector=layer_selector, read_fp32=read_fp32)

    @property
    def last_idx(self):
        return self.tk.last_idx

    def _active(self) -> bool:
        return (not self._selecting) and super()._active()

    # ---- load / unload
    def load_library(self, lib) -> None:
        super().load_library(lib)
        if getattr(lib, "sel_K", None) is None:
            raise ValueError("TopKLibraryInjector needs a TopKLibrary (residual library + sel_K attention keys)")
        first = self.itf.inject_layers[0]
        self.tk.set_keys(lib.sel_K, lib.mask[first])
        self.tk.last_idx = None

    def unload(self) -> None:
        super().unload()
        self.tk.clear()

    @property
    def full_read(self) -> bool:
        return self.tk.k >= self.tk.n_valid

    # ---- hooks
    def _attach(self) -> None:
        super()._attach()
        blocks = decoder_layers(self.model)

        def att_pre(mod, args, kwargs):
            if self._selecting:
                x = kwargs["hidden_states"] if "hidden_states" in kwargs else args[0]
                self.tk.pos = self.sel_pos
                with torch.no_grad():
                    self.tk.select_from_input(x)
                raise _StopSelect

        self._handles.append(self.tk.att.register_forward_pre_hook(att_pre, with_kwargs=True))
        hf = _is_hf(self.model)

        def top_pre(mod, args, kwargs):            # every model(...) call: prefill / decode / train
            if self._selecting or not self._active():
                return None
            x = kwargs.get("input_ids")
            if x is None:
                x = kwargs.get("inputs_embeds")
            if x is None and args:
                x = args[0]
            self._sel_this_forward = True
            if x is None or self.full_read:
                return None
            if x.shape[1] == 1 and self.tk.last_idx is not None:
                return None                        # decode step: reuse the selected set
            kw = dict(kwargs)
            if "past_key_values" in kw:
                kw["past_key_values"] = None
            if "use_cache" in kw or hasattr(self.model, "generation_config"):
                kw["use_cache"] = False
            kw.pop("logits_to_keep", None)
            self._run_select(lambda: mod(*args, **kw))
            return None

        self._handles.append(self.model.register_forward_pre_hook(top_pre, with_kwargs=True))

        def block0_pre(mod, args):                 # models whose logits() bypasses model.__call__
            if self._selecting or not self._active():
                return None
            if hf:                                 # HF: the selection happens in top_pre
                self._sel_this_forward = False
                return None
            if self._sel_this_forward:
                self._sel_this_forward = False
                return None
            if self.full_read:
                return None
            x = args[0]
            if x.shape[1] == 1 and self.tk.last_idx is not None:
                return None
            self._run_select(lambda: self.model.forward(x))
            return None

        self._handles.append(blocks[0].register_forward_pre_hook(block0_pre))

    def _run_select(self, fn) -> None:
        self._selecting = True
        self.n_select_passes += 1
        try:
            with torch.no_grad():
                fn()
        except _StopSelect:
            pass
        finally:
            self._selecting = False
        if self.tk.last_idx is None:
            raise RuntimeError("D8 selection pass did not reach the selection layer")

    # ---- branch
    def _sel_attn(self, q_rows: torch.Tensor, sel: ops.PagedLibrary, k: int) -> torch.Tensor:
        """Read weights over the k selected slots for a few query rows (torch, differentiable in q)."""
        Ks = sel.pages[0, :k, : sel.d_valid].float()
        a = q_rows.float() @ Ks.T
        return torch.softmax(a * self.read_temp, -1) if self.read_softmax else a / (k ** 0.5)

    def _branch(self, h: torch.Tensor, li: int) -> torch.Tensor:
        if self.lib is None or self.full_read:
            return super()._branch(h, li)
        idx = self.tk.last_idx                                       # [B', k]
        hn = rms_norm(h.float())
        q = itf_query(self.itf, hn)                                  # [B, T, d_s]
        B_, T_, d = q.shape
        pl = self._pool(li, hn)
        n_flat = self.lib.mask[li].shape[1]
        idx = _on(idx, hn)
        if idx.shape[0] != B_:
            idx = idx[:1]
        k = idx.shape[1]
        sets = [idx] if idx.shape[0] == 1 else [idx[b:b + 1] for b in range(B_)]
        rows = [q.reshape(B_ * T_, d)] if len(sets) == 1 else [q[b] for b in range(B_)]
        rs, sels = [], []
        for ii, qr in zip(sets, rows):
            sel = ops.gather_library(pl, ii, n_flat)
            M = qr.shape[0]
            one = torch.ones(M, 1, dtype=torch.float32, device=q.device)
            zero = torch.zeros(M, 1, dtype=torch.int32, device=q.device)
            rs.append(ops.read_rows(qr, one, zero, one, sel, self.read_temp, self.read_softmax))
            sels.append(sel)
        r = (rs[0] if len(rs) == 1 else torch.stack(rs)).reshape(B_, T_, -1)
        C, N = self.lib.mask[li].shape
        if self.record_attn:             # [C, N] read attention at the last position (zero off the set)
            a = self._sel_attn(q[0, -1:], sels[0], k)[0]
            full = torch.zeros(C * N, dtype=a.dtype, device=a.device).index_put((idx[0],), a.detach())
            self.last_attn[li] = full.view(C, N).float().cpu()
        if self.training_attn and torch.is_grad_enabled():
            a = self._sel_attn(q[0, self.attn_pos:][:1], sels[0], k)[0]
            full = torch.zeros(C * N, dtype=a.dtype, device=a.device).index_put((idx[0],), a)
            self.attn_terms.append(full.view(C, N).float())
        delta = write_delta(self.itf, hn, r, li, self.gain_scale)
        self.last_route = None
        if self.selector is not None:
            delta = self.selector.apply(delta, h, li)
        return delta


__all__ = ["attn_geometry", "reader_queries", "attn_layer_map", "sel_layer_for", "TopKLibrary",
           "attach_sel_keys", "TopKSelector", "TopKLibraryInjector"]
