"""D8: question-dependent slot top-k selection inside the read branch (the API of xenc/topk_read.py).

Selection (once per multi-token forward): the reader's own attention queries at a selection layer
(pre-RoPE, after q_norm), at one prompt position, are scored against slot-aligned attention keys
of the library, s_i = pool_h(q_h . k_{kv(h), i}) (GQA; pool = max over heads by default), and
the top-k valid slots are kept (`last_idx` [B, k], flat into [C * N]).  Scores run on
`xenc_select_scores` and the top-k on `xenc_topk_rows` (descending, ties to the lower index).

Read (every injection layer): the read restricted to the k selected slots, one softmax over them,
q = L2(A . rms_norm(h)).  The selected slot rows are gathered (`xenc_gather_pages`) into a
one-chunk library per selection set and read with route weight 1 by the Library-read kernels (the
decode operators for a few rows, the differentiable MFMA operators for many rows or autograd).
Single-token decode forwards reuse the selected set.  k >= the number of valid slots skips the
selection and reads exactly like LibraryInjector.

The selection query comes from a pre-pass of the bare reader (the injector inactive) that stops
at the selection layer's attention: a forward pre-hook on the model triggers it for HF models;
for models whose logits() bypasses __call__, a pre-hook on decoder block 0 does.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import ops
from .depth import decoder_layers, rho_key, rho_layer_map
from .injector import LibraryInjector, write_delta
from .library import Library


def _here(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if t.device == like.device else t.to(like.device)


# ============================================================================ attention geometry
def attn_geometry(att) -> dict:
    """Head layout of an attention module: head dim, kv heads, GQA groups, query heads, and whether
    q_proj also emits a gate (its output twice the query width)."""
    hd = int(att.head_dim)
    n_kv = att.k_proj.out_features // hd
    groups = int(getattr(att, "num_key_value_groups", 1))
    n_q = n_kv * groups
    width = att.q_proj.out_features
    if width not in (n_q * hd, 2 * n_q * hd):
        raise ValueError(f"q_proj emits {width} features, which fits neither {n_q} heads x {hd} nor twice that")
    return {"hd": hd, "n_kv": n_kv, "groups": groups, "n_q": n_q, "gated": width == 2 * n_q * hd}


def reader_queries(att, x: torch.Tensor, geo: dict) -> torch.Tensor:
    """The attention module's own queries before RoPE (after q_norm when it has one), [B, n_q, T, hd]."""
    B, T, _ = x.shape
    hd = geo["hd"]
    heads = att.q_proj(x).view(B, T, geo["n_q"], -1)[..., :hd]    # a gated q_proj puts the gate second
    if hasattr(att, "q_norm"):
        heads = att.q_norm(heads)
    return heads.permute(0, 2, 1, 3)


def _has_softmax_attention(block) -> bool:
    att = getattr(block, "self_attn", None)
    return att is not None and all(hasattr(att, p) for p in ("q_proj", "k_proj", "v_proj"))


def attn_layer_map(model, depths) -> dict:
    """rho -> the first softmax-attention layer at or after the rho layer, else the last one
    (xenc/depth_skill.py:130-141)."""
    full = [i for i, b in enumerate(decoder_layers(model)) if _has_softmax_attention(b)]
    if not full:
        raise ValueError("the model has no self-attention module with q_proj / k_proj / v_proj")
    return {rho: next((j for j in full if j >= li), full[-1]) for rho, li in rho_layer_map(model, depths).items()}


def sel_layer_for(model, sel_rho: float) -> int:
    return int(attn_layer_map(model, [float(sel_rho)])[float(sel_rho)])


# ============================================================================ selection-key library
class TopKLibrary(Library):
    """A residual Library plus sel_K [C, N, d_k]: the slot-aligned attention keys used for
    selection."""

    sel_K: torch.Tensor

    def subset(self, idx) -> "TopKLibrary":
        out = super().subset(idx)
        picks = torch.as_tensor([int(i) for i in idx] if hasattr(idx, "__iter__") else [int(idx)],
                                device=self.sel_K.device)
        width = next(iter(out.mask.values())).shape[1]
        out.sel_K = self.sel_K.index_select(0, picks)[:, :width].clone()
        return out

    def to(self, device=None, dtype=None) -> "TopKLibrary":
        super().to(device=device, dtype=dtype)
        self.sel_K = self.sel_K.to(device=device, dtype=dtype)
        return self


def attach_sel_keys(lib: Library, attn_cache: dict, sel_rho: float) -> TopKLibrary:
    """Turn `lib` (in place) into a TopKLibrary whose sel_K holds the attention cache's keys at
    sel_rho, zero-padded to lib's [C, N].  The two harvests must be slot-aligned: the same chunks
    with the same valid counts (ValueError otherwise)."""
    mask = next(iter(lib.mask.values()))
    C, N = mask.shape
    blocks = [ch["K"][rho_key(ch["K"], sel_rho)] for ch in attn_cache["chunks"]]
    if len(blocks) != C:
        raise ValueError(f"the attention cache has {len(blocks)} chunks, the library {C}")
    counts = mask.sum(-1).tolist()
    for c, (b, n) in enumerate(zip(blocks, counts)):
        if b.shape[0] != int(n):
            raise ValueError(f"chunk {c} holds {b.shape[0]} attention keys but {int(n)} library slots")
    dev = next(iter(lib.K.values())).device
    keys = torch.zeros(C, N, blocks[0].shape[-1], dtype=torch.float32, device=dev)
    for c, b in enumerate(blocks):
        keys[c, :b.shape[0]] = b.to(device=dev, dtype=torch.float32)
    lib.__class__ = TopKLibrary
    lib.sel_K = keys
    return lib


# ============================================================================ selector
class TopKSelector:
    """Scores the reader's queries at `sel_layer` against the loaded selection keys.  keys
    [S, n_kv, hd] (flat over C * N) with `valid` [S]; per-head scores [B, n_q, T, S] are pooled
    over heads ("max" | "mean") and over positions (query: "last" | "all_max" | "all_mean") into
    [B, S] with invalid slots at -inf; `last_idx` [B, k] is the top-k in descending order, ties to
    the lower index."""

    def __init__(self, model, sel_layer: int, k: int = 64, pool: str = "max", query: str = "last",
                 kmap: dict | None = None):
        att = getattr(decoder_layers(model)[sel_layer], "self_attn", None)
        if att is None or not hasattr(att, "q_proj"):
            raise ValueError(f"layer {sel_layer} has no softmax self-attention with a q_proj")
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
        flat = sel_K.reshape(-1, sel_K.shape[-1]).float()
        if self.kmap is not None:                       # keys of another encoder mapped into the reader's space
            flat = torch.addmm(self.kmap["b"].to(flat), flat, self.kmap["W"].to(flat).T)
        n_kv, hd = self.geo["n_kv"], self.geo["hd"]
        if flat.shape[-1] != n_kv * hd:
            raise ValueError(f"selection keys have {flat.shape[-1]} features, the reader's keys {n_kv * hd} "
                             "(keys of another model need a key map)")
        self.keys = flat.view(-1, n_kv, hd).contiguous()
        self.valid = valid.reshape(-1).bool()

    def clear(self) -> None:
        self.keys = self.valid = None
        self.last_idx = self.last_scores = self.last_head_scores = None

    @property
    def n_valid(self) -> int:
        return 0 if self.valid is None else int(self.valid.sum())

    # ---- scoring
    def head_scores(self, q: torch.Tensor) -> torch.Tensor:
        """q [B, n_q, T, hd] -> [B, n_q, T, S]: query head h scores kv head h // groups (no RoPE)."""
        B, n_q, T, hd = q.shape
        K = _here(self.keys, q)
        grouped = q.float().view(B, self.geo["n_kv"], self.geo["groups"], T, hd)
        return torch.einsum("bkgtd,skd->bkgts", grouped, K).reshape(B, n_q, T, -1)

    def pool_scores(self, s: torch.Tensor, query: str | None = None, pool: str | None = None) -> torch.Tensor:
        """[B, n_q, T, S] -> [B, S]: positions pooled per `query`, then heads per `pool`."""
        over_t = {"last": lambda x: x[:, :, -1], "all_max": lambda x: x.amax(2), "all_mean": lambda x: x.mean(2)}
        which = query or self.query
        if which not in over_t:
            raise ValueError(f"unknown selection query {which!r}")
        s = over_t[which](s)
        s = s.amax(1) if (pool or self.pool) == "max" else s.mean(1)
        return s.masked_fill(~_here(self.valid, s)[None], float("-inf"))

    def select_from_input(self, x: torch.Tensor) -> torch.Tensor:
        """x: the selection layer attention's input [B, T, d] (after its input norm).  The
        last-position scores and the top-k run on the HIP kernels."""
        upto = (self.pos if self.pos >= 0 else x.shape[1] + self.pos) + 1
        q = reader_queries(self.att, x[:, :upto], self.geo)
        if self.query == "last" and not self.keep_heads:
            self.keys = _here(self.keys, q)
            scores = ops.select_scores(q[:, :, -1].float().contiguous(), self.keys, _here(self.valid, q), self.pool)
        else:
            s = self.head_scores(q)
            if self.keep_heads:
                self.last_head_scores = s.detach()
            scores = self.pool_scores(s).contiguous()
        self.last_scores = scores.detach()
        idx, _ = ops.topk_rows(scores.float(), min(self.k, self.n_valid))
        self.last_idx = idx.long()
        return self.last_idx


# ============================================================================ the selection pre-pass
class _SelectionDone(Exception):
    """Raised by the selection layer's pre-hook to end the pre-pass there."""


class _CaptureAtSelectionLayer:
    """Forward pre-hook (with kwargs) on the selection layer's attention: during a pre-pass, score
    its input and end the pass."""

    def __init__(self, owner: "TopKLibraryInjector"):
        self.owner = owner

    def __call__(self, module, args, kwargs):
        inj = self.owner
        if not inj._selecting:
            return None
        x = kwargs["hidden_states"] if "hidden_states" in kwargs else args[0]
        inj.tk.pos = inj.sel_pos
        with torch.no_grad():
            inj.tk.select_from_input(x)
        raise _SelectionDone


class _ModelCall:
    """Forward pre-hook (with kwargs) on the model: every model(...) call of a prefill, decode
    step or training forward.  Runs the pre-pass with the same inputs, no cache."""

    def __init__(self, owner: "TopKLibraryInjector"):
        self.owner = owner

    def __call__(self, module, args, kwargs):
        inj = self.owner
        if inj._selecting or not inj._active():
            return None
        inj._model_level_call = True
        x = next((kwargs[k] for k in ("input_ids", "inputs_embeds") if kwargs.get(k) is not None),
                 args[0] if args else None)
        if inj._wants_selection(x):
            kw = {k: v for k, v in kwargs.items() if k != "logits_to_keep"}
            if "past_key_values" in kw:
                kw["past_key_values"] = None
            if "use_cache" in kw or hasattr(inj.model, "generation_config"):
                kw["use_cache"] = False
            inj._run_selection(lambda: module(*args, **kw))
        return None


class _BlockZeroCall:
    """Forward pre-hook on decoder block 0, for models whose logits() runs the blocks without
    model.__call__: selects there when no model-level call did for this forward."""

    def __init__(self, owner: "TopKLibraryInjector"):
        self.owner = owner

    def __call__(self, module, args):
        inj = self.owner
        if inj._selecting or not inj._active():
            return None
        if inj._model_level_call:
            inj._model_level_call = False
            return None
        x = args[0]
        if inj._wants_selection(x):
            inj._run_selection(lambda: inj.model.forward(x))
        return None


def _is_hf(model: nn.Module) -> bool:
    try:
        from transformers import PreTrainedModel
    except ImportError:        # no transformers: every model is driven through block 0
        return False
    return isinstance(model, PreTrainedModel)


# ============================================================================ injector
class TopKLibraryInjector(LibraryInjector):
    """LibraryInjector whose read covers only the selected slots."""

    def __init__(self, model, interface, selector: TopKSelector, read_softmax: bool = True,
                 read_temp: float = 12.0, route_temp: float = 10.0, top_k: int = 0, layer_selector=None,
                 read_fp32: bool = True):
        self.tk = selector
        self._selecting = False
        self._model_level_call = False
        self.sel_pos = -1
        self.n_select_passes = 0
        super().__init__(model, interface, read_softmax=read_softmax, read_temp=read_temp,
                         route_temp=route_temp, top_k=top_k, selector=layer_selector, read_fp32=read_fp32)

    @property
    def last_idx(self):
        return self.tk.last_idx

    @property
    def full_read(self) -> bool:
        return self.tk.k >= self.tk.n_valid

    def _active(self) -> bool:
        return not self._selecting and super()._active()

    # ---- load / unload
    def load_library(self, lib) -> None:
        super().load_library(lib)
        if getattr(lib, "sel_K", None) is None:
            raise ValueError("TopKLibraryInjector reads a TopKLibrary (a residual library with sel_K attention keys)")
        self.tk.set_keys(lib.sel_K, lib.mask[self.itf.inject_layers[0]])
        self.tk.last_idx = None

    def unload(self) -> None:
        super().unload()
        self.tk.clear()

    # ---- selection pre-pass
    def _attach(self) -> None:
        super()._attach()
        self._handles.append(self.tk.att.register_forward_pre_hook(_CaptureAtSelectionLayer(self), with_kwargs=True))
        self._handles.append(self.model.register_forward_pre_hook(_ModelCall(self), with_kwargs=True))
        if not _is_hf(self.model):      # HF models always pass through model.__call__
            self._handles.append(decoder_layers(self.model)[0].register_forward_pre_hook(_BlockZeroCall(self)))

    def _wants_selection(self, x) -> bool:
        """A multi-position forward selects; a one-position decode step reuses the last set."""
        if x is None or self.full_read:
            return False
        return not (x.shape[1] == 1 and self.tk.last_idx is not None)

    def _run_selection(self, forward) -> None:
        self._selecting = True
        self.n_select_passes += 1
        try:
            with torch.no_grad():
                forward()
        except _SelectionDone:
            pass
        finally:
            self._selecting = False
        if self.tk.last_idx is None:
            raise RuntimeError("the D8 selection pass ended before the selection layer")

    # ---- branch
    def _selected_attention(self, q_rows: torch.Tensor, sel: ops.PagedLibrary, k: int) -> torch.Tensor:
        """Read weights over the k selected slots for a few query rows (torch, differentiable in q)."""
        keys = sel.pages[0, :k, :sel.d_valid].float()
        s = q_rows.float() @ keys.T
        return torch.softmax(s * self.read_temp, -1) if self.read_softmax else s / k ** 0.5

    def _scatter_map(self, li: int, idx_row: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
        """[C, N] map with the selected slots' weights a and 0 elsewhere."""
        C, N = self.lib.mask[li].shape
        return torch.zeros(C * N, dtype=a.dtype, device=a.device).index_put((idx_row,), a).view(C, N)

    def _branch(self, h: torch.Tensor, li: int) -> torch.Tensor:
        if self.lib is None or self.full_read:
            return super()._branch(h, li)
        hn, q = self._query(h)                                       # q [B, T, d_s]
        B, T, d = q.shape
        pool = self._pool(li, hn)
        n_flat = self.lib.mask[li].shape[1]
        idx = _here(self.tk.last_idx, hn)
        if idx.shape[0] != B:
            idx = idx[:1]
        k = idx.shape[1]
        shared = idx.shape[0] == 1                                   # one set serves every batch row
        groups = [(idx, q.reshape(B * T, d))] if shared else [(idx[b:b + 1], q[b]) for b in range(B)]
        reads, libs = [], []
        for sel_idx, rows in groups:
            sel = ops.gather_library(pool, sel_idx, n_flat)
            M = rows.shape[0]
            one = torch.ones(M, 1, dtype=torch.float32, device=q.device)
            first = torch.zeros(M, 1, dtype=torch.int32, device=q.device)
            reads.append(ops.read_rows(rows, one, first, one, sel, self.read_temp, self.read_softmax))
            libs.append(sel)
        r = (reads[0] if shared else torch.stack(reads)).reshape(B, T, -1)
        if self.record_attn:
            a = self._selected_attention(q[0, -1:], libs[0], k)[0]
            self.last_attn[li] = self._scatter_map(li, idx[0], a.detach()).float().cpu()
        if self.training_attn and torch.is_grad_enabled():
            a = self._selected_attention(q[0, self.attn_pos:][:1], libs[0], k)[0]
            self.attn_terms.append(self._scatter_map(li, idx[0], a).float())
        delta = write_delta(self.itf, hn, r, li, self.gain_scale)
        self.last_route = None
        if self.selector is not None:
            delta = self.selector.apply(delta, h, li)
        return delta


__all__ = ["attn_geometry", "reader_queries", "attn_layer_map", "sel_layer_for", "TopKLibrary",
           "attach_sel_keys", "TopKSelector", "TopKLibraryInjector"]
