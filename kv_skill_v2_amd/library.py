"""Library: the chunk operators of one or more documents, keyed by reader layer.

Per reader layer li (the API of xenc/library.py:21-136):
    K[li]    [C, N_max, d_s]  chunk slot rows, zero-padded past each chunk's n_c valid rows
    mask[li] [C, N_max] bool  valid slots (a prefix of each row)
    S[li]    [C, d_s]         summary key L2(mean of the valid rows), used for routing
    V[li]    [C, N_max, d_s]  values, only when the chunks carry untied values (else V is None
                              and K serves as the values)

On top of the reference layout, `paged(li, device)` gives the device pool the HIP read kernels
take: fp16 pages [C, N_pad, d_pad] (one page per chunk, N and d rounded up to 64 with masked
slots / zero features), the page table, valid counts and fp32 S.  It is built once per
(layer, device) and dropped whenever the Library is moved, cast or re-centred.
"""

from __future__ import annotations

import torch
from torch.nn.utils.rnn import pad_sequence

from .depth import rho_key, rho_layer_map

_EPS = 1e-6
PAGE_ALIGN = 64   # page slots and features are padded to this for the MFMA prefill kernels


def l2(x: torch.Tensor) -> torch.Tensor:
    return x / (x.norm(dim=-1, keepdim=True) + _EPS)


def _field(chunk, name):
    if hasattr(chunk, name):
        return getattr(chunk, name)
    return chunk.get(name) if isinstance(chunk, dict) else None


class Library:
    def __init__(self, chunks: list, reader_layers: list[int], depths, device="cpu",
                 dtype=torch.float32, meta: list[dict] | None = None, center: dict | None = None):
        """chunks: rho-keyed chunk operators (objects with .K / .V, or dicts with "K" / "V"), each
        K[rho] of shape [n_c, d_s].  reader_layers[i] serves sorted(depths)[i].  center: optional
        {rho: mu [d_s]}; every valid slot then becomes L2(slot - mu[rho])."""
        if not chunks:
            raise ValueError("Library needs at least one chunk")
        depths = sorted(float(r) for r in depths)
        if len(reader_layers) != len(depths):
            raise ValueError(f"{len(reader_layers)} reader layers for {len(depths)} depths")
        self.depths = depths
        self.reader_layers = list(reader_layers)
        self.rho_of = dict(zip(self.reader_layers, depths))
        Ks = [_field(c, "K") for c in chunks]
        Vs = [_field(c, "V") for c in chunks]
        untied = any(v is not None and v is not k for v, k in zip(Vs, Ks))
        if meta is None:
            meta = []
            for c in chunks:
                m = getattr(c, "meta", None)
                if m is None and isinstance(c, dict):
                    m = {k: v for k, v in c.items() if k not in ("K", "V")}
                meta.append(dict(m or {}))
        self.chunk_meta = meta
        self.K, self.mask, self.S = {}, {}, {}
        self.V = {} if untied else None
        for li, rho in self.rho_of.items():
            rows = [k[rho_key(k, rho)].to(device=device, dtype=dtype) for k in Ks]
            n = torch.tensor([r.shape[0] for r in rows], device=device)
            Kt = pad_sequence(rows, batch_first=True)
            M = torch.arange(Kt.shape[1], device=device).view(1, -1) < n.view(-1, 1)
            if center is not None:   # a centre dict must cover every depth (KeyError otherwise)
                mu = center[rho_key(center, rho)].to(device=device, dtype=dtype)
                Kt = torch.where(M.unsqueeze(-1), l2(Kt - mu), torch.zeros_like(Kt))
            self.K[li], self.mask[li] = Kt, M
            if untied:
                vrows = [(v if v is not None else k) for v, k in zip(Vs, Ks)]
                self.V[li] = pad_sequence([v[rho_key(v, rho)].to(device=device, dtype=dtype) for v in vrows],
                                          batch_first=True)
        self.center = center
        self._summaries()

    def _summaries(self) -> None:
        self.S = {}
        for li, Kt in self.K.items():
            M = self.mask[li]
            tot = (Kt * M.unsqueeze(-1).to(Kt.dtype)).sum(1)
            cnt = M.sum(1, keepdim=True).clamp_min(1).to(Kt.dtype)
            self.S[li] = l2(tot / cnt)
        self._paged = {}

    # ------------------------------------------------------------------ properties
    @property
    def n_chunks(self) -> int:
        return next(iter(self.K.values())).shape[0]

    @property
    def d_s(self) -> int:
        return next(iter(self.K.values())).shape[-1]

    @property
    def layers(self) -> list[int]:
        return sorted(self.K)

    def n_valid(self, li: int) -> torch.Tensor:
        return self.mask[li].sum(-1)

    # ------------------------------------------------------------------ ops
    def to(self, device=None, dtype=None) -> "Library":
        """Move / cast in place (the mask stays bool); returns self."""
        for li in list(self.K):
            self.K[li] = self.K[li].to(device=device, dtype=dtype)
            self.S[li] = self.S[li].to(device=device, dtype=dtype)
            self.mask[li] = self.mask[li].to(device=device)
            if self.V is not None:
                self.V[li] = self.V[li].to(device=device, dtype=dtype)
        self._paged = {}
        return self

    def subset(self, idx) -> "Library":
        """The Library of chunks `idx` alone (re-trimmed to their longest chunk, S recomputed)."""
        idx = [int(i) for i in (idx if hasattr(idx, "__iter__") else [idx])]
        if not idx:
            raise ValueError("empty subset")
        new = object.__new__(Library)
        new.depths, new.reader_layers, new.rho_of = self.depths, self.reader_layers, dict(self.rho_of)
        new.center = getattr(self, "center", None)
        new.chunk_meta = [self.chunk_meta[i] for i in idx]
        new.K, new.mask = {}, {}
        new.V = {} if self.V is not None else None
        for li in self.K:
            sel = torch.tensor(idx, device=self.K[li].device)
            M = self.mask[li].index_select(0, sel)
            n = int(M.sum(-1).max())
            new.mask[li] = M[:, :n].clone()
            new.K[li] = self.K[li].index_select(0, sel)[:, :n].clone()
            if new.V is not None:
                new.V[li] = self.V[li].index_select(0, sel)[:, :n].clone()
        new._summaries()
        return new

    @staticmethod
    def from_doc_cache(cache: dict, reader_model, depths=None, device=None, dtype=torch.float32,
                       center: dict | None = None) -> "Library":
        """From a document cache dict {"depths", "chunks": [{"K": {rho: rows}, "start", "n_tokens"}],
        "doc_id", "encoder"} for the given reader model."""
        depths = sorted(float(r) for r in (depths or cache["depths"]))
        rmap = rho_layer_map(reader_model, depths)
        if device is None:
            device = reader_model.device if hasattr(reader_model, "device") else "cpu"
        meta = [{"doc_id": cache.get("doc_id", ""), "start": int(c.get("start", 0)),
                 "n_tokens": int(c.get("n_tokens", 0)), "encoder": cache.get("encoder", "")}
                for c in cache["chunks"]]
        return Library(cache["chunks"], [rmap[r] for r in depths], depths, device, dtype, meta=meta,
                       center=center)

    # ------------------------------------------------------------------ device pool
    def paged(self, li: int, device):
        """The HIP read pool of layer li on `device` (kv_skill_v2_amd.ops.PagedLibrary), built on
        first use and cached until the Library changes."""
        from .ops import PagedLibrary

        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        key = (li, device)
        pl = self._paged.get(key)
        if pl is None:
            V = self.V[li] if self.V is not None else None
            pl = PagedLibrary.from_padded(self.K[li], self.mask[li], self.S[li].float(), device=device,
                                          V=V, pad_to=PAGE_ALIGN)
            self._paged[key] = pl
        return pl


__all__ = ["Library", "l2", "PAGE_ALIGN"]
