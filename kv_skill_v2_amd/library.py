"""Library: the chunk operators of one or more documents, keyed by reader layer.

Per reader layer li (the attributes of xenc/library.py:25-136):
    K[li]    [C, N_max, d_s]  chunk slot rows, zero past each chunk's n_c valid rows
    mask[li] [C, N_max] bool  valid slots (a prefix of each row)
    S[li]    [C, d_s]         summary key L2(mean of the valid rows), used for routing
    V[li]    [C, N_max, d_s]  values, only when the chunks carry untied values (else V is None
                              and K serves as the values)

Every layer is assembled the same way from a list of per-chunk row blocks [n_c, d_s] (`_assemble`):
the constructor passes the cache rows (centred first when a centre is given), `subset` passes
the valid rows of the chosen chunks, so a subset is by construction the Library those chunks
would build alone.

`paged(li, device)` gives the device pool the HIP read kernels take: fp16 pages [C, N_pad, d_pad]
(one page per chunk, N and d rounded up to 64 with masked slots / zero features), the page table,
valid counts and fp32 S.  It is built once per (layer, device) and dropped whenever the Library is
moved, cast or re-centred.
"""

from __future__ import annotations

import torch
from torch.nn.utils.rnn import pad_sequence

from .depth import rho_key, rho_layer_map

_EPS = 1e-6
PAGE_ALIGN = 64   # page slots and features are padded to this for the MFMA prefill kernels


def l2(x: torch.Tensor) -> torch.Tensor:
    return x / (torch.linalg.vector_norm(x, dim=-1, keepdim=True) + _EPS)


def _get(chunk, name):
    """Field `name` of a chunk given as an object (attribute) or a cache dict (key)."""
    if isinstance(chunk, dict):
        return chunk.get(name)
    return getattr(chunk, name, None)


def _meta_of(chunk) -> dict:
    m = getattr(chunk, "meta", None)
    if m is None and isinstance(chunk, dict):
        m = {k: v for k, v in chunk.items() if k not in ("K", "V")}
    return dict(m or {})


def _assemble(blocks: list[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor]:
    """(padded [C, N_max, d], valid-prefix mask [C, N_max]) from per-chunk blocks [n_c, d]."""
    padded = pad_sequence(blocks, batch_first=True)
    counts = torch.tensor([b.shape[0] for b in blocks], device=padded.device)
    mask = torch.arange(padded.shape[1], device=padded.device)[None, :] < counts[:, None]
    return padded, mask


def masked_mean_l2(K: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """S = L2(sum of the valid rows / max(n_c, 1)) per chunk."""
    m = mask.to(K.dtype)
    total = torch.einsum("cnd,cn->cd", K, m)
    return l2(total / m.sum(1, keepdim=True).clamp_min(1))


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
            raise ValueError(f"got {len(reader_layers)} reader layers for {len(depths)} depths")
        keys = [_get(c, "K") for c in chunks]
        vals = [_get(c, "V") for c in chunks]
        untied = any(v is not None and v is not k for k, v in zip(keys, vals))
        self.depths = depths
        self.reader_layers = list(reader_layers)
        self.rho_of = dict(zip(self.reader_layers, depths))
        self.chunk_meta = list(meta) if meta is not None else [_meta_of(c) for c in chunks]
        self.center = center
        self.K, self.mask, self.S = {}, {}, {}
        self.V = {} if untied else None

        def rows_at(src, rho):
            return [x[rho_key(x, rho)].to(device=device, dtype=dtype) for x in src]

        for li, rho in self.rho_of.items():
            kb = rows_at(keys, rho)
            if center is not None:   # a centre dict must cover every depth (KeyError otherwise)
                mu = center[rho_key(center, rho)].to(device=device, dtype=dtype)
                kb = [l2(b - mu) for b in kb]
            vb = rows_at([v if v is not None else k for k, v in zip(keys, vals)], rho) if untied else None
            self._set_layer(li, kb, vb)
        self._summaries()

    def _set_layer(self, li: int, key_blocks: list, value_blocks: list | None) -> None:
        self.K[li], self.mask[li] = _assemble(key_blocks)
        if value_blocks is not None:
            self.V[li] = _assemble(value_blocks)[0]

    def _summaries(self) -> None:
        self.S = {li: masked_mean_l2(self.K[li], self.mask[li]) for li in self.K}
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
        for table in (self.K, self.S) + ((self.V,) if self.V is not None else ()):
            for li in table:
                table[li] = table[li].to(device=device, dtype=dtype)
        for li in self.mask:
            self.mask[li] = self.mask[li].to(device=device)
        self._paged = {}
        return self

    def subset(self, idx) -> "Library":
        """The Library of chunks `idx` alone: their valid rows reassembled (trimmed to the longest
        of them) and their summaries recomputed."""
        picks = [int(i) for i in idx] if hasattr(idx, "__iter__") else [int(idx)]
        if not picks:
            raise ValueError("subset needs at least one chunk index")
        out = Library.__new__(type(self))
        out.depths, out.reader_layers, out.rho_of = self.depths, self.reader_layers, dict(self.rho_of)
        out.center = self.center
        out.chunk_meta = [self.chunk_meta[i] for i in picks]
        out.K, out.mask, out.S = {}, {}, {}
        out.V = {} if self.V is not None else None
        for li in self.K:
            n = self.n_valid(li).tolist()
            kb = [self.K[li][i, :n[i]] for i in picks]
            vb = [self.V[li][i, :n[i]] for i in picks] if self.V is not None else None
            out._set_layer(li, kb, vb)
        out._summaries()
        return out

    @staticmethod
    def from_doc_cache(cache: dict, reader_model, depths=None, device=None, dtype=torch.float32,
                       center: dict | None = None) -> "Library":
        """From a document cache dict {"depths", "chunks": [{"K": {rho: rows}, "start", "n_tokens"}],
        "doc_id", "encoder"} for the given reader model (depth rho -> its reader layer)."""
        use = sorted(float(r) for r in (depths if depths else cache["depths"]))
        layer_of = rho_layer_map(reader_model, use)
        if device is None:
            device = getattr(reader_model, "device", "cpu")
        doc, enc = cache.get("doc_id", ""), cache.get("encoder", "")
        meta = [dict(doc_id=doc, start=int(ch.get("start", 0)), n_tokens=int(ch.get("n_tokens", 0)), encoder=enc)
                for ch in cache["chunks"]]
        return Library(cache["chunks"], [layer_of[r] for r in use], use, device, dtype, meta=meta, center=center)

    # ------------------------------------------------------------------ device pool
    def paged(self, li: int, device):
        """The HIP read pool of layer li on `device` (kv_skill_v2_amd.ops.PagedLibrary), built on
        first use and cached until the Library changes."""
        from .ops import PagedLibrary

        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        key = (li, device)
        if key not in self._paged:
            V = self.V[li] if self.V is not None else None
            self._paged[key] = PagedLibrary.from_padded(self.K[li], self.mask[li], self.S[li].float(),
                                                        device=device, V=V, pad_to=PAGE_ALIGN)
        return self._paged[key]


__all__ = ["Library", "l2", "masked_mean_l2", "PAGE_ALIGN"]
