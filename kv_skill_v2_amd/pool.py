"""LibraryPool: a static device pool of Library pages that documents are loaded into and evicted
from, with an in-place "active set" view for graph-captured decode steps.

This is the Library-read counterpart of the vLLM plugin's static operator pool
(`Pools(capacity_tokens)`, xenc/d23_vllm_plugin.py:84-119: allocated once, with a zero dummy
block at the end, so captured graphs keep valid pointers while documents come and go).

    pool = LibraryPool(capacity_chunks=4096, slots_per_page=512, d=2048, device="cuda")
    pool.load("doc-a", load_doc_cache(path_a), rho=0.5, center=mu)   # one upload, one build kernel
    lib = pool.activate(["doc-a", "doc-b"])     # PagedLibrary over the static view buffers

- Pages, summary keys and valid counts live in tensors of fixed capacity (+1 zero dummy page).
  `load` writes a document's chunks into a free page range with `xenc_build_pages`: no
  reallocation, so the addresses never change.  `evict` returns the range.
- `activate(docs)` rewrites the static view buffers in place: the page table (chunk -> page),
  the valid counts, the chunk-ordered summary keys (gathered from the pool by a device copy) and
  the per-document chunk offsets.  The returned `PagedLibrary` holds views of those buffers, so
  a HIP graph captured over a read of one active set replays on any later active set with the
  same shape (documents and chunk counts per document); a different shape needs a new capture,
  as in the plugin.
- Loading and activation are host-driven set-up steps (like the plugin's `load_docs` / `fill`);
  nothing in them belongs inside a captured region.
"""

from __future__ import annotations

import torch

from . import ops
from .depth import rho_key


class LibraryPool:
    def __init__(self, capacity_chunks: int, slots_per_page: int, d: int, device, max_docs: int = 64,
                 pad_to: int = 64):
        if capacity_chunks < 1 or slots_per_page < 1 or d < 8 or d % 8 or max_docs < 1:
            raise ValueError("capacity_chunks, slots_per_page >= 1, d a multiple of 8, max_docs >= 1")
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("LibraryPool lives on a ROCm GPU (there is no CPU path)")
        rnd = lambda x: -(-x // pad_to) * pad_to  # noqa: E731
        self.device = device
        self.capacity = int(capacity_chunks)
        self.N = rnd(int(slots_per_page))
        self.d = int(d)
        self.dp = rnd(self.d)
        if self.dp > 4096:
            raise ValueError(f"d={d} pads to {self.dp} > 4096")
        self.dummy = self.capacity                      # the zero page after the capacity
        P = self.capacity + 1
        self.pages = torch.zeros(P, self.N, self.dp, dtype=torch.float16, device=device)
        self.S = torch.zeros(P, self.dp, dtype=torch.float32, device=device)
        self.nvalid = torch.ones(P, dtype=torch.int32, device=device)
        self.free: list[tuple[int, int]] = [(0, self.capacity)]      # (start, length), sorted
        self.docs: dict = {}                    # doc id -> {"start", "chunks", "nvalid"}
        self.max_docs = int(max_docs)
        # Static view buffers of the active set (rewritten in place by activate).
        self.v_page = torch.full((self.capacity,), self.dummy, dtype=torch.int32, device=device)
        self.v_nvalid = torch.ones(self.capacity, dtype=torch.int32, device=device)
        self.v_S = torch.zeros(self.capacity, self.dp, dtype=torch.float32, device=device)
        self.v_ptr = torch.zeros(self.max_docs + 1, dtype=torch.int32, device=device)
        self.active: list = []

    # ------------------------------------------------------------------ documents
    def _alloc(self, n: int) -> int:
        for i, (s, ln) in enumerate(self.free):
            if ln >= n:
                if ln == n:
                    self.free.pop(i)
                else:
                    self.free[i] = (s + n, ln - n)
                return s
        # The reference's static pool reports a full pool as torch.cuda.OutOfMemoryError
        # (xenc/d23_vllm_plugin.py:181-183), the error its serving retry path keys on.
        raise torch.cuda.OutOfMemoryError(f"no free range of {n} pages in the pool (free ranges: {self.free})")

    def _release(self, start: int, n: int) -> None:
        self.free.append((start, n))
        self.free.sort()
        merged: list[tuple[int, int]] = []
        for s, ln in self.free:
            if merged and merged[-1][0] + merged[-1][1] == s:
                merged[-1] = (merged[-1][0], merged[-1][1] + ln)
            else:
                merged.append((s, ln))
        self.free = merged

    def load(self, doc_id, cache: dict, rho: float, center: dict | None = None) -> None:
        """Build the chunks of one document cache (depth rho) into a free page range, centring
        the slot rows by center[rho] when given (xenc/library.py:47-74)."""
        if doc_id in self.docs:
            raise KeyError(f"document {doc_id!r} is already loaded")
        chunks = cache["chunks"]
        if not chunks:
            raise ValueError("a document needs at least one chunk")
        rows = [ch["K"][rho_key(ch["K"], rho)] for ch in chunks]
        n = [int(r.shape[0]) for r in rows]
        if min(n) < 1 or max(n) > self.N:
            raise ValueError(f"chunk rows must lie in [1, {self.N}] (got {min(n)}..{max(n)})")
        if any(r.dim() != 2 or r.shape[-1] != self.d for r in rows):
            raise ValueError(f"chunk rows must be [n_c, {self.d}]")
        mu = None
        if center is not None:
            mu = center[rho_key(center, rho)].to(device=self.device, dtype=torch.float32).contiguous()
            if mu.shape != (self.d,):
                raise ValueError(f"centre must be [{self.d}]")
        C = len(rows)
        start = self._alloc(C)
        try:
            off = [0]
            for c in n:
                off.append(off[-1] + c)
            flat = torch.cat([r.to(torch.float16) for r in rows]).to(self.device).contiguous()
            row_off = torch.tensor(off, dtype=torch.int64, device=self.device)
            ops.build_pages(flat, row_off, self.d, self.N, self.dp, mu,
                            out=(self.pages[start:start + C], self.S[start:start + C],
                                 self.nvalid[start:start + C]))
        except Exception:
            self._release(start, C)
            raise
        self.docs[doc_id] = {"start": start, "chunks": C, "nvalid": n}

    def evict(self, doc_id) -> None:
        """Return a document's pages to the free list (their contents stay until reused).  An
        active document cannot be evicted."""
        if doc_id in self.active:
            raise RuntimeError(f"document {doc_id!r} is in the active set; activate another set first")
        e = self.docs.pop(doc_id)
        self._release(e["start"], e["chunks"])

    # ------------------------------------------------------------------ active set
    def activate(self, doc_ids) -> ops.PagedLibrary:
        """Make documents doc_ids (library g = doc_ids[g]) the active set and return the
        PagedLibrary over the static view buffers."""
        doc_ids = list(doc_ids)
        if not doc_ids or len(doc_ids) > self.max_docs:
            raise ValueError(f"activate 1..{self.max_docs} documents")
        ents = [self.docs[d] for d in doc_ids]
        Ctot = sum(e["chunks"] for e in ents)
        if Ctot > self.capacity:
            raise ValueError("the active set holds more chunks than the pool")
        page = torch.cat([torch.arange(e["start"], e["start"] + e["chunks"], dtype=torch.int32)
                          for e in ents])
        nv = [x for e in ents for x in e["nvalid"]]
        ptr = [0]
        for e in ents:
            ptr.append(ptr[-1] + e["chunks"])
        self.v_page[:Ctot].copy_(page)
        self.v_page[Ctot:].fill_(self.dummy)
        self.v_nvalid[:Ctot].copy_(torch.tensor(nv, dtype=torch.int32))
        self.v_S[:Ctot].copy_(self.S.index_select(0, self.v_page[:Ctot].long()))
        self.v_ptr[:len(ptr)].copy_(torch.tensor(ptr, dtype=torch.int32))
        self.active = doc_ids
        return ops.PagedLibrary(self.pages, self.v_page[:Ctot], self.v_nvalid[:Ctot],
                                self.v_ptr[:len(ptr)], self.v_S[:Ctot],
                                n_chunks=[e["chunks"] for e in ents], nvalid=nv, d_valid=self.d)


__all__ = ["LibraryPool"]
