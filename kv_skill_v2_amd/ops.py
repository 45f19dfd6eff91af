"""Torch-facing operations of the Library read, each a thin call through the C ABI.

`PagedLibrary` is the HBM layout the kernels read: a pool of fp16 pages (one chunk per page,
`slots_per_page` slot rows of `d` halves each), a page table (chunk -> page), per-chunk valid
slot counts, fp32 summary keys and CSR offsets grouping chunks into libraries.  One call can
serve many libraries (the batched paged decode) or one library shared by every query row.

Every function here requires ROCm device tensors and raises otherwise: there is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import _lib
from . import torch_ops  # noqa: F401  (registers the torch.ops.xenc operators)
from ._lib import check, lib, ptr, stream_handle


def _require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} is on {t.device}: the Library read runs only on a ROCm GPU "
                           "(there is no CPU path)")


def _i32(x, device) -> torch.Tensor:
    return torch.as_tensor(x, dtype=torch.int32, device=device).contiguous()


def build_pages(rows: torch.Tensor, row_off: torch.Tensor, d: int, slots_per_page: int, d_pad: int,
                mu: torch.Tensor | None = None, out=None):
    """xenc_build_pages on device-resident input: rows fp16 [R, d] (chunk c = rows
    row_off[c] .. row_off[c+1]-1, row_off int64 [C+1]) -> (pages fp16 [C, slots_per_page, d_pad],
    S fp32 [C, d_pad], nvalid int32 [C]), centring by mu fp32 [d] when given.  out = (pages, S,
    nvalid) writes into existing contiguous tensors of those shapes (e.g. a range of a static
    pool) instead of new ones.  The caller guarantees every chunk has 1 .. slots_per_page rows."""
    for t, name in ((rows, "rows"), (row_off, "row_off")):
        _require_device(t, name)
    if rows.dtype != torch.float16 or rows.dim() != 2 or rows.shape[1] != d or not rows.is_contiguous():
        raise ValueError(f"rows must be contiguous fp16 [R, {d}]")
    if row_off.dtype != torch.int64 or row_off.dim() != 1 or not row_off.is_contiguous():
        raise ValueError("row_off must be contiguous int64 [C+1]")
    if mu is not None and (mu.dtype != torch.float32 or mu.shape != (d,) or not mu.is_contiguous()):
        raise ValueError(f"mu must be contiguous fp32 [{d}]")
    C = row_off.numel() - 1
    dev = rows.device
    if out is None:
        pages = torch.empty(C, slots_per_page, d_pad, dtype=torch.float16, device=dev)
        S = torch.empty(C, d_pad, dtype=torch.float32, device=dev)
        nv = torch.empty(C, dtype=torch.int32, device=dev)
    else:
        pages, S, nv = out
        for t, shape, dt, name in ((pages, (C, slots_per_page, d_pad), torch.float16, "pages"),
                                   (S, (C, d_pad), torch.float32, "S"), (nv, (C,), torch.int32, "nvalid")):
            _require_device(t, name)
            if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous():
                raise ValueError(f"out {name} must be contiguous {dt} {shape}")
    check(lib().xenc_build_pages(ptr(rows), ptr(row_off), C, d, ptr(mu), slots_per_page, d_pad,
                                 ptr(pages), slots_per_page * d_pad, ptr(S), d_pad, ptr(nv),
                                 stream_handle(dev)), "xenc_build_pages")
    return pages, S, nv


@dataclass
class PagedLibrary:
    """Device layout of one or more Libraries (see include/xenc_hip.h)."""

    pages: torch.Tensor          # fp16 [P, slots_per_page, d]
    chunk_page: torch.Tensor     # int32 [Ctot]
    chunk_nvalid: torch.Tensor   # int32 [Ctot]
    chunk_ptr: torch.Tensor      # int32 [G+1]
    S: torch.Tensor              # fp32 [Ctot, d]
    n_chunks: list[int] = field(default_factory=list)   # host copy: chunks per library
    nvalid: list[int] = field(default_factory=list)     # host copy: valid slots per chunk
    values: torch.Tensor | None = None   # fp16 [P, slots_per_page, d] when V is untied from K
    d_valid: int = 0                     # leading feature dims in use (the rest is zero padding)
    _frag: dict = field(default_factory=dict, repr=False, compare=False)
    _plans: dict = field(default_factory=dict, repr=False, compare=False)
    _kept: dict = field(default_factory=dict, repr=False, compare=False)

    def __post_init__(self):
        for name in ("pages", "chunk_page", "chunk_nvalid", "chunk_ptr", "S"):
            _require_device(getattr(self, name), name)
        P, N, d = self.pages.shape
        if self.pages.dtype != torch.float16 or not self.pages.is_contiguous():
            raise ValueError("pages must be a contiguous fp16 [P, slots, d] tensor")
        if d % 8:
            raise ValueError(f"d={d} must be a multiple of 8")
        Ctot = self.chunk_page.numel()
        if self.S.shape != (Ctot, d) or self.S.dtype != torch.float32 or not self.S.is_contiguous():
            raise ValueError(f"S must be contiguous fp32 [{Ctot}, {d}], got {tuple(self.S.shape)}")
        if not self.n_chunks:
            cp = self.chunk_ptr.cpu().tolist()
            self.n_chunks = [b - a for a, b in zip(cp[:-1], cp[1:])]
        if not self.nvalid:
            self.nvalid = self.chunk_nvalid.cpu().tolist()
        if sum(self.n_chunks) != Ctot or min(self.n_chunks) < 1:
            raise ValueError("every library needs >= 1 chunk and chunk_ptr must cover all chunks")
        if min(self.nvalid) < 1 or max(self.nvalid) > N:
            raise ValueError(f"valid slots per chunk must lie in [1, {N}]")
        cpg = self.chunk_page
        if int(cpg.min()) < 0 or int(cpg.max()) >= P:
            raise ValueError(f"page table entries must lie in [0, {P})")
        if self.values is not None:
            _require_device(self.values, "values")
            if (self.values.shape != self.pages.shape or self.values.dtype != torch.float16
                    or not self.values.is_contiguous()):
                raise ValueError("values must be a contiguous fp16 tensor shaped like pages")
        if not 0 < self.d_valid <= d:
            self.d_valid = d

    # ------------------------------------------------------------------ constructors
    @staticmethod
    def from_padded(K: torch.Tensor, mask: torch.Tensor, S: torch.Tensor, device=None, V=None,
                    pad_to: int = 1) -> "PagedLibrary":
        """One library from the reference layout K [C, N, d], mask [C, N] (valid prefix), S [C, d]
        (and untied values V [C, N, d])."""
        return PagedLibrary.from_libraries([(K, mask, S, V)], device=device, pad_to=pad_to)

    @staticmethod
    def from_libraries(libs, device=None, slots_per_page: int | None = None,
                       pad_to: int = 1) -> "PagedLibrary":
        """Several libraries [(K [C,N,d], mask [C,N], S [C,d][, V [C,N,d]]), ...] packed into one
        pool, page id = global chunk id.  Masks must be valid prefixes (slots 0..n-1 valid), as
        Library builds them.  pad_to > 1 rounds d and the page size up to a multiple of it with
        zero features / masked slots (the read is unchanged; the MFMA prefill path needs 64)."""
        device = torch.device(device) if device is not None else libs[0][0].device
        d = libs[0][0].shape[-1]
        rnd = lambda x: -(-x // pad_to) * pad_to  # noqa: E731
        N = rnd(slots_per_page or max(int(lb[0].shape[1]) for lb in libs))
        dp = rnd(d)
        untied = any(len(lb) > 3 and lb[3] is not None for lb in libs)
        pages, vals, Ss, nv, nch = [], [], [], [], []
        for lb in libs:
            K, M, S = lb[:3]
            V = lb[3] if len(lb) > 3 else None
            C, n_max, dk = K.shape
            if dk != d:
                raise ValueError("all libraries must share d")
            cnt = M.sum(-1).to(torch.int64)
            pref = torch.arange(n_max, device=M.device).view(1, -1) < cnt.view(-1, 1)
            if not torch.equal(pref, M.bool()):
                raise ValueError("mask must mark a prefix of valid slots per chunk")
            pg = torch.zeros(C, N, dp, dtype=torch.float16, device=device)
            pg[:, :n_max, :d] = K.to(device=device, dtype=torch.float16)
            pages.append(pg)
            if untied:
                vg = torch.zeros(C, N, dp, dtype=torch.float16, device=device)
                vg[:, :n_max, :d] = (V if V is not None else K).to(device=device, dtype=torch.float16)
                vals.append(vg)
            sp = torch.zeros(C, dp, dtype=torch.float32, device=device)
            sp[:, :d] = S.to(device=device, dtype=torch.float32)
            Ss.append(sp)
            nv += cnt.tolist()
            nch.append(C)
        ptr_ = [0]
        for c in nch:
            ptr_.append(ptr_[-1] + c)
        Ctot = ptr_[-1]
        return PagedLibrary(torch.cat(pages).contiguous(), _i32(list(range(Ctot)), device),
                            _i32(nv, device), _i32(ptr_, device), torch.cat(Ss).contiguous(),
                            n_chunks=nch, nvalid=nv,
                            values=torch.cat(vals).contiguous() if untied else None, d_valid=d)

    @staticmethod
    def from_doc_caches(caches, rho: float, device, center: dict | None = None,
                        slots_per_page: int | None = None, pad_to: int = 64) -> "PagedLibrary":
        """The pool of depth rho for one or more document caches (the dicts load_doc_cache
        returns: {"chunks": [{"K": {rho: fp16 [n_c, d]}, ["V": {...}], ...}], ...}), one library
        per cache, built on the device by xenc_build_pages: the chunk rows go up in one copy and
        one kernel writes the zero-padded fp16 pages, the fp32 summary keys S = L2(masked mean)
        and the valid counts, centring the rows as L2(row - mu) when center = {rho: mu} is given
        (the math of Library.__init__ / _summaries, xenc/library.py:47-74, at the Library's fp32
        precision before the fp16 store).  Untied values are copied uncentred, as the reference
        does."""
        from .depth import rho_key

        device = torch.device(device)
        _require_device(torch.empty(0, device=device), "device")
        if isinstance(caches, dict):
            caches = [caches]
        if not caches:
            raise ValueError("from_doc_caches needs at least one cache")
        rows, vrows, nch = [], [], []
        for cache in caches:
            chunks = cache["chunks"]
            if not chunks:
                raise ValueError("Library needs at least one chunk")
            nch.append(len(chunks))
            for ch in chunks:
                k = ch["K"]
                rows.append(k[rho_key(k, rho)])
                v = ch.get("V") if isinstance(ch, dict) else None
                vrows.append(None if v is None else v[rho_key(v, rho)])
                if vrows[-1] is not None and vrows[-1].shape != rows[-1].shape:
                    raise ValueError("untied values must match the key rows' shape")
        d = int(rows[0].shape[-1])
        n = [int(r.shape[0]) for r in rows]
        if min(n) < 1:
            raise ValueError("every chunk needs at least one slot row")
        if any(r.dim() != 2 or r.shape[-1] != d for r in rows):
            raise ValueError(f"chunk rows must all be [n_c, {d}]")
        rnd = lambda x: -(-x // pad_to) * pad_to  # noqa: E731
        N = rnd(slots_per_page or max(n))
        if N < max(n):
            raise ValueError(f"slots_per_page={N} is below the longest chunk ({max(n)} slots)")
        dp = rnd(d)
        if d % 8 or dp > 4096:
            raise ValueError(f"d={d} must be a multiple of 8 and pad to at most 4096")
        mu = None
        if center is not None:
            mu = center[rho_key(center, rho)].to(device=device, dtype=torch.float32).contiguous()
            if mu.shape != (d,):
                raise ValueError(f"centre must be [{d}], got {tuple(mu.shape)}")
        Ctot = len(rows)
        off = [0]
        for c in n:
            off.append(off[-1] + c)
        off_d = torch.tensor(off, dtype=torch.int64, device=device)

        def flat(src):
            return torch.cat([r.to(torch.float16) for r in src]).to(device).contiguous()

        pages, S, nv = build_pages(flat(rows), off_d, d, N, dp, mu)
        values = None
        if any(v is not None for v in vrows):
            values = build_pages(flat([v if v is not None else k for v, k in zip(vrows, rows)]), off_d,
                                 d, N, dp)[0]
        ptr_ = [0]
        for c in nch:
            ptr_.append(ptr_[-1] + c)
        return PagedLibrary(pages, torch.arange(Ctot, dtype=torch.int32, device=device), nv,
                            _i32(ptr_, device), S, n_chunks=nch, nvalid=n, values=values, d_valid=d)

    # ------------------------------------------------------------------ properties
    @property
    def d(self) -> int:
        return self.pages.shape[-1]

    @property
    def slots_per_page(self) -> int:
        return self.pages.shape[1]

    @property
    def n_libraries(self) -> int:
        return len(self.n_chunks)

    @property
    def cmax(self) -> int:
        return max(self.n_chunks)

    @property
    def device(self) -> torch.device:
        return self.pages.device

    def kept(self, top_k: int) -> int:
        """Width of the routed-index arrays: max over libraries of the kept chunk count (kept per
        top_k: the chunk counts of a pool do not change after construction)."""
        k = self._kept.get(top_k)
        if k is None:
            k = self._kept[top_k] = max(c if (top_k <= 0 or top_k >= c) else top_k for c in self.n_chunks)
        return k

    def check_prefill(self) -> None:
        """The MFMA prefill kernels step d and the slots by 64 and take a page of <= 512 slots."""
        if self.d % 64 or self.slots_per_page % 64 or self.slots_per_page > 512:
            raise ValueError(f"the prefill read needs d % 64 == 0 and slots_per_page % 64 == 0, <= 512 "
                             f"(got d={self.d}, slots={self.slots_per_page}); build the pool with padding")

    def fragment_pages(self, layout: int, values: bool = False) -> torch.Tensor:
        """Fragment-ordered copy of the pages (or of the untied values) for the prefill MFMA
        kernels (layout 0: scores operand, [P][slots/32][d/16][64][8]; layout 1: readout operand,
        [P][d/32][slots/16][64][8]), built on first use by xenc_fragment_pages and kept with the
        pool (the library is resident across steps)."""
        src = self.values if (values and self.values is not None) else self.pages
        key = (layout, src is self.values)
        t = self._frag.get(key)
        if t is None:
            P, N, d = src.shape
            t = torch.empty(P, N, d, dtype=torch.float16, device=self.device)
            check(lib().xenc_fragment_pages(ptr(src), P, N, d, layout, ptr(t),
                                            stream_handle(self.device)), "xenc_fragment_pages")
            self._frag[key] = t
        return t

    def sub_pages(self) -> "SubPages":
        """This pool split into pages of at most SUB_SPAN slots for the MFMA kernels (see
        SubPages), built on first use and kept with the pool."""
        t = self._frag.get("sub")
        if t is None:
            t = self._frag["sub"] = _build_sub_pages(self)
        return t

    def plan(self, rows_per_library) -> "RowPlan":
        """Row plan for this pool, cached per row-count tuple (avoids small host->device copies
        on every step of a fixed-shape loop)."""
        key = tuple(int(r) for r in rows_per_library)
        p = self._plans.get(key)
        if p is None:
            if len(self._plans) >= 64:
                self._plans.clear()
            p = self._plans[key] = row_plan(self, key)
        return p


def _groups(lib_: PagedLibrary, M: int, q_group) -> torch.Tensor:
    if (isinstance(q_group, torch.Tensor) and q_group.is_cuda and q_group.dtype == torch.int32
            and q_group.dim() == 1 and q_group.shape[0] == M and q_group.is_contiguous()
            and q_group.device == lib_.device):
        return q_group          # the per-token path: already a device int32 vector
    if q_group is None:
        if lib_.n_libraries != 1:
            raise ValueError("q_group is required when the pool holds several libraries")
        return torch.zeros(M, dtype=torch.int32, device=lib_.device)
    if not isinstance(q_group, torch.Tensor) or not q_group.is_cuda:
        gh = torch.as_tensor(q_group)
        if gh.numel() and (int(gh.min()) < 0 or int(gh.max()) >= lib_.n_libraries):
            raise ValueError(f"q_group entries must lie in [0, {lib_.n_libraries})")
    g = torch.as_tensor(q_group, device=lib_.device).to(torch.int32).contiguous()
    if g.shape != (M,):
        raise ValueError(f"q_group must have shape ({M},)")
    # Device-resident q_group is not read back (no host sync); the kernels clamp it to a library.
    return g


def _query(q: torch.Tensor, d: int) -> torch.Tensor:
    _require_device(q, "q")
    if q.dim() != 2 or q.shape[1] != d:
        raise ValueError(f"q must be [M, {d}], got {tuple(q.shape)}")
    if q.dtype != torch.float32:
        q = q.to(torch.float32)
    if q.stride(1) != 1 or q.stride(0) % 4 or q.data_ptr() % 16:
        q = q.contiguous()
    return q


def route_topk(q: torch.Tensor, lib_: PagedLibrary, q_group=None, top_k: int = 0,
               route_temp: float = 10.0):
    """(w_dense [M, cmax], idx [M, kk] int32, w_sel [M, kk]) for query rows q [M, d].

    Operator xenc::route_topk (HIP route kernels, kv_skill_v2_amd/csrc/route.hip); replaces
    LibraryInjector.route (xenc/injector.py:220-229)."""
    q = _query(q, lib_.d)
    g = _groups(lib_, q.shape[0], q_group)
    return torch.ops.xenc.route_topk(q, lib_.S, lib_.chunk_ptr, g, int(top_k), float(route_temp), lib_.cmax,
                                     lib_.kept(int(top_k)))


def default_nsplit(units: int, slots_per_page: int) -> int:
    """Slot splits per routed page.  With >= 128 (query, page) units one workgroup per page
    (measured best on the B = 64 batched decode); fewer units are split so that about
    min(8 * units, 128) workgroups stream the pages, in pieces of >= 32 slots.  Very few units
    stay at 8 splits per page because the last workgroup merges every partial: one query x 4
    pages (the single-sequence decode) measured 34.4 / 23.4 / 18.9 / 17.8 / 20.0 / 26.9 us per
    step at 1 / 2 / 4 / 8 / 16 / 32 splits."""
    units = max(units, 1)
    want = max(1, math.ceil(min(8 * units, 128) / units))
    return int(max(1, min(want, max(1, slots_per_page // 32), 64)))


class _Workspaces:
    """Decode workspaces, one per (device, stream), grown on demand.  A workspace serves calls of
    up to `rows` query rows (its capacity, passed to every call); its arrival counters are zeroed
    once by a kernel (xenc_decode_workspace_init) and every call leaves them zero."""

    def __init__(self):
        self._ws = {}
        self._fits = set()       # (device, stream, M, kk, nsplit, d) already checked to fit

    def get(self, device: torch.device, stream: int, M: int, kk: int, nsplit: int, d: int):
        key = (device.index, stream)
        hit = self._ws.get(key)
        if hit is not None and (key, M, kk, nsplit, d) in self._fits:
            return hit
        buf, rows = hit if hit is not None else (None, 0)
        L = lib()
        if buf is None or rows < M or buf.numel() < L.xenc_decode_workspace_bytes(rows, kk, nsplit, d):
            rows = max(rows, M, 64)
            size = L.xenc_decode_workspace_bytes(rows, kk, nsplit, d)
            if buf is not None:
                size = max(size, buf.numel())
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            check(L.xenc_decode_workspace_init(ptr(buf), size, rows, stream), "xenc_decode_workspace_init")
            self._ws[key] = (buf, rows)
            self._fits = {f for f in self._fits if f[0] != key}
        self._fits.add((key, M, kk, nsplit, d))
        return buf, rows


_WORKSPACES = _Workspaces()


def library_read_decode(q: torch.Tensor, lib_: PagedLibrary, idx: torch.Tensor, w_sel: torch.Tensor,
                        q_group=None, read_temp: float = 12.0, softmax: bool = True,
                        nsplit: int | None = None) -> torch.Tensor:
    """r [M, d] fp32: route-weighted masked-softmax (or linear) read over the routed pages.

    HIP kernel `decode_read_kernel` (kv_skill_v2_amd/csrc/decode.hip: split-K partials merged by
    the last-arriving workgroup of each query row);
    replaces the read of LibraryInjector._branch (xenc/injector.py:239-265)."""
    q = _query(q, lib_.d)
    M = q.shape[0]
    if lib_.values is not None:
        raise ValueError("the decode kernel reads K = V tied pages; untied values take the prefill path")
    g = _groups(lib_, M, q_group)
    _require_device(idx, "idx")
    if idx.dim() != 2 or idx.shape[0] != M or w_sel.shape != idx.shape:
        raise ValueError("idx and w_sel must both be [M, kk]")
    idx = idx.to(torch.int32).contiguous()
    w_sel = w_sel.to(torch.float32).contiguous()
    kk = idx.shape[1]
    if M == 0 or kk == 0:
        return torch.zeros(M, lib_.d, dtype=torch.float32, device=q.device)
    ns = int(nsplit) if nsplit is not None else default_nsplit(M * kk, lib_.slots_per_page)
    ws, rows = _WORKSPACES.get(q.device, stream_handle(q.device), M, kk, ns, lib_.d)
    return torch.ops.xenc.library_read(q, lib_.pages, lib_.chunk_page, lib_.chunk_nvalid, lib_.chunk_ptr, g,
                                       idx, w_sel, float(read_temp), bool(softmax), ns, ws, rows)


def route_read_decode(q: torch.Tensor, lib_: PagedLibrary, q_group=None, top_k: int = 0,
                      route_temp: float = 10.0, read_temp: float = 12.0, softmax: bool = True,
                      nsplit: int | None = None):
    """(w [M, cmax], idx [M, kk], w_sel [M, kk], r [M, d]): route_topk and library_read_decode in
    one operator call (xenc::route_read), equal to them bit for bit.  When every library has at
    most 64 chunks and the rows do not share libraries, the top-k + softmax runs in the read
    kernel's prologue: one launch fewer per step (LibraryInjector.route and the read of _branch,
    xenc/injector.py:220-265)."""
    q = _query(q, lib_.d)
    M = q.shape[0]
    if lib_.values is not None:
        raise ValueError("the decode kernel reads K = V tied pages; untied values take the prefill path")
    g = _groups(lib_, M, q_group)
    kk = lib_.kept(int(top_k))
    ns = int(nsplit) if nsplit is not None else default_nsplit(M * kk, lib_.slots_per_page)
    ws, rows = _WORKSPACES.get(q.device, stream_handle(q.device), max(M, 1), kk, ns, lib_.d)
    return torch.ops.xenc.route_read(q, lib_.S, lib_.pages, lib_.chunk_page, lib_.chunk_nvalid, lib_.chunk_ptr, g,
                                     int(top_k), float(route_temp), lib_.cmax, kk, float(read_temp), bool(softmax),
                                     ns, ws, rows)


# ---------------------------------------------------------------------------------------------
# Prefill / registration read (MFMA) and the autograd of routing + read
ROWS_SCORES, ROWS_READOUT, ROWS_ROUTE_BWD = 128, 128, 16
ROUTE_TILE = 32            # rows and chunks per tile of the many-row routing kernel
ROUTE_ROWS_MIN = 64        # from this many rows differentiable routing uses the many-row routing kernel


def write_back(r: torch.Tensor, W: torch.Tensor, row_group: torch.Tensor | None = None,
               bias: torch.Tensor | None = None, row_scale: torch.Tensor | None = None) -> torch.Tensor:
    """out[m] = row_scale[m] * (W[g_m] @ r[m] + bias[g_m]) on xenc_write_back: the write of the
    decode path's epilogue (xenc/injector.py:71-74, 266-267).  r fp32 [M, d]; W fp32 [d_out, d]
    (one library) or [G, d_out, d] (one weight per library / depth, selected by row_group int32
    [M]); bias [d_out] or [G, d_out]; row_scale fp32 [M].  Returns fp32 [M, d_out]."""
    _require_device(r, "r")
    _require_device(W, "W")
    if r.dtype != torch.float32 or r.dim() != 2 or r.stride(1) != 1:
        raise ValueError("r must be fp32 [M, d] with unit column stride")
    if W.dtype != torch.float32 or W.dim() not in (2, 3) or W.stride(-1) != 1:
        raise ValueError("W must be fp32 [d_out, d] or [G, d_out, d] with unit column stride")
    W3 = W if W.dim() == 3 else W.unsqueeze(0)
    G, d_out, d = W3.shape
    M = r.shape[0]
    if r.shape[1] != d:
        raise ValueError(f"r has {r.shape[1]} columns, W takes {d}")
    if row_group is not None:
        _require_device(row_group, "row_group")
        if row_group.dtype != torch.int32 or row_group.shape != (M,) or not row_group.is_contiguous():
            raise ValueError("row_group must be contiguous int32 [M]")
    if bias is not None:
        _require_device(bias, "bias")
        b2 = bias if bias.dim() == 2 else bias.unsqueeze(0)
        if bias.dtype != torch.float32 or b2.shape[-1] != d_out or b2.shape[0] not in (1, G) or b2.stride(-1) != 1:
            raise ValueError(f"bias must be fp32 [{d_out}] or [{G}, {d_out}]")
        if b2.shape[0] != G:
            b2 = b2.expand(G, d_out)
    if row_scale is not None:
        _require_device(row_scale, "row_scale")
        if row_scale.dtype != torch.float32 or row_scale.shape != (M,) or not row_scale.is_contiguous():
            raise ValueError("row_scale must be contiguous fp32 [M]")
    out = torch.empty(M, d_out, dtype=torch.float32, device=r.device)
    check(lib().xenc_write_back(ptr(r), r.stride(0), M, d, ptr(row_group), G, ptr(W3), W3.stride(0),
                                W3.stride(1), d_out, ptr(bias), b2.stride(0) if bias is not None else 0,
                                ptr(row_scale), ptr(out), out.stride(0), stream_handle(r.device)),
          "xenc_write_back")
    return out


def selector_weights(z: torch.Tensor, k: int):
    """(w [B, n] dense, idx int32 [B, k], w_sel [B, k]) on xenc_selector_weights: top-k of each
    row of z fp32 [B, n] (descending, ties to the lower index), softmax over the kept logits
    (LayerSelector._weights_from_logits, xenc/selector.py:59-67)."""
    _require_device(z, "z")
    if z.dtype != torch.float32 or z.dim() != 2 or z.stride(1) != 1:
        raise ValueError("z must be fp32 [B, n] with unit column stride")
    B, n = z.shape
    w = torch.empty(B, n, dtype=torch.float32, device=z.device)
    idx = torch.empty(B, k, dtype=torch.int32, device=z.device)
    w_sel = torch.empty(B, k, dtype=torch.float32, device=z.device)
    check(lib().xenc_selector_weights(ptr(z), z.stride(0), B, n, int(k), ptr(w), w.stride(0), ptr(idx),
                                      ptr(w_sel), k, stream_handle(z.device)), "xenc_selector_weights")
    return w, idx, w_sel


def selector_apply(delta: torch.Tensor, h: torch.Tensor, w_row: torch.Tensor, log_alpha,
                   k: int = 1) -> torch.Tensor:
    """out [B, d] = sum over a token's k rows of w * exp(log_alpha) * delta / (|delta| / (|h| + 1e-6)
    + 1e-6) on xenc_selector_apply (LayerSelector.apply, xenc/selector.py:106-110, summed over
    the k selected layers).  delta fp32 [B * k, d] (the k rows of token b at b*k .. b*k+k-1),
    h fp32 [B, d], w_row fp32 [B * k]; log_alpha a float or a device scalar tensor (read by the
    kernel: no host synchronisation)."""
    for t, n in ((delta, "delta"), (h, "h"), (w_row, "w_row")):
        _require_device(t, n)
    if delta.dtype != torch.float32 or h.dtype != torch.float32 or w_row.dtype != torch.float32:
        raise ValueError("delta, h and w_row must be fp32")
    if delta.dim() != 2 or h.dim() != 2 or delta.stride(1) != 1 or h.stride(1) != 1:
        raise ValueError("delta and h must be 2-D with unit column stride")
    B, d = h.shape
    if delta.shape != (B * k, d) or w_row.numel() != B * k:
        raise ValueError(f"delta must be [{B * k}, {d}] and w_row [{B * k}]")
    w_row = w_row.reshape(-1).contiguous()
    la = (log_alpha.detach().float().reshape(1).to(h.device) if isinstance(log_alpha, torch.Tensor)
          else torch.full((1,), float(log_alpha), dtype=torch.float32, device=h.device))
    out = torch.empty(B, d, dtype=torch.float32, device=h.device)
    check(lib().xenc_selector_apply(B, int(k), d, ptr(delta), delta.stride(0), ptr(h), h.stride(0), ptr(w_row),
                                    ptr(la), ptr(out), out.stride(0), stream_handle(h.device)),
          "xenc_selector_apply")
    return out


def gate_scale(hn: torch.Tensor, gate_w: torch.Tensor, gate_b: torch.Tensor, log_gain: torch.Tensor,
               gain_scale: float = 1.0, row_token: torch.Tensor | None = None,
               row_pos: torch.Tensor | None = None) -> torch.Tensor:
    """scale [M] = gain_scale * exp(log_gain[p]) * sigmoid(hn[t] . gate_w + gate_b[p]) on
    xenc_gate_scale (itf_gate, itf_gain, xenc/injector.py:59-69); t = row_token[m] (default m),
    p = row_pos[m] (default 0).  hn fp32 [*, d]; gate_b, log_gain fp32 [n_pos]."""
    for t, n in ((hn, "hn"), (gate_w, "gate_w"), (gate_b, "gate_b"), (log_gain, "log_gain")):
        _require_device(t, n)
    if hn.dtype != torch.float32 or hn.dim() != 2 or hn.stride(1) != 1:
        raise ValueError("hn must be fp32 [rows, d] with unit column stride")
    d = hn.shape[1]
    gw, gb, lg = (t.detach().float().reshape(-1).contiguous() for t in (gate_w, gate_b, log_gain))
    if gw.numel() != d or gb.numel() != lg.numel() or gb.numel() < 1:
        raise ValueError("gate_w must have d entries and gate_b / log_gain one per position")
    M = hn.shape[0] if row_token is None else row_token.numel()
    rt = None if row_token is None else row_token.to(torch.int32).reshape(-1).contiguous()
    rp = None if row_pos is None else row_pos.to(torch.int32).reshape(-1).contiguous()
    if rp is not None and rp.numel() != M:
        raise ValueError("row_pos must have one entry per row")
    out = torch.empty(M, dtype=torch.float32, device=hn.device)
    check(lib().xenc_gate_scale(M, d, ptr(hn), hn.stride(0), ptr(rt), ptr(rp), gb.numel(), ptr(gw), ptr(gb),
                                ptr(lg), float(gain_scale), ptr(out), stream_handle(hn.device)), "xenc_gate_scale")
    return out


def multi_depth_prepare(z: torch.Tensor, k: int, q_all: torch.Tensor, hn: torch.Tensor,
                        gate_w: torch.Tensor, gate_b: torch.Tensor, log_gain: torch.Tensor,
                        gain_scale: float = 1.0):
    """The per-token work of a multi-depth decode step in one launch (xenc_multi_depth_prepare):
    z fp32 [B, L] selector logits, q_all fp32 [L, B, d] each depth's query rows, hn fp32 [B, d_r].
    Returns (w [B, L], top int32 [B, k], wtop [B, k], q_rows [B*k, d], scale [B*k]): the
    selector_weights outputs, q_rows[b*k + j] = q_all[top[b, j], b] and scale[b*k + j] =
    gate_scale(hn, ..., row_token=b, row_pos=top[b, j]) — each equal to the separate calls."""
    for t, n in ((z, "z"), (q_all, "q_all"), (hn, "hn"), (gate_w, "gate_w"), (gate_b, "gate_b"),
                 (log_gain, "log_gain")):
        _require_device(t, n)
    if z.dtype != torch.float32 or z.dim() != 2 or z.stride(1) != 1:
        raise ValueError("z must be fp32 [B, L] with unit column stride")
    B, L = z.shape
    if q_all.dtype != torch.float32 or q_all.dim() != 3 or q_all.shape[:2] != (L, B) or q_all.stride(2) != 1:
        raise ValueError(f"q_all must be fp32 [{L}, {B}, d] with unit column stride")
    if hn.dtype != torch.float32 or hn.dim() != 2 or hn.shape[0] != B or hn.stride(1) != 1:
        raise ValueError(f"hn must be fp32 [{B}, d_r] with unit column stride")
    d, d_r = q_all.shape[2], hn.shape[1]
    gw, gb, lg = (t.detach().float().reshape(-1).contiguous() for t in (gate_w, gate_b, log_gain))
    if gw.numel() != d_r or gb.numel() != L or lg.numel() != L:
        raise ValueError(f"gate_w must have {d_r} entries and gate_b / log_gain one per depth ({L})")
    dev = z.device
    w = torch.empty(B, L, dtype=torch.float32, device=dev)
    top = torch.empty(B, k, dtype=torch.int32, device=dev)
    wtop = torch.empty(B, k, dtype=torch.float32, device=dev)
    q_rows = torch.empty(B * k, d, dtype=torch.float32, device=dev)
    scale = torch.empty(B * k, dtype=torch.float32, device=dev)
    check(lib().xenc_multi_depth_prepare(ptr(z), z.stride(0), B, L, int(k), ptr(q_all), q_all.stride(0),
                                         q_all.stride(1), d, ptr(hn), hn.stride(0), d_r, ptr(gw), ptr(gb),
                                         ptr(lg), float(gain_scale), ptr(w), w.stride(0), ptr(top), ptr(wtop),
                                         k, ptr(q_rows), q_rows.stride(0), ptr(scale), stream_handle(dev)),
          "xenc_multi_depth_prepare")
    return w, top, wtop, q_rows, scale


def multi_depth_prepare_route(z: torch.Tensor, k: int, q_all: torch.Tensor, hn: torch.Tensor,
                              gate_w: torch.Tensor, gate_b: torch.Tensor, log_gain: torch.Tensor,
                              lib_: PagedLibrary, top_k: int = 0, route_temp: float = 10.0,
                              gain_scale: float = 1.0):
    """multi_depth_prepare, then route_topk of its q_rows with each row's depth as its library,
    with the routing dots in the same launch as the per-token work (xenc_multi_depth_prepare_route;
    at most 64 depths).  Returns (w, top, wtop, q_rows, scale, w_route [B*k, cmax], idx [B*k, kk],
    w_sel [B*k, kk]), equal bit for bit to the two calls (LayerSelector._weights_from_logits and
    LibraryInjector.route at each kept layer: xenc/selector.py:59-67, xenc/injector.py:220-229)."""
    for t, n in ((z, "z"), (q_all, "q_all"), (hn, "hn"), (gate_w, "gate_w"), (gate_b, "gate_b"),
                 (log_gain, "log_gain")):
        _require_device(t, n)
    if z.dtype != torch.float32 or z.dim() != 2 or z.stride(1) != 1:
        raise ValueError("z must be fp32 [B, L] with unit column stride")
    B, L = z.shape
    if L != lib_.n_libraries:
        raise ValueError(f"the pool must hold one library per depth ({L}), it holds {lib_.n_libraries}")
    if L > 64:
        raise ValueError("at most 64 depths")
    if q_all.dtype != torch.float32 or q_all.dim() != 3 or q_all.shape[:2] != (L, B) or q_all.shape[2] != lib_.d:
        raise ValueError(f"q_all must be fp32 [{L}, {B}, {lib_.d}]")
    if q_all.stride(2) != 1 or q_all.stride(0) % 4 or q_all.stride(1) % 4 or q_all.data_ptr() % 16:
        q_all = q_all.contiguous()
    if hn.dtype != torch.float32 or hn.dim() != 2 or hn.shape[0] != B or hn.stride(1) != 1:
        raise ValueError(f"hn must be fp32 [{B}, d_r] with unit column stride")
    d, d_r = lib_.d, hn.shape[1]
    gw, gb, lg = (t.detach().float().reshape(-1).contiguous() for t in (gate_w, gate_b, log_gain))
    if gw.numel() != d_r or gb.numel() != L or lg.numel() != L:
        raise ValueError(f"gate_w must have {d_r} entries and gate_b / log_gain one per depth ({L})")
    dev = z.device
    kk = lib_.kept(int(top_k))
    w = torch.empty(B, L, dtype=torch.float32, device=dev)
    top = torch.empty(B, k, dtype=torch.int32, device=dev)
    wtop = torch.empty(B, k, dtype=torch.float32, device=dev)
    q_rows = torch.empty(B * k, d, dtype=torch.float32, device=dev)
    scale = torch.empty(B * k, dtype=torch.float32, device=dev)
    w_route = torch.empty(B * k, lib_.cmax, dtype=torch.float32, device=dev)
    idx = torch.empty(B * k, kk, dtype=torch.int32, device=dev)
    w_sel = torch.empty(B * k, kk, dtype=torch.float32, device=dev)
    check(lib().xenc_multi_depth_prepare_route(
        ptr(z), z.stride(0), B, L, int(k), ptr(q_all), q_all.stride(0), q_all.stride(1), d, ptr(hn),
        hn.stride(0), d_r, ptr(gw), ptr(gb), ptr(lg), float(gain_scale), ptr(w), w.stride(0), ptr(top),
        ptr(wtop), k, ptr(q_rows), q_rows.stride(0), ptr(scale), ptr(lib_.S), ptr(lib_.chunk_ptr), L,
        int(top_k), float(route_temp), ptr(w_route), w_route.stride(0), ptr(idx), ptr(w_sel), kk,
        stream_handle(dev)), "xenc_multi_depth_prepare_route")
    return w, top, wtop, q_rows, scale, w_route, idx, w_sel


def select_scores(q: torch.Tensor, keys: torch.Tensor, valid: torch.Tensor | None = None,
                  pool: str = "max") -> torch.Tensor:
    """Pooled selection scores [B, S] on xenc_select_scores: q fp32 [B, n_q, hd] (one position),
    keys fp32 [S, n_kv, hd], valid bool [S] (xenc/topk_read.py:205-226)."""
    for t, n in ((q, "q"), (keys, "keys")):
        _require_device(t, n)
    if q.dtype != torch.float32 or keys.dtype != torch.float32 or q.dim() != 3 or keys.dim() != 3:
        raise ValueError("q [B, n_q, hd] and keys [S, n_kv, hd] must be fp32")
    B, n_q, hd = q.shape
    S, n_kv, hk = keys.shape
    if hk != hd or n_q % n_kv:
        raise ValueError(f"head dims {hd} / {hk} or groups {n_q} / {n_kv} do not match")
    if pool not in ("max", "mean"):
        raise ValueError(f"unknown pool {pool!r}")
    q, keys = q.contiguous(), keys.contiguous()
    vb = None
    if valid is not None:
        _require_device(valid, "valid")
        if valid.numel() != S:
            raise ValueError(f"valid must have {S} entries")
        vb = valid.reshape(-1).to(torch.uint8).contiguous()
    out = torch.empty(B, S, dtype=torch.float32, device=q.device)
    check(lib().xenc_select_scores(ptr(q), B, n_q, n_kv, hd, ptr(keys), S, ptr(vb), int(pool == "mean"),
                                   ptr(out), out.stride(0), stream_handle(q.device)), "xenc_select_scores")
    return out


def topk_rows(scores: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(idx int32 [B, k], values [B, k]): the k largest entries of each row of scores fp32 [B, S]
    in descending order, ties to the lower index, on xenc_topk_rows."""
    _require_device(scores, "scores")
    if scores.dtype != torch.float32 or scores.dim() != 2 or scores.stride(1) != 1:
        raise ValueError("scores must be fp32 [B, S] with unit column stride")
    B, S = scores.shape
    idx = torch.empty(B, k, dtype=torch.int32, device=scores.device)
    vals = torch.empty(B, k, dtype=torch.float32, device=scores.device)
    check(lib().xenc_topk_rows(ptr(scores), scores.stride(0), B, S, int(k), ptr(idx), ptr(vals), k,
                               stream_handle(scores.device)), "xenc_topk_rows")
    return idx, vals


def gather_library(lib_: PagedLibrary, idx: torch.Tensor, n_flat: int, pad_to: int = 64) -> PagedLibrary:
    """One-chunk libraries of the selected slots: set g's chunk holds the slot rows of the flat
    indices idx[g, :k] (chunk f // n_flat, slot f % n_flat of lib_'s single library), in
    selection order, zero-padded to a multiple of pad_to slots; values are gathered the same way
    when lib_ carries untied values.  Reading it with route weight 1 is the read over the selected
    slots (xenc/topk_read.py:390-410)."""
    _single(lib_)
    _require_device(idx, "idx")
    if idx.dim() != 2:
        raise ValueError("idx must be [G, k]")
    G, k = idx.shape
    if k < 1:
        raise ValueError("select at least one slot")
    kpad = -(-k // pad_to) * pad_to
    ii = idx.to(torch.int32).contiguous()
    dev = lib_.device

    def gather(src):
        out = torch.empty(G, kpad, lib_.d, dtype=torch.float16, device=dev)
        check(lib().xenc_gather_pages(ptr(src), lib_.slots_per_page, lib_.slots_per_page * lib_.d, lib_.d,
                                      ptr(lib_.chunk_page), lib_.chunk_page.numel(), int(n_flat), ptr(ii), k,
                                      G, k, kpad, ptr(out), stream_handle(dev)), "xenc_gather_pages")
        return out

    pages = gather(lib_.pages)
    values = gather(lib_.values) if lib_.values is not None else None
    return PagedLibrary(pages, torch.arange(G, dtype=torch.int32, device=dev),
                        torch.full((G,), k, dtype=torch.int32, device=dev),
                        torch.arange(G + 1, dtype=torch.int32, device=dev),
                        torch.zeros(G, lib_.d, dtype=torch.float32, device=dev),
                        n_chunks=[1] * G, nvalid=[k] * G, values=values, d_valid=lib_.d_valid)


def _prefix(counts) -> list[int]:
    out = [0]
    for c in counts:
        out.append(out[-1] + int(c))
    return out


@dataclass
class RowPlan:
    """Query rows grouped by library (rows of library g are contiguous) and the per-library tile
    offsets each prefill kernel walks.  Built on the host once per (pool, rows) shape."""

    rows: list[int]
    row_ptr: torch.Tensor
    score_tiles: torch.Tensor
    n_score: int
    readout_tiles: torch.Tensor
    n_readout: int
    route_tiles: torch.Tensor
    n_route: int
    logit_tiles: torch.Tensor
    n_logit: int

    @property
    def M(self) -> int:
        return sum(self.rows)


def row_plan(lib_: PagedLibrary, rows_per_library) -> RowPlan:
    rows = [int(r) for r in rows_per_library]
    if len(rows) != lib_.n_libraries or min(rows) < 0:
        raise ValueError(f"need one non-negative row count per library ({lib_.n_libraries})")
    dev = lib_.device
    d_tiles = -(-lib_.d // 256)
    sc = _prefix(-(-t // ROWS_SCORES) * c for t, c in zip(rows, lib_.n_chunks))
    ro = _prefix(-(-t // ROWS_READOUT) * d_tiles for t in rows)
    rb = _prefix(-(-t // ROWS_ROUTE_BWD) for t in rows)
    lg = _prefix(-(-t // ROUTE_TILE) * -(-c // ROUTE_TILE) for t, c in zip(rows, lib_.n_chunks))
    return RowPlan(rows, _i32(_prefix(rows), dev), _i32(sc, dev), sc[-1], _i32(ro, dev), ro[-1],
                   _i32(rb, dev), rb[-1], _i32(lg, dev), lg[-1])


def cast_f16(x: torch.Tensor) -> torch.Tensor:
    """fp32 rows -> contiguous fp16 rows (HIP cast kernel)."""
    _require_device(x, "x")
    x = x.to(torch.float32)
    if x.stride(-1) != 1 or x.stride(0) % 4 or x.data_ptr() % 16:
        x = x.contiguous()
    M, d = x.shape
    y = torch.empty(M, d, dtype=torch.float16, device=x.device)
    check(lib().xenc_cast_rows_f16(ptr(x), x.stride(0), M, d, ptr(y), stream_handle(x.device)),
          "xenc_cast_rows_f16")
    return y


def unpack_p(p: torch.Tensor, M: int) -> torch.Tensor:
    """Octet-major p / dS [cmax*slots/8, M, 8] -> row-major [M, cmax*slots] (a view copy)."""
    return p.view(-1, M, 8).permute(1, 0, 2).reshape(M, -1)


def _prefill_operands(lib_: PagedLibrary, plan: RowPlan) -> tuple:
    """The pool's tensor operands of xenc::library_prefill_fwd / _bwd_dq after q (and qh), w."""
    return (lib_.fragment_pages(0), lib_.fragment_pages(1, values=True), lib_.fragment_pages(0, values=True),
            lib_.fragment_pages(1), lib_.chunk_ptr, lib_.chunk_page, lib_.chunk_nvalid, plan.row_ptr,
            plan.score_tiles, plan.readout_tiles, plan.n_score, plan.n_readout, lib_.slots_per_page)


def prefill_forward(q: torch.Tensor, w: torch.Tensor, lib_: PagedLibrary, plan: RowPlan,
                    read_temp: float = 12.0, softmax: bool = True, qh: torch.Tensor | None = None):
    """(r [M, d] fp32, p fp16 octet-major [cmax*slots/8, M, 8]): the route-weighted masked-softmax
    (or linear) read of many query rows, operator xenc::library_prefill_fwd (HIP kernels
    scores_kernel<0|2> + readout_kernel, kv_skill_v2_amd/csrc/prefill.hip); differentiable in q
    and w.  unpack_p gives p row-major.  qh: q as fp16 rows already (route_topk_rows(...,
    emit_f16=True) writes them); cast here when not given."""
    lib_.check_prefill()
    q = _query(q, lib_.d)
    M, d = q.shape
    if M != plan.M or w.shape != (M, lib_.cmax):
        raise ValueError(f"q must have {plan.M} rows and w shape ({plan.M}, {lib_.cmax})")
    if w.dtype != torch.float32 or not w.is_contiguous():
        w = w.to(torch.float32).contiguous()
    if qh is not None and (qh.dtype != torch.float16 or qh.shape != (M, d) or not qh.is_contiguous()):
        raise ValueError(f"qh must be contiguous fp16 [{M}, {d}]")
    fk, fv, fvs, fkr, *rest = _prefill_operands(lib_, plan)
    ragged = min(lib_.n_chunks) != lib_.cmax
    return torch.ops.xenc.library_prefill_fwd(q, qh, w, fk, fv, fvs, fkr, *rest, float(read_temp), bool(softmax),
                                              ragged)


def prefill_backward(g: torch.Tensor, w: torch.Tensor, p: torch.Tensor, lib_: PagedLibrary,
                     plan: RowPlan, read_temp: float = 12.0, softmax: bool = True):
    """(dq through the read [M, d] fp32, gamma = dL/dw through the read [M, cmax] fp32) given the
    upstream gradient g = dL/dr: operator xenc::library_prefill_bwd_dq (scores_kernel<1|3>,
    u = g . V, then readout_kernel, dq = dS . K)."""
    g = _query(g, lib_.d)
    M, d = g.shape
    w = w.to(torch.float32).contiguous()
    if p.shape != (lib_.cmax * lib_.slots_per_page // 8, M, 8) or not p.is_contiguous():
        raise ValueError("p must be the octet-major probabilities prefill_forward returned")
    _, _, fvs, fkr, *rest = _prefill_operands(lib_, plan)
    return torch.ops.xenc.library_prefill_bwd_dq(g, w, p, fvs, fkr, *rest, float(read_temp), bool(softmax))


def prefill_backward_routed(g: torch.Tensor, w: torch.Tensor, p: torch.Tensor, lib_: PagedLibrary, plan: RowPlan,
                            read_temp: float = 12.0, softmax: bool = True, route_temp: float = 10.0,
                            dw_ext: torch.Tensor | None = None) -> torch.Tensor:
    """dq [M, d] fp32 through the read and the routing, given g = dL/dr (and dw_ext, the gradient
    that reaches w from elsewhere): operator xenc::library_prefill_bwd_routed (scores_kernel<1|3>,
    then route_coef_kernel and readout_kernel with the routing term folded in).  Equals
    prefill_backward's dq followed by route_backward with dw = gamma, in one pass over dq."""
    g = _query(g, lib_.d)
    M, d = g.shape
    w = w.to(torch.float32).contiguous()
    if p.shape != (lib_.cmax * lib_.slots_per_page // 8, M, 8) or not p.is_contiguous():
        raise ValueError("p must be the octet-major probabilities prefill_forward returned")
    if dw_ext is not None:
        if dw_ext.shape != w.shape:
            raise ValueError(f"dw_ext must have shape {tuple(w.shape)}")
        dw_ext = dw_ext.to(torch.float32).contiguous()
    _, _, fvs, fkr, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, st, rt, n_s, n_r, slots = _prefill_operands(lib_, plan)
    return torch.ops.xenc.library_prefill_bwd_routed(g, w, p, dw_ext, lib_.S, fvs, fkr, chunk_ptr, chunk_page,
                                                     chunk_nvalid, row_ptr, st, rt, n_s, n_r, slots, float(read_temp),
                                                     bool(softmax), float(route_temp))


def route_backward(w: torch.Tensor, dw: torch.Tensor, lib_: PagedLibrary, plan: RowPlan,
                   route_temp: float, dq: torch.Tensor, dw_ext: torch.Tensor | None = None) -> torch.Tensor:
    """dq += route_temp * sum_c w (dw - sum w dw) S_c, in place (operator xenc::route_backward_)."""
    w = w.to(torch.float32).contiguous()
    dw = dw.to(torch.float32).contiguous()
    if dw_ext is not None:
        dw_ext = dw_ext.to(torch.float32).contiguous()
    torch.ops.xenc.route_backward_(dq, w, dw, dw_ext, lib_.S, lib_.chunk_ptr, plan.row_ptr, plan.route_tiles,
                                   plan.n_route, float(route_temp))
    return dq


def route_topk_rows(q: torch.Tensor, lib_: PagedLibrary, plan: RowPlan, top_k: int = 0,
                    route_temp: float = 10.0, emit_f16: bool = False):
    """route_topk for query rows grouped by library as in `plan` (rows of library g contiguous):
    the q . S dots as 32 x 32 fp32 MFMA tiles, then the same top-k / softmax per row (operator
    xenc::route_rows: route_rows_logits_kernel + route_rows_select_kernel; differentiable in q
    through w).  Returns (w, idx, w_sel), plus q as fp16 rows from the same pass (the MFMA read's
    operand) when emit_f16."""
    q = _query(q, lib_.d)
    if q.shape[0] != plan.M:
        raise ValueError(f"q must have {plan.M} rows")
    if lib_.cmax > 1024:
        raise ValueError("the many-row routing takes libraries of at most 1024 chunks")
    out = torch.ops.xenc.route_rows(q, lib_.S, lib_.chunk_ptr, plan.row_ptr, plan.logit_tiles, plan.route_tiles,
                                    plan.n_logit, plan.n_route, int(top_k), float(route_temp), lib_.cmax,
                                    lib_.kept(int(top_k)), bool(emit_f16))
    return out if emit_f16 else out[:3]


def _plan_groups(plan: RowPlan) -> torch.Tensor:
    g = torch.repeat_interleave(torch.arange(len(plan.rows)), torch.tensor(plan.rows))
    return g.to(torch.int32)


class _RouteFewRows(torch.autograd.Function):
    """Differentiable routing of fewer rows than the many-row kernel's tiles pay for: forward by
    xenc::route_topk, backward by xenc::route_backward_."""

    @staticmethod
    def forward(ctx, q, lib_, plan, top_k, route_temp):
        qg = _plan_groups(plan).to(q.device)
        w, idx, wsel = route_topk(q.detach(), lib_, qg, top_k=top_k, route_temp=route_temp)
        ctx.save_for_backward(w)
        ctx.lib, ctx.plan, ctx.route_temp = lib_, plan, route_temp
        ctx.mark_non_differentiable(idx, wsel)
        return w, idx, wsel

    @staticmethod
    def backward(ctx, dw, _didx, _dwsel):
        (w,) = ctx.saved_tensors
        dq = torch.zeros(w.shape[0], ctx.lib.d, dtype=torch.float32, device=w.device)
        if dw is not None:
            route_backward(w, dw, ctx.lib, ctx.plan, ctx.route_temp, dq)
        return dq, None, None, None, None


def route_differentiable(q: torch.Tensor, lib_: PagedLibrary, plan: RowPlan, top_k: int, route_temp: float,
                         emit_f16: bool = False):
    """(w, idx, w_sel[, qh]) with autograd through w: the many-row routing operator for at least
    ROUTE_ROWS_MIN rows, the few-row one below."""
    if plan.M >= ROUTE_ROWS_MIN and lib_.cmax <= 1024:
        return route_topk_rows(q, lib_, plan, top_k, route_temp, emit_f16=emit_f16)
    out = _RouteFewRows.apply(_query(q, lib_.d), lib_, plan, int(top_k), float(route_temp))
    return (*out, None) if emit_f16 else out


def library_read(q: torch.Tensor, lib_: PagedLibrary, plan: RowPlan, top_k: int = 0,
                 read_temp: float = 12.0, route_temp: float = 10.0, read_softmax: bool = True):
    """(r [M, d], w [M, cmax]) with autograd through both routing and the read (MFMA path).  The
    routing pass also writes the fp16 rows the read takes, so q is read from HBM once."""
    if not prefill_ok(lib_) and not _mfma_pages_ok(lib_):
        lib_.check_prefill()
    if prefill_ok(lib_) and plan.M >= ROUTE_ROWS_MIN and lib_.cmax <= 1024:
        # routing and read as one autograd node (xenc::library_read_routed): its backward writes dq
        # once, with the routing term folded into the readout
        q = _query(q, lib_.d)
        if q.shape[0] != plan.M:
            raise ValueError(f"q must have {plan.M} rows")
        fk, fv, fvs, fkr, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles, readout_tiles, n_score, \
            n_readout, slots = _prefill_operands(lib_, plan)
        r, w, _, _, _ = torch.ops.xenc.library_read_routed(
            q, lib_.S, chunk_ptr, row_ptr, plan.logit_tiles, plan.route_tiles, plan.n_logit, plan.n_route,
            int(top_k), float(route_temp), lib_.cmax, lib_.kept(int(top_k)), fk, fv, fvs, fkr, chunk_page,
            chunk_nvalid, score_tiles, readout_tiles, n_score, n_readout, slots, float(read_temp),
            bool(read_softmax), min(lib_.n_chunks) != lib_.cmax)
        return r, w
    w, _, _, qh = route_differentiable(q, lib_, plan, int(top_k), float(route_temp), emit_f16=True)
    if prefill_ok(lib_):
        r, _ = prefill_forward(q, w, lib_, plan, float(read_temp), bool(read_softmax), qh=qh)
    else:   # pages longer than 512 slots
        r = read_sub_pages(q, w, lib_, plan, float(read_temp), bool(read_softmax), qh=qh)
    return r, w


# ----------------------------------------------------------------------------- pages > 512 slots
SUB_SPAN = 512   # slots per sub-page: the MFMA scores tile covers one page of at most this many


@dataclass
class SubPages:
    """A pool whose pages are longer than SUB_SPAN slots, re-paged for the MFMA kernels: chunk c
    becomes ceil(n_c / SUB_SPAN) sub-chunks (sub-chunk j holds its slots SUB_SPAN j .. SUB_SPAN
    (j + 1) - 1), the sub-chunks of a library in chunk order.

    lib     the re-paged pool (untied values re-paged alike)
    tied    the same pool with the keys as values (the gradient of a sub-chunk's log-sum-exp)
    parent  int64 [G, cmax_sub]: the local chunk of each local sub-chunk (0 past a library's end)
    valid   bool [G, cmax_sub]: the sub-chunk exists
    ratio   fp32 [G, cmax_sub]: sqrt(n_sub / n_chunk), the linear read's 1 / sqrt(n) per chunk"""

    lib: PagedLibrary
    tied: PagedLibrary
    parent: torch.Tensor
    valid: torch.Tensor
    ratio: torch.Tensor


def _build_sub_pages(lib_: PagedLibrary) -> SubPages:
    span, N, d, dev = SUB_SPAN, lib_.slots_per_page, lib_.d, lib_.device
    blocks = -(-N // span)
    cpage = lib_.chunk_page.cpu().tolist()
    src_page, src_block, nv_sub, n_sub, parent_local = [], [], [], [], []
    for n in lib_.nvalid:
        n_sub.append(-(-n // span))
    c0 = 0
    for nch in lib_.n_chunks:
        for c in range(nch):
            gc = c0 + c
            for j in range(n_sub[gc]):
                src_page.append(cpage[gc])
                src_block.append(j)
                nv_sub.append(min(span, lib_.nvalid[gc] - j * span))
                parent_local.append(c)
        c0 += nch
    sp_t, sb_t = (torch.tensor(x, dtype=torch.int64, device=dev) for x in (src_page, src_block))

    def repage(src):
        padded = torch.nn.functional.pad(src, (0, 0, 0, blocks * span - N)) if blocks * span != N else src
        return padded.view(src.shape[0], blocks, span, d)[sp_t, sb_t].contiguous()

    pages = repage(lib_.pages)
    values = repage(lib_.values) if lib_.values is not None else None
    subs_per_lib, c0 = [], 0
    for nch in lib_.n_chunks:
        subs_per_lib.append(sum(n_sub[c0:c0 + nch]))
        c0 += nch
    ptr_ = [0]
    for k in subs_per_lib:
        ptr_.append(ptr_[-1] + k)
    parent_global = torch.tensor([g for g, k in enumerate(n_sub) for _ in range(k)], dtype=torch.int64, device=dev)
    P = len(src_page)
    sub = PagedLibrary(pages, torch.arange(P, dtype=torch.int32, device=dev), _i32(nv_sub, dev), _i32(ptr_, dev),
                       lib_.S[parent_global].contiguous(), n_chunks=subs_per_lib, nvalid=nv_sub, values=values,
                       d_valid=lib_.d_valid)
    tied = PagedLibrary(pages, sub.chunk_page, sub.chunk_nvalid, sub.chunk_ptr, sub.S, n_chunks=subs_per_lib,
                        nvalid=nv_sub, d_valid=lib_.d_valid)
    tied._frag, tied._plans = sub._frag, sub._plans   # the key-side fragment copies are the same
    G, cmax_sub = lib_.n_libraries, max(subs_per_lib)
    parent = torch.zeros(G, cmax_sub, dtype=torch.int64)
    valid = torch.zeros(G, cmax_sub, dtype=torch.bool)
    ratio = torch.zeros(G, cmax_sub, dtype=torch.float32)
    i = 0
    c0 = 0
    for g, (nch, k) in enumerate(zip(lib_.n_chunks, subs_per_lib)):
        for j in range(k):
            pc = parent_local[i]
            parent[g, j], valid[g, j] = pc, True
            ratio[g, j] = math.sqrt(nv_sub[i] / lib_.nvalid[c0 + pc])
            i += 1
        c0 += nch
    return SubPages(sub, tied, parent.to(dev), valid.to(dev), ratio.to(dev))


class _SubPageLse(torch.autograd.Function):
    """a [M, cmax_sub] = logsumexp_n(read_temp * q . K[j, n]) per (row, sub-chunk) (operator
    xenc::library_prefill_lse); backward: dq = read_temp * sum_j g_j sum_n p[j, n] K[j, n], the
    read of the tied sub-pages with weights g (xenc::library_prefill_fwd)."""

    @staticmethod
    def forward(ctx, q, qh, sp: SubPages, splan: RowPlan, read_temp: float):
        L = sp.lib
        lse = torch.ops.xenc.library_prefill_lse(q, qh, L.fragment_pages(0), L.chunk_ptr, L.chunk_page,
                                                 L.chunk_nvalid, splan.row_ptr, splan.score_tiles, splan.n_score,
                                                 L.slots_per_page, float(read_temp), L.cmax)
        ctx.save_for_backward(q)
        ctx.sp, ctx.splan, ctx.read_temp = sp, splan, float(read_temp)
        return lse

    @staticmethod
    def backward(ctx, g):
        (q,) = ctx.saved_tensors
        g = torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=0.0).contiguous()
        with torch.no_grad():
            o, _ = prefill_forward(q, g, ctx.sp.tied, ctx.splan, ctx.read_temp, True)
        return o * ctx.read_temp, None, None, None, None


def read_sub_pages(q: torch.Tensor, w: torch.Tensor, lib_: PagedLibrary, plan: RowPlan, read_temp: float = 12.0,
                   softmax: bool = True, qh: torch.Tensor | None = None) -> torch.Tensor:
    """r [M, d]: the read of a pool with pages longer than SUB_SPAN slots on the MFMA kernels,
    differentiable in q and w like prefill_forward.  A chunk's masked softmax over its n slots
    splits over its sub-chunks j: r = sum_c w_c sum_j pi_j o_j, o_j the softmax read of sub-chunk
    j and pi = softmax over the chunk's sub-chunks of their log-sum-exps a_j (linear read: pi_j =
    sqrt(n_j / n) undoes the sub-chunk's own 1 / sqrt(n_j)).  The sub-chunk weights W = w pi feed
    the ordinary read of the re-paged pool (xenc/injector.py:239-265 for any page length)."""
    sp = lib_.sub_pages()
    splan = sp.lib.plan(plan.rows)
    rg = torch.repeat_interleave(torch.arange(len(plan.rows), device=q.device),
                                 torch.as_tensor(plan.rows, device=q.device))
    par, val = sp.parent[rg], sp.valid[rg]
    W = w.to(torch.float32).gather(1, par) * val
    if softmax:
        a = _SubPageLse.apply(q, qh, sp, splan, read_temp).masked_fill(~val, float("-inf"))
        amax = torch.full(w.shape, float("-inf"), device=q.device).scatter_reduce(1, par, a.detach(), "amax")
        e = torch.exp(a - amax.gather(1, par)).masked_fill(~val, 0.0)
        den = torch.zeros(w.shape, device=q.device).scatter_add(1, par, e)
        W = W * e / den.gather(1, par).clamp_min(torch.finfo(torch.float32).tiny)
    else:
        W = W * sp.ratio[rg]
    r, _ = prefill_forward(q, W.contiguous(), sp.lib, splan, float(read_temp), bool(softmax), qh=qh)
    return r


def _mfma_pages_ok(lib_: PagedLibrary) -> bool:
    """The MFMA kernels can read this pool, directly or as sub-pages."""
    return lib_.d % 64 == 0 and lib_.slots_per_page % 64 == 0


# Above this many query rows on one library the MFMA prefill path reads it (each page once per
# 128-row tile); at or below it the split-K decode path does (each page once per row).
DECODE_MAX_ROWS = 8


def prefill_ok(lib_: PagedLibrary) -> bool:
    return lib_.d % 64 == 0 and lib_.slots_per_page % 64 == 0 and lib_.slots_per_page <= 512


def _pad_rows(q: torch.Tensor, lib_: PagedLibrary) -> torch.Tensor:
    _require_device(q, "q")
    if q.dim() != 2 or q.shape[1] != lib_.d_valid:
        raise ValueError(f"q must be [M, {lib_.d_valid}], got {tuple(q.shape)}")
    q = q.to(torch.float32)
    return torch.nn.functional.pad(q, (0, lib_.d - lib_.d_valid)) if lib_.d != lib_.d_valid else q


def _single(lib_: PagedLibrary) -> None:
    if lib_.n_libraries != 1:
        raise ValueError("this entry point reads one library; use route_topk / library_read_decode for pools")


def route_rows(q: torch.Tensor, lib_: PagedLibrary, top_k: int = 0, route_temp: float = 10.0):
    """(w [M, C], idx [M, kk], w_sel [M, kk]) for M query rows over ONE library
    (LibraryInjector.route, xenc/injector.py:220-229).  Differentiable in q (through w) when q
    requires grad; q has d_valid features (zero-padded here to the pool's width)."""
    _single(lib_)
    qp = _pad_rows(q, lib_)
    if torch.is_grad_enabled() and q.requires_grad:
        return route_differentiable(qp, lib_, lib_.plan([qp.shape[0]]), int(top_k), float(route_temp))
    return route_topk(qp, lib_, None, top_k, route_temp)


def read_rows(q: torch.Tensor, w: torch.Tensor, idx: torch.Tensor, w_sel: torch.Tensor,
              lib_: PagedLibrary, read_temp: float = 12.0, read_softmax: bool = True) -> torch.Tensor:
    """r [M, d_valid]: the read of M query rows over ONE library given their routing (the read of
    LibraryInjector._branch, xenc/injector.py:239-265).

    With autograd (q or w requires grad), untied values, or more than DECODE_MAX_ROWS rows it runs
    the MFMA prefill path (differentiable in q and w; pages longer than 512 slots as sub-pages,
    read_sub_pages); otherwise, and for forward reads of tied pages longer than 512 slots, the
    split-K decode path."""
    _single(lib_)
    qp = _pad_rows(q, lib_)
    M = qp.shape[0]
    grad = torch.is_grad_enabled() and (q.requires_grad or w.requires_grad)
    mfma = grad or lib_.values is not None or M > DECODE_MAX_ROWS
    if mfma and not prefill_ok(lib_) and not (grad or lib_.values is not None):
        mfma = False        # a forward read of larger pages: the split-K decode path takes any size
    if mfma and prefill_ok(lib_):
        r, _ = prefill_forward(qp, w, lib_, lib_.plan([M]), float(read_temp), bool(read_softmax))
    elif mfma:
        if not _mfma_pages_ok(lib_):
            lib_.check_prefill()
        r = read_sub_pages(qp, w, lib_, lib_.plan([M]), float(read_temp), bool(read_softmax))
    else:
        r = library_read_decode(qp, lib_, idx, w_sel, None, read_temp, read_softmax)
    return r[:, :lib_.d_valid] if lib_.d != lib_.d_valid else r


def branch_read(q: torch.Tensor, lib_: PagedLibrary, top_k: int = 0, read_temp: float = 12.0,
                route_temp: float = 10.0, read_softmax: bool = True):
    """(r [M, d_valid], w [M, C]): route_rows + read_rows.  Under autograd with at least
    ROUTE_ROWS_MIN rows (and a pool the MFMA read takes), library_read instead: routing and read as
    one operator."""
    _single(lib_)
    M = q.shape[0]
    if (torch.is_grad_enabled() and q.requires_grad and prefill_ok(lib_) and M >= ROUTE_ROWS_MIN
            and lib_.cmax <= 1024):
        r, w = library_read(_pad_rows(q, lib_), lib_, lib_.plan([M]), int(top_k), float(read_temp),
                            float(route_temp), bool(read_softmax))
        return (r[:, :lib_.d_valid] if lib_.d != lib_.d_valid else r), w
    w, idx, wsel = route_rows(q, lib_, top_k, route_temp)
    return read_rows(q, w, idx, wsel, lib_, read_temp, read_softmax), w


# ----------------------------------------------------------------------------- D18 multi-document read
_D18_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


@dataclass
class D18Operators:
    """One layer's document operators packed for xenc_d18_read: K, V [Hkv, Ntot, hd] (documents
    back to back, one dtype), doc_ptr int32 [D + 1] on the device, lengths N_d."""
    K: torch.Tensor
    V: torch.Tensor
    doc_ptr: torch.Tensor
    lengths: list

    @property
    def n_docs(self) -> int:
        return len(self.lengths)


def d18_pack(ops) -> D18Operators:
    """Pack [(K_d, V_d) [Hkv, N_d, hd], ...] (the operator list of lib_read) once per load."""
    if isinstance(ops, D18Operators):
        return ops
    if not ops:
        raise ValueError("d18: need at least one document operator")
    K0 = ops[0][0]
    for K, V in ops:
        if K.shape != V.shape or K.dim() != 3 or K.shape[0] != K0.shape[0] or K.shape[2] != K0.shape[2]:
            raise ValueError("d18: every operator is (K, V) [Hkv, N_d, hd] with one Hkv and hd")
        if K.dtype != K0.dtype or V.dtype != K0.dtype or K0.dtype not in _D18_DTYPES:
            raise ValueError("d18: operators are fp16, bf16 or fp32, all one dtype")
        _require_device(K, "K_d")
        _require_device(V, "V_d")
    lengths = [int(K.shape[1]) for K, _ in ops]
    ptr_ = [0]
    for n in lengths:
        ptr_.append(ptr_[-1] + n)
    return D18Operators(torch.cat([K for K, _ in ops], 1).contiguous(), torch.cat([V for _, V in ops], 1).contiguous(),
                        torch.tensor(ptr_, dtype=torch.int32, device=K0.device), lengths)


def d18_nsplit(T: int, hkv: int, lengths, own: int) -> int:
    """Key splits per unit: about one partials workgroup per CU (256) with at least 128 keys per
    split (a decode step of 6 documents x 2048 rows, 2 kv heads: 16 splits, the fastest of 4-32
    measured)."""
    units = T * hkv * (len(lengths) + 1)
    want = -(-256 // max(units, 1))
    return max(1, min(32, want, max(max(lengths), own) // 128))


def d18_read(qd: torch.Tensor, qo: torch.Tensor, ops, Kown: torch.Tensor, Vown: torch.Tensor, scale: float,
             skip: int = 0, beta: float = 1.0, top_k: int = 0, force: int | None = None,
             wfix: torch.Tensor | None = None, nsplit: int | None = None) -> dict:
    """The attention core of lib_read (xenc/d18_library.py:63-90) on HIP (csrc/d18.hip →
    xenc_d18_read): qd [D, Hq, T, hd] the query rotated for each document (at N_d + P + t), qo
    [Hq, T, hd] rotated at P + t, ops the operators (a list of (K_d, V_d) [Hkv, N_d, hd] or
    d18_pack's result), Kown / Vown [Hkv, P + T, hd] the own rows (row t sees P + t + 1 of them).
    -> {"o" [T, Hq*hd] (before the gate and o_proj), "w", "r", "rmax" [Hkv, G, T, D], "n" [D]}.
    Forward only: the reference evaluates D18 under no_grad."""
    P_ops = d18_pack(ops)
    D, Hq, T, hd = qd.shape
    Hkv = P_ops.K.shape[0]
    if D != P_ops.n_docs or qo.shape != (Hq, T, hd) or P_ops.K.shape[2] != hd or Hq % Hkv:
        raise ValueError("d18: qd [D, Hq, T, hd], qo [Hq, T, hd] and the operators must agree")
    if Kown.shape != Vown.shape or Kown.dim() != 3 or Kown.shape[0] != Hkv or Kown.shape[2] != hd \
            or Kown.shape[1] < T:
        raise ValueError("d18: Kown / Vown are [Hkv, P + T, hd]")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (qd, qo, Kown, Vown)):
        raise RuntimeError("d18_read has no backward: call it under torch.no_grad()")
    for name, t in (("qd", qd), ("qo", qo), ("Kown", Kown), ("Vown", Vown)):
        _require_device(t, name)
    dev = qd.device
    P = Kown.shape[1] - T
    G = Hq // Hkv
    qd_ = qd.detach().float().transpose(1, 2).contiguous()          # [D, T, Hq, hd]
    qo_ = qo.detach().float().transpose(0, 1).contiguous()          # [T, Hq, hd]
    ko, vo = Kown.detach().float().contiguous(), Vown.detach().float().contiguous()
    out = torch.empty(T, Hq, hd, dtype=torch.float32, device=dev)
    w = torch.empty(Hkv, G, T, D, dtype=torch.float32, device=dev)
    r = torch.empty_like(w)
    rmax = torch.empty_like(w)
    wf = None
    if force is None and wfix is not None:
        wf = wfix.detach().to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if wf.numel() != D:
            raise ValueError("d18: wfix has one weight per document")
    S = d18_nsplit(T, Hkv, P_ops.lengths, P + T) if nsplit is None else int(nsplit)
    nbytes = lib().xenc_d18_workspace_bytes(T, Hq, D, hd, S)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
    check(lib().xenc_d18_read(_D18_DTYPES[P_ops.K.dtype], T, Hq, Hkv, hd, D, ptr(qd_), ptr(qo_),
                              ptr(P_ops.K), ptr(P_ops.V), P_ops.K.stride(0), P_ops.K.stride(1), ptr(P_ops.doc_ptr),
                              ptr(ko), ptr(vo), ko.stride(0), ko.stride(1), P, float(scale), int(skip), float(beta),
                              int(top_k), -1 if force is None else int(force), ptr(wf), S, ptr(out), ptr(w), ptr(r),
                              ptr(rmax), ptr(ws), ws.numel(), stream_handle(dev)), "xenc_d18_read")
    n = torch.tensor([float(m - skip) if m > skip else float(m) for m in P_ops.lengths], device=dev)
    return {"o": out.reshape(T, Hq * hd), "w": w, "r": r, "rmax": rmax, "n": n}


__all__ = ["PagedLibrary", "route_topk", "library_read_decode", "route_read_decode", "default_nsplit", "RowPlan", "row_plan",
           "cast_f16", "prefill_forward", "prefill_backward", "route_backward", "route_topk_rows", "route_differentiable",
           "library_read", "route_rows", "read_rows", "branch_read", "unpack_p", "DECODE_MAX_ROWS",
           "build_pages", "write_back", "multi_depth_prepare", "read_sub_pages", "SubPages", "SUB_SPAN", "select_scores", "topk_rows", "gather_library", "selector_weights",
           "selector_apply", "gate_scale", "D18Operators", "d18_pack", "d18_read", "d18_nsplit"]
