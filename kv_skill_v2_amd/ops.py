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
from ._lib import check, lib, ptr, stream_handle


def _require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} is on {t.device}: the Library read runs only on a ROCm GPU "
                           "(there is no CPU path)")


def _i32(x, device) -> torch.Tensor:
    return torch.as_tensor(x, dtype=torch.int32, device=device).contiguous()


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

    # ------------------------------------------------------------------ constructors
    @staticmethod
    def from_padded(K: torch.Tensor, mask: torch.Tensor, S: torch.Tensor, device=None) -> "PagedLibrary":
        """One library from the reference layout K [C, N, d], mask [C, N] (valid prefix), S [C, d]."""
        return PagedLibrary.from_libraries([(K, mask, S)], device=device)

    @staticmethod
    def from_libraries(libs, device=None, slots_per_page: int | None = None) -> "PagedLibrary":
        """Several libraries [(K [C,N,d], mask [C,N], S [C,d]), ...] packed into one pool, page id =
        global chunk id.  Masks must be valid prefixes (slots 0..n-1 valid), as Library builds them."""
        device = torch.device(device) if device is not None else libs[0][0].device
        d = libs[0][0].shape[-1]
        N = slots_per_page or max(int(K.shape[1]) for K, _, _ in libs)
        pages, Ss, nv, nch = [], [], [], []
        for K, M, S in libs:
            C, n_max, dk = K.shape
            if dk != d:
                raise ValueError("all libraries must share d")
            cnt = M.sum(-1).to(torch.int64)
            pref = torch.arange(n_max, device=M.device).view(1, -1) < cnt.view(-1, 1)
            if not torch.equal(pref, M.bool()):
                raise ValueError("mask must mark a prefix of valid slots per chunk")
            pg = torch.zeros(C, N, d, dtype=torch.float16, device=device)
            pg[:, :n_max] = K.to(device=device, dtype=torch.float16)
            pages.append(pg)
            Ss.append(S.to(device=device, dtype=torch.float32))
            nv += cnt.tolist()
            nch.append(C)
        ptr_ = [0]
        for c in nch:
            ptr_.append(ptr_[-1] + c)
        Ctot = ptr_[-1]
        return PagedLibrary(torch.cat(pages).contiguous(), _i32(list(range(Ctot)), device),
                            _i32(nv, device), _i32(ptr_, device), torch.cat(Ss).contiguous(),
                            n_chunks=nch, nvalid=nv)

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
        """Width of the routed-index arrays: max over libraries of the kept chunk count."""
        return max(c if (top_k <= 0 or top_k >= c) else top_k for c in self.n_chunks)


def _groups(lib_: PagedLibrary, M: int, q_group) -> torch.Tensor:
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
    q = q.to(torch.float32)
    if q.stride(1) != 1 or q.stride(0) % 4 or q.data_ptr() % 16:
        q = q.contiguous()
    return q


def route_topk(q: torch.Tensor, lib_: PagedLibrary, q_group=None, top_k: int = 0,
               route_temp: float = 10.0):
    """(w_dense [M, cmax], idx [M, kk] int32, w_sel [M, kk]) for query rows q [M, d].

    HIP kernel `route_topk_kernel` (kv_skill_v2_amd/csrc/route.hip); replaces
    LibraryInjector.route (xenc/injector.py:220-229)."""
    q = _query(q, lib_.d)
    M = q.shape[0]
    g = _groups(lib_, M, q_group)
    kk = lib_.kept(int(top_k))
    dev = q.device
    w = torch.empty(M, lib_.cmax, dtype=torch.float32, device=dev)
    idx = torch.empty(M, kk, dtype=torch.int32, device=dev)
    wsel = torch.empty(M, kk, dtype=torch.float32, device=dev)
    if M == 0:
        return w, idx, wsel
    rc = lib().xenc_route_topk(ptr(q), q.stride(0), M, lib_.d, ptr(lib_.S), ptr(lib_.chunk_ptr),
                               ptr(g), lib_.n_libraries, int(top_k), float(route_temp), ptr(w),
                               w.stride(0), ptr(idx), ptr(wsel), kk, stream_handle(dev))
    check(rc, "xenc_route_topk")
    return w, idx, wsel


def default_nsplit(units: int, slots_per_page: int) -> int:
    """Slot splits per routed page.  With >= 512 (query, page) units one workgroup per page
    fills the 256 CUs (measured best on the B = 64 batched decode); fewer units are split down
    to 16-slot pieces so a single query still spreads over many CUs."""
    want = max(1, math.ceil(512 / max(units, 1)))
    return int(max(1, min(want, max(1, slots_per_page // 16), 64)))


class _Workspaces:
    """Decode workspaces, one per (device, stream), grown on demand.  Its arrival counters are
    zeroed once by a kernel (xenc_decode_workspace_init) and every call leaves them zero."""

    def __init__(self):
        self._ws = {}

    def get(self, device: torch.device, stream: int, nbytes: int, M: int) -> torch.Tensor:
        key = (device.index, stream)
        buf, zeroed = self._ws.get(key, (None, 0))
        if buf is None or buf.numel() < nbytes or zeroed < M:
            size = max(nbytes, buf.numel() if buf is not None else 0)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            zeroed = max(M, zeroed)
            check(lib().xenc_decode_workspace_init(ptr(buf), size, zeroed, stream),
                  "xenc_decode_workspace_init")
            self._ws[key] = (buf, zeroed)
        return buf


_WORKSPACES = _Workspaces()


def library_read_decode(q: torch.Tensor, lib_: PagedLibrary, idx: torch.Tensor, w_sel: torch.Tensor,
                        q_group=None, read_temp: float = 12.0, softmax: bool = True,
                        nsplit: int | None = None) -> torch.Tensor:
    """r [M, d] fp32: route-weighted masked-softmax (or linear) read over the routed pages.

    HIP kernels `decode_split_kernel` + `decode_merge_kernel` (kv_skill_v2_amd/csrc/decode.hip);
    replaces the read of LibraryInjector._branch (xenc/injector.py:239-265)."""
    q = _query(q, lib_.d)
    M = q.shape[0]
    g = _groups(lib_, M, q_group)
    _require_device(idx, "idx")
    if idx.dim() != 2 or idx.shape[0] != M or w_sel.shape != idx.shape:
        raise ValueError("idx and w_sel must both be [M, kk]")
    idx = idx.to(torch.int32).contiguous()
    w_sel = w_sel.to(torch.float32).contiguous()
    kk = idx.shape[1]
    r = torch.empty(M, lib_.d, dtype=torch.float32, device=q.device)
    if M == 0 or kk == 0:
        return r.zero_()
    ns = int(nsplit) if nsplit is not None else default_nsplit(M * kk, lib_.slots_per_page)
    L = lib()
    wsb = L.xenc_decode_workspace_bytes(M, kk, ns, lib_.d)
    st = stream_handle(q.device)
    ws = _WORKSPACES.get(q.device, st, wsb, M)
    rc = L.xenc_library_read_decode(
        ptr(q), q.stride(0), M, lib_.d, ptr(lib_.pages), lib_.slots_per_page,
        lib_.pages.stride(0), ptr(lib_.chunk_page), ptr(lib_.chunk_nvalid), ptr(lib_.chunk_ptr),
        ptr(g), lib_.n_libraries, ptr(idx), ptr(w_sel), kk, float(read_temp), int(bool(softmax)),
        ns, ptr(r), r.stride(0), ptr(ws), ws.numel(), st)
    check(rc, "xenc_library_read_decode")
    return r


__all__ = ["PagedLibrary", "route_topk", "library_read_decode", "default_nsplit"]
