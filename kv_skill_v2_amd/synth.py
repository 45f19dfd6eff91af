"""Seeded synthetic Libraries and queries for the Library-read workloads.

Conventions (fixed for every workload): slots are N(0,1) rows, L2-normalised, then stored as
fp16 (the operator cache stores fp16 rows, xenc/depth_skill.py:258-261, 299-307), so the fp32
math of the reference sees exactly the values the kernels read.  Every library's last chunk is
cut to a seeded tail length in [tail_lo, N]; padded slots are zero.  S = L2(masked mean) in fp32.
Queries are N(0, 1/d) rows normalised as itf_query does (q / (|q| + 1e-6)).
Seeds: 0 slots, 1 tails, 2 queries, 3 chunks per library, 4 page shuffle, 5 selector logits,
6 interface matrices, 7 upstream gradient.

Large pools are generated on the device with a device generator (values then differ from a CPU
generator with the same seed, but are reproducible on the device).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

EPS = 1e-6


def _gen(seed: int, device) -> torch.Generator:
    dev = torch.device(device)
    g = torch.Generator(device=dev if dev.type == "cuda" else "cpu")
    g.manual_seed(seed)
    return g


def unit_rows_fp16(n: int, d: int, g: torch.Generator, device) -> torch.Tensor:
    x = torch.randn(n, d, generator=g, device=device)
    return (x / (x.norm(dim=-1, keepdim=True) + EPS)).to(torch.float16)


def queries(M: int, d: int, device="cpu", seed: int = 2) -> torch.Tensor:
    g = _gen(seed, device)
    q = torch.randn(M, d, generator=g, device=device) / d ** 0.5
    return q / (q.norm(dim=-1, keepdim=True) + EPS)


def masked_summaries(pages: torch.Tensor, nvalid: torch.Tensor) -> torch.Tensor:
    """S [C, d] fp32 = L2(mean of the first nvalid rows) of fp16 pages [C, N, d]."""
    C, N, d = pages.shape
    mask = torch.arange(N, device=pages.device).view(1, N) < nvalid.view(C, 1).to(pages.device)
    m = (pages.float() * mask.unsqueeze(-1)).sum(1) / nvalid.to(pages.device).clamp_min(1).view(C, 1).float()
    return m / (m.norm(dim=-1, keepdim=True) + EPS)


@dataclass
class SynthPool:
    pages: torch.Tensor          # fp16 [P, N, d]
    chunk_page: torch.Tensor     # int32 [Ctot]
    chunk_nvalid: torch.Tensor   # int32 [Ctot]
    chunk_ptr: torch.Tensor      # int32 [G+1]
    S: torch.Tensor              # fp32 [Ctot, d]
    n_chunks: list
    nvalid: list

    def library(self, g: int):
        """(K [C,N,d] fp32, mask [C,N], S [C,d]) of library g on the pool's device (page-table order)."""
        a, b = int(self.chunk_ptr[g]), int(self.chunk_ptr[g + 1])
        pg = self.chunk_page[a:b].long()
        K = self.pages[pg].float()
        nv = self.chunk_nvalid[a:b].long()
        N = K.shape[1]
        M = torch.arange(N, device=K.device).view(1, N) < nv.view(-1, 1)
        return K, M, self.S[a:b]


def pool(n_chunks: list[int], N: int, d: int, device="cpu", tail_lo: int = 64, shuffle: bool = True,
         block: int = 64) -> SynthPool:
    """Libraries with the given chunk counts packed into one page pool (page table = seeded shuffle)."""
    dev = torch.device(device)
    G = len(n_chunks)
    Ctot = sum(n_chunks)
    gt = _gen(1, "cpu")
    tails = torch.randint(min(tail_lo, N), N + 1, (G,), generator=gt)
    nvalid = []
    for c, t in zip(n_chunks, tails.tolist()):
        nvalid += [N] * (c - 1) + [t]
    perm = torch.randperm(Ctot, generator=_gen(4, "cpu")) if shuffle else torch.arange(Ctot)
    chunk_page = perm.to(torch.int32)
    pages = torch.empty(Ctot, N, d, dtype=torch.float16, device=dev)
    gs = _gen(0, dev)
    nv_t = torch.tensor(nvalid, dtype=torch.int32)
    S = torch.empty(Ctot, d, dtype=torch.float32, device=dev)
    for c0 in range(0, Ctot, block):            # chunk order; written at their shuffled pages
        c1 = min(Ctot, c0 + block)
        rows = unit_rows_fp16((c1 - c0) * N, d, gs, dev).view(c1 - c0, N, d)
        nv = nv_t[c0:c1].to(dev)
        keep = torch.arange(N, device=dev).view(1, N) < nv.view(-1, 1)
        rows = rows * keep.unsqueeze(-1).to(rows.dtype)
        pages[chunk_page[c0:c1].long().to(dev)] = rows
        S[c0:c1] = masked_summaries(rows, nv)
    ptr = [0]
    for c in n_chunks:
        ptr.append(ptr[-1] + c)
    return SynthPool(pages, chunk_page.to(dev), nv_t.to(dev), torch.tensor(ptr, dtype=torch.int32, device=dev),
                     S, list(n_chunks), nvalid)


def batched_chunk_counts(B: int, cmin: int, cmax: int, seed: int = 3) -> list[int]:
    return torch.randint(cmin, cmax + 1, (B,), generator=_gen(seed, "cpu")).tolist()


# ---------------------------------------------------------------------------- named workloads
WORKLOADS = {
    # C2: one query token, one document of 16 x 512 slots, d_s = 2048, top-4
    "single_decode": dict(B=1, chunks=(16, 16), N=512, d=2048, top_k=4),
    # C3: 64 sequences, each its own Library of U{8..64} chunks x 512 slots, d_s = 2048, top-8
    "batched_paged_decode": dict(B=64, chunks=(8, 64), N=512, d=2048, top_k=8),
}


# C5: 8 candidate depths, each a Library of 64 x 512 slots (d_s = 2560) shared by the batch of 32
# tokens; a selector keeps the top-2 depths per token (seeded logits), routing keeps top-8 chunks
# per selected depth, and each read is written back through that depth's B [5120, 2560] (fp32).
MULTI_DEPTH = dict(depths=8, chunks=64, N=512, d=2560, B=32, k_sel=2, top_k=8, d_r=5120)


def multi_depth_workload(device="cuda"):
    """(SynthPool of the 8 depth Libraries, selector logits z [B, 8] (seed 5), queries
    q_all [8, B, d] (seed 2), hidden states h [B, d_r] and B_w^T [8, d, d_r] ~ N(0, 1/d) (seed 6))."""
    c = MULTI_DEPTH
    P = pool([c["chunks"]] * c["depths"], c["N"], c["d"], device=device)
    z = torch.randn(c["B"], c["depths"], generator=_gen(5, "cpu")).to(device)
    q_all = queries(c["depths"] * c["B"], c["d"], device=device).view(c["depths"], c["B"], c["d"])
    g6 = _gen(6, device)
    h = torch.randn(c["B"], c["d_r"], generator=g6, device=device)
    BwT = torch.randn(c["depths"], c["d"], c["d_r"], generator=g6, device=device) / c["d"] ** 0.5
    return P, z, q_all, h, BwT


def decode_workload(name: str, device="cuda", **over):
    """(SynthPool, q [B, d], q_group [B], top_k) for a named decode workload."""
    cfg = {**WORKLOADS[name], **over}
    B = cfg["B"]
    lo, hi = cfg["chunks"]
    counts = [lo] * B if lo == hi else batched_chunk_counts(B, lo, hi)
    P = pool(counts, cfg["N"], cfg["d"], device=device)
    q = queries(B, cfg["d"], device=device)
    return P, q, torch.arange(B, dtype=torch.int32, device=device), cfg["top_k"]


__all__ = ["SynthPool", "pool", "queries", "unit_rows_fp16", "masked_summaries", "batched_chunk_counts",
           "decode_workload", "WORKLOADS", "MULTI_DEPTH", "multi_depth_workload"]
