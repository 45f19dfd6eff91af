"""GPU: the static LibraryPool (the Library-read counterpart of the plugin's static operator pool,
xenc/d23_vllm_plugin.py:84-119).  Documents built into the pool read exactly like the same
documents built into a fresh pool (bit for bit: same kernels, only the page numbers differ);
an evicted range is reused; a read captured in a HIP graph over one active set replays on a
later active set of the same shape; and the guards."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops
from kv_skill_v2_amd.depth import unit_rows
from kv_skill_v2_amd.pool import LibraryPool

pytestmark = pytest.mark.gpu

RHO = 0.5
D = 256


def say(*a):
    print("[case]", *a, flush=True)


def _cache(n_slots, seed, d=D):
    g = torch.Generator().manual_seed(seed)
    return {"chunks": [{"K": {RHO: unit_rows(n, d, g).half()}, "start": 0, "n_tokens": n} for n in n_slots],
            "depths": [RHO], "doc_id": str(seed), "encoder": "synthetic"}


DOCS = {"a": _cache([512, 40, 512, 7, 300, 512], 1), "b": _cache([64, 128, 3, 512, 500, 90], 2),
        "c": _cache([33, 512, 256, 1], 3), "d": _cache([100, 200, 300, 400, 500, 512], 4)}


def _read(lib, q, qg, top_k=3):
    _, idx, wsel = ops.route_topk(q, lib, qg, top_k=top_k)
    return ops.library_read_decode(q, lib, idx, wsel, qg)


def test_pool_reads_like_fresh_build_and_reuses_ranges(dev):
    say("pool load / activate / evict")
    center = {RHO: 0.2 * torch.randn(D, generator=torch.Generator().manual_seed(9))}
    pool = LibraryPool(capacity_chunks=16, slots_per_page=512, d=D, device=dev)
    for name in ("a", "b", "c"):
        pool.load(name, DOCS[name], RHO, center=center)
    assert [pool.docs[n]["start"] for n in "abc"] == [0, 6, 12]
    q = unit_rows(6, D, torch.Generator().manual_seed(5)).to(dev)
    qg = torch.tensor([0, 1, 0, 1, 1, 0], dtype=torch.int32, device=dev)
    lib = pool.activate(["a", "c"])
    fresh = ops.PagedLibrary.from_doc_caches([DOCS["a"], DOCS["c"]], RHO, dev, center=center)
    assert torch.equal(lib.S, fresh.S)
    assert torch.equal(_read(lib, q, qg), _read(fresh, q, qg))
    # the read also matches the oracle Library of the same centred rows
    r = _read(lib, q, qg).cpu().double()
    for m, g in enumerate(qg.tolist()):
        rows = [c["K"][RHO] for c in DOCS["ac"[g]]["chunks"]]
        K, M, S = O.library_tensors(rows, dtype=torch.float64, center_mu=center[RHO].double())
        qm = q[m].cpu().view(1, 1, -1).double()
        if float(O.boundary_gap(qm, S, 3).min()) > 2e-5:
            ref, _ = O.branch_read(qm, K, M, S, top_k=3)
            assert float((r[m] - ref.view(-1)).abs().max()) < 2e-3
    with pytest.raises(RuntimeError):
        pool.evict("a")                        # active
    pool.activate(["c"])
    pool.evict("b")
    pool.load("d", DOCS["d"], RHO, center=center)
    assert pool.docs["d"]["start"] == 6        # b's freed range
    lib2 = pool.activate(["d", "a"])
    fresh2 = ops.PagedLibrary.from_doc_caches([DOCS["d"], DOCS["a"]], RHO, dev, center=center)
    assert torch.equal(_read(lib2, q, qg), _read(fresh2, q, qg))
    free_before = list(pool.free)
    with pytest.raises(torch.cuda.OutOfMemoryError):   # the reference's full-pool error
        pool.load("e", _cache([5] * 5, 7), RHO)  # 5 chunks; all 16 pages are taken (a, d, c)
    assert "e" not in pool.docs and pool.free == free_before


def test_graph_replays_on_a_new_active_set(dev):
    """Capture route + read over active set (a, c); activate (d, c) (same shape: 6 + 4 chunks);
    every replay equals the eager read of the set active at that time."""
    say("pool graph replay")
    pool = LibraryPool(capacity_chunks=20, slots_per_page=512, d=D, device=dev)
    for name in "acd":
        pool.load(name, DOCS[name], RHO)
    q = unit_rows(4, D, torch.Generator().manual_seed(11)).to(dev)
    qg = torch.tensor([0, 1, 1, 0], dtype=torch.int32, device=dev)
    lib = pool.activate(["a", "c"])

    def step():
        return _read(lib, q, qg, top_k=2)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        out = step()
    for rep, docs in enumerate((["a", "c"], ["d", "c"], ["a", "c"], ["d", "c"])):
        pool.activate(docs)
        gph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        _ = torch.randn(512, device=dev).sum()
        ref = _read(ops.PagedLibrary.from_doc_caches([DOCS[x] for x in docs], RHO, dev), q, qg, top_k=2)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (rep, docs)


def test_pool_guards(dev):
    say("pool guards")
    pool = LibraryPool(capacity_chunks=8, slots_per_page=128, d=64, device=dev)
    with pytest.raises(ValueError):
        pool.load("x", _cache([200], 1, d=64), RHO)             # more slots than a page
    with pytest.raises(ValueError):
        pool.load("x", _cache([10], 1, d=32), RHO)              # wrong d
    pool.load("x", _cache([10, 20], 1, d=64), RHO)
    with pytest.raises(KeyError):
        pool.load("x", _cache([10], 2, d=64), RHO)
    with pytest.raises(KeyError):
        pool.activate(["nope"])
    with pytest.raises(ValueError):
        pool.activate([])
    assert pool.free == [(2, 6)]
    pool.evict("x")
    assert pool.free == [(0, 8)]
