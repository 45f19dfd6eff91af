"""GPU: the Library pool built on the device from document caches (xenc_build_pages) against the
oracle's Library tensors (xenc/library.py:47-74): pages equal the fp16 slot rows (bit-exact
without centring, within one fp16 rounding of the fp64 centred rows with it), S within 1e-5 of
the fp64 summaries, zero padding everywhere else; then the routed read over the built pool
against the oracle's read, determinism, untied values, a cache file round trip, and guards."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops
from kv_skill_v2_amd.depth import load_doc_cache, save_doc_cache, unit_rows

pytestmark = pytest.mark.gpu

RHO = (0.25, 0.75)


def say(*a):
    print("[case]", *a, flush=True)


def _cache(n_slots, d, seed, untied=False, doc="doc"):
    g = torch.Generator().manual_seed(seed)
    chunks = []
    start = 0
    for n in n_slots:
        c = {"K": {r: unit_rows(n, d, g).half() for r in RHO}, "start": start, "n_tokens": n}
        if untied:
            c["V"] = {r: unit_rows(n, d, g).half() for r in RHO}
        chunks.append(c)
        start += n
    return {"chunks": chunks, "d_s": d, "doc_id": doc, "encoder": "synthetic", "chunk_tokens": 512,
            "depths": list(RHO)}


def _center(d, seed):
    g = torch.Generator().manual_seed(seed)
    return {r: 0.3 * torch.randn(d, generator=g) for r in RHO}


def _check_pool(lib, caches, rho, center):
    d = lib.d_valid
    mu = center[rho].double() if center is not None else None
    base = 0
    for gi, cache in enumerate(caches):
        rows = [c["K"][rho] for c in cache["chunks"]]
        K, M, S = O.library_tensors(rows, dtype=torch.float64, center_mu=mu)
        C, n_max, _ = K.shape
        pages = lib.pages[base:base + C].cpu()
        assert lib.n_chunks[gi] == C
        assert lib.chunk_nvalid[base:base + C].cpu().tolist() == M.sum(-1).tolist()
        for c, r in enumerate(rows):
            n = r.shape[0]
            if center is None:
                assert torch.equal(pages[c, :n, :d], r)
            else:
                err = (pages[c, :n, :d].double() - K[c, :n]).abs().max()
                assert float(err) <= 2.0 ** -11 * 1.001, float(err)   # one fp16 rounding of |x| <= 1
            assert float(pages[c, n:].abs().max() if n < pages.shape[1] else 0.0) == 0.0
            assert float(pages[c, :, d:].abs().max() if d < pages.shape[2] else 0.0) == 0.0
        s = lib.S[base:base + C].cpu().double()
        assert float((s[:, :d] - S).abs().max()) < 1e-5
        assert float(s[:, d:].abs().max() if d < s.shape[1] else 0.0) == 0.0
        base += C


@pytest.mark.parametrize("d,centred", [(256, False), (256, True), (200, True), (1024, False), (4096, True)])
def test_build_matches_library_tensors(dev, d, centred):
    say("pool build", dict(d=d, centred=centred))
    caches = [_cache([512, 37, 1, 300, 512, 64], d, 1, doc="a"), _cache([5, 129, 511], d, 2, doc="b")]
    center = _center(d, 3) if centred else None
    for rho in RHO:
        lib = ops.PagedLibrary.from_doc_caches(caches, rho, dev, center=center)
        assert lib.slots_per_page == 512 and lib.d == -(-d // 64) * 64 and lib.d_valid == d
        _check_pool(lib, caches, rho, center)


def test_build_many_chunks_and_slot_padding(dev):
    """Many small chunks (grid >> CUs), pages padded to a fixed slots_per_page."""
    say("pool build many chunks")
    g = torch.Generator().manual_seed(5)
    n = torch.randint(1, 65, (900,), generator=g).tolist()
    caches = [_cache(n[:450], 128, 6), _cache(n[450:], 128, 7)]
    center = _center(128, 8)
    lib = ops.PagedLibrary.from_doc_caches(caches, 0.75, dev, center=center, slots_per_page=96)
    assert lib.slots_per_page == 128
    _check_pool(lib, caches, 0.75, center)


def test_built_pool_reads_like_oracle(dev):
    """Route + decode read over the built pool against the oracle on the fp64 Library."""
    say("pool build -> route + read")
    d = 256
    caches = [_cache([512, 200, 17, 512, 3, 90, 400], d, 11), _cache([64, 64, 1, 33], d, 12)]
    center = _center(d, 13)
    lib = ops.PagedLibrary.from_doc_caches(caches, 0.25, dev, center=center)
    g = torch.Generator().manual_seed(14)
    q = unit_rows(6, d, g)
    qg = torch.tensor([0, 1, 0, 1, 1, 0], dtype=torch.int32)
    _, idx, wsel = ops.route_topk(q.to(dev), lib, qg.to(dev), top_k=3)
    out = ops.library_read_decode(q.to(dev), lib, idx, wsel, qg.to(dev)).cpu().double()
    for m, gi in enumerate(qg.tolist()):
        rows = [c["K"][0.25] for c in caches[gi]["chunks"]]
        K, M, S = O.library_tensors(rows, dtype=torch.float64, center_mu=center[0.25].double())
        qm = q[m].view(1, 1, -1).double()
        assert float(O.boundary_gap(qm, S, 3).min()) > 2e-5      # far above the fp32 dot rounding
        ref, _ = O.branch_read(qm, K, M, S, top_k=3)
        assert float((out[m] - ref.view(-1)).abs().max()) < 2e-3


def test_build_is_deterministic_and_untied_values(dev):
    say("pool build determinism / untied V")
    caches = [_cache([300, 12, 512], 192, 21, untied=True)]
    center = _center(192, 22)
    a = ops.PagedLibrary.from_doc_caches(caches, 0.75, dev, center=center)
    b = ops.PagedLibrary.from_doc_caches(caches, 0.75, dev, center=center)
    assert torch.equal(a.S, b.S) and torch.equal(a.pages, b.pages)
    assert a.values is not None
    for c, ch in enumerate(caches[0]["chunks"]):
        v = ch["V"][0.75]
        n = v.shape[0]
        assert torch.equal(a.values[c, :n, :192].cpu(), v)          # values are not centred
        assert float(a.values[c, n:].abs().max() if n < 512 else 0.0) == 0.0
    _check_pool(a, caches, 0.75, center)


def test_build_from_cache_file(dev, tmp_path):
    say("pool build from a cache file")
    cache = _cache([100, 512, 7], 128, 31)
    path = tmp_path / "docs" / "a.pt"
    save_doc_cache(cache, str(path))
    back = load_doc_cache(str(path))
    lib = ops.PagedLibrary.from_doc_caches(back, 0.25, dev)
    _check_pool(lib, [cache], 0.25, None)


def test_build_guards(dev):
    say("pool build guards")
    cache = _cache([10, 20], 64, 41)
    with pytest.raises(ValueError):
        ops.PagedLibrary.from_doc_caches(cache, 0.25, dev, slots_per_page=8, pad_to=8)   # < 20 slots
    empty = _cache([10, 20], 64, 41)
    empty["chunks"][1]["K"] = {r: torch.zeros(0, 64, dtype=torch.float16) for r in RHO}
    with pytest.raises(ValueError):
        ops.PagedLibrary.from_doc_caches(empty, 0.25, dev)
    with pytest.raises(KeyError):
        ops.PagedLibrary.from_doc_caches(cache, 0.5, dev)
    with pytest.raises(ValueError):
        ops.PagedLibrary.from_doc_caches(cache, 0.25, dev, center={0.25: torch.zeros(32)})
