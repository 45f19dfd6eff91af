"""GPU: xenc_library_read_decode_noalloc (the allocation-free decode read, a file-scope scratch
array in place of the workspace) against xenc_library_read_decode, both called through the C ABI
on the same inputs.  The two share their kernels, so the results must be bit-identical.  Two
calls in a row: the second with a smaller input (fewer rows, fewer routed chunks), over the
first call's leftover scratch contents; one large call (two-pass merge) and small ones (the
in-kernel merge with its arrival counters, which every call must leave zero).  Sizes past the
scratch are rejected with XENC_ESCRATCH before any launch."""

from __future__ import annotations

import pytest
import torch

from kv_skill_v2_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

ESCRATCH = -6


def say(*a):
    print("[case]", *a, flush=True)


def _noalloc(q, lib, idx, wsel, qg, nsplit, read_temp=12.0, softmax=True):
    M, d = q.shape
    r = torch.full((M, lib.d), float("nan"), dtype=torch.float32, device=q.device)
    rc = _lib.lib().xenc_library_read_decode_noalloc(
        q.data_ptr(), q.stride(0), M, lib.d, lib.pages.data_ptr(), lib.slots_per_page, lib.pages.stride(0),
        lib.chunk_page.data_ptr(), lib.chunk_nvalid.data_ptr(), lib.chunk_ptr.data_ptr(), qg.data_ptr(),
        lib.n_libraries, idx.data_ptr(), wsel.data_ptr(), idx.shape[1], float(read_temp), int(softmax),
        int(nsplit), r.data_ptr(), r.stride(0), _lib.stream_handle(q.device))
    return rc, r


def _case(dev, counts, N, d, M, top_k, seed):
    P = synth.pool(counts, N, d, device=dev)
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    q = synth.queries(M, d, device=dev, seed=seed)
    qg = (torch.arange(M, device=dev) % len(counts)).to(torch.int32)
    _, idx, wsel = ops.route_topk(q, lib, qg, top_k=top_k)
    return lib, q, qg, idx, wsel


@pytest.mark.parametrize("order", ["large_then_small", "small_then_smaller"])
def test_noalloc_matches_workspace_entry_point(dev, order):
    if order == "large_then_small":
        # 64 rows x 8 routed pages: 512 workgroups, two-pass merge; then 3 rows x 2 pages with
        # 4 splits each (24 workgroups, in-kernel merge through the counters)
        calls = [(synth.batched_chunk_counts(64, 8, 16), 512, 2048, 64, 8, 1),
                 ([5, 9, 3], 256, 1024, 3, 2, 4)]
    else:
        calls = [([16], 512, 2048, 4, 4, 8), ([7], 128, 512, 1, 3, 2)]
    for i, (counts, N, d, M, top_k, nsplit) in enumerate(calls):
        say("noalloc", order, dict(call=i, libraries=len(counts), N=N, d=d, M=M, top_k=top_k, nsplit=nsplit))
        lib, q, qg, idx, wsel = _case(dev, counts, N, d, M, top_k, seed=30 + i)
        for softmax in (True, False):
            ref = ops.library_read_decode(q, lib, idx, wsel, qg, softmax=softmax, nsplit=nsplit)
            rc, got = _noalloc(q, lib, idx, wsel, qg, nsplit, softmax=softmax)
            torch.cuda.synchronize()
            assert rc == 0, _lib.lib().xenc_strerror(rc)
            assert torch.equal(got, ref), (i, softmax, (got - ref).abs().max().item())
            # a repeat over this call's own leftovers: same bits
            rc, again = _noalloc(q, lib, idx, wsel, qg, nsplit, softmax=softmax)
            torch.cuda.synchronize()
            assert rc == 0 and torch.equal(again, ref)


def test_noalloc_rejects_sizes_past_the_scratch(dev):
    say("noalloc size guards")
    lib, q, qg, idx, wsel = _case(dev, [4], 64, 256, 2, 2, seed=40)
    L = _lib.lib()
    st = _lib.stream_handle(dev)
    r = torch.zeros(2, lib.d, device=dev)
    args = lambda M, kk, nsplit, d: (q.data_ptr(), d, M, d, lib.pages.data_ptr(), lib.slots_per_page,  # noqa: E731
                                     lib.pages.stride(0), lib.chunk_page.data_ptr(), lib.chunk_nvalid.data_ptr(),
                                     lib.chunk_ptr.data_ptr(), qg.data_ptr(), 1, idx.data_ptr(), wsel.data_ptr(),
                                     kk, 12.0, 1, nsplit, r.data_ptr(), d, st)
    # more rows than the scratch's counter region
    assert L.xenc_library_read_decode_noalloc(*args(1025, 2, 1, 256)) == ESCRATCH
    # partials past 64 MiB: 1024 rows x 8 pages x 4 splits x 4096 floats
    assert L.xenc_library_read_decode_noalloc(*args(1024, 8, 4, 4096)) == ESCRATCH
    # bad arguments keep their own code
    assert L.xenc_library_read_decode_noalloc(*args(2, 2, 0, 256)) == -1
    with pytest.raises(ValueError):
        _lib.check(ESCRATCH, "xenc_library_read_decode_noalloc")
    torch.cuda.synchronize()
