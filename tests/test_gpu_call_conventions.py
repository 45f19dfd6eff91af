"""GPU: the calling conventions a caller of the reference's injector relies on.

- query rows given as a strided view (rows of a wider tensor), at a misaligned offset, or in
  fp16 / bf16 give the same bits as the same rows passed contiguous in fp32 (fp16 / bf16 rows are
  compared with their fp32 upcast, which is what the reference's read_fp32 path computes with);
- two streams reading at once: each stream has its own decode workspace, so calls issued on two
  streams without synchronisation between them give the bits of the same calls made one by one."""

from __future__ import annotations

import pytest
import torch

from kv_skill_v2_amd import ops, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _lib(P, dev):
    return ops.PagedLibrary(P.pages.to(dev), P.chunk_page.to(dev), P.chunk_nvalid.to(dev), P.chunk_ptr.to(dev),
                            P.S.to(dev), n_chunks=P.n_chunks, nvalid=P.nvalid)


def _same(a, b):
    return all(torch.equal(x, y) for x, y in zip(a, b))


def test_strided_misaligned_and_half_queries(dev):
    say("query layouts")
    d = 512
    P = synth.pool([9, 14, 5], 128, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    M = 7
    qg = torch.tensor([0, 1, 2, 1, 0, 2, 1], dtype=torch.int32, device=dev)
    q = synth.queries(M, d, device=dev, seed=4)
    ref = ops.route_read_decode(q, lib, qg, top_k=3)
    wide = torch.zeros(M, d + 24, device=dev)
    wide[:, :d] = q
    assert _same(ops.route_read_decode(wide[:, :d], lib, qg, top_k=3), ref)       # row stride d + 24
    shifted = torch.zeros(M, d + 1, device=dev)
    shifted[:, 1:] = q
    assert _same(ops.route_read_decode(shifted[:, 1:], lib, qg, top_k=3), ref)    # 4-byte offset: copied
    for dt in (torch.float16, torch.bfloat16):
        qh = q.to(dt)
        assert _same(ops.route_read_decode(qh, lib, qg, top_k=3),
                     ops.route_read_decode(qh.float(), lib, qg, top_k=3)), dt
    # the many-row MFMA path takes the same views
    plan = ops.row_plan(lib, [70, 0, 0])
    qm = synth.queries(70, d, device=dev, seed=6)
    wide = torch.zeros(70, d + 24, device=dev)
    wide[:, :d] = qm
    with torch.no_grad():
        r1, w1 = ops.library_read(qm, lib, plan, top_k=2)
        r2, w2 = ops.library_read(wide[:, :d], lib, plan, top_k=2)
    assert torch.equal(r1, r2) and torch.equal(w1, w2)


def test_two_streams_at_once(dev):
    say("two streams")
    d = 1024
    P = synth.pool([12, 20, 7, 16], 256, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    qa = synth.queries(6, d, device=dev, seed=31)
    qb = synth.queries(9, d, device=dev, seed=32)
    ga = torch.tensor([0, 1, 2, 3, 1, 0], dtype=torch.int32, device=dev)
    gb = torch.tensor([3, 2, 1, 0, 0, 1, 2, 3, 2], dtype=torch.int32, device=dev)
    ref_a = [t.clone() for t in ops.route_read_decode(qa, lib, ga, top_k=4)]
    ref_b = [t.clone() for t in ops.route_read_decode(qb, lib, gb, top_k=4)]
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for _ in range(4):
        with torch.cuda.stream(sa):
            oa = ops.route_read_decode(qa, lib, ga, top_k=4)
        with torch.cuda.stream(sb):
            ob = ops.route_read_decode(qb, lib, gb, top_k=4)
        outs.append((oa, ob))
    torch.cuda.synchronize()
    for oa, ob in outs:
        assert _same(oa, ref_a) and _same(ob, ref_b)
