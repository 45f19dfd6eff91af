"""GPU parity of the MFMA prefill read (forward and autograd backward) against the CPU oracle.

The kernels take fp16 operands (q, the probabilities p, dS, the upstream gradient) with fp32
accumulation, so the bar is the task's fp16 tolerance: max-abs 2e-3 and relative 1e-2 on r; for
gradients (whose scale is set by the upstream gradient) the same relative bar on the norm and on
the largest entry."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _lib(P, dev):
    return ops.PagedLibrary(P.pages.to(dev), P.chunk_page.to(dev), P.chunk_nvalid.to(dev), P.chunk_ptr.to(dev),
                            P.S.to(dev), n_chunks=P.n_chunks, nvalid=P.nvalid)


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item(), ((a - b).abs().max() / b.abs().max()).item()


CASES = [
    # (d, N, chunks per library, rows per library, top_k)
    (256, 512, [4], [64], 2),
    (128, 64, [5, 3], [300, 17], 0),
    (256, 192, [7], [130], 3),
    (2048, 512, [6], [256], 0),
    (512, 128, [9, 2, 4], [40, 200, 129], 4),
]


@pytest.mark.parametrize("d,N,counts,rows,top_k", CASES)
def test_prefill_forward_parity(dev, d, N, counts, rows, top_k):
    say("prefill fwd", dict(d=d, N=N, counts=counts, rows=rows, top_k=top_k))
    P = synth.pool(counts, N, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    plan = ops.row_plan(lib, rows)
    q = synth.queries(sum(rows), d, device="cpu", seed=13)
    with torch.no_grad():
        r, w = ops.library_read(q.to(dev), lib, plan, top_k=top_k)
        wg, _, _ = ops.route_topk(q.to(dev), lib, ops._plan_groups(plan).to(dev), top_k=top_k)
        _, p = ops.prefill_forward(q.to(dev), wg, lib, plan)
    torch.cuda.synchronize()
    r, p = r.cpu().double(), ops.unpack_p(p, sum(rows)).cpu().float()
    off = 0
    for g, T in enumerate(rows):
        K, M, S = P.library(g)
        qg = q[off:off + T].double().view(1, T, d)
        ref, _ = O.branch_read(qg, K.double(), M, S.double(), top_k=top_k)
        err = (r[off:off + T] - ref[0]).abs().max().item()
        rel = ((r[off:off + T] - ref[0]).norm() / ref.norm()).item()
        assert err <= 2e-3 and rel <= 1e-2, (g, err, rel)
        a = torch.einsum("td,cnd->tcn", qg[0], K.double())
        pref = torch.softmax((a * 12.0).masked_fill(~M, float("-inf")), -1)
        C = K.shape[0]
        pk = p[off:off + T, :C * N].view(T, C, N).double()
        assert (pk - pref).abs().max().item() <= 1e-3, g
        off += T


@pytest.mark.parametrize("d,N,counts,rows,top_k", CASES)
def test_prefill_backward_parity(dev, d, N, counts, rows, top_k):
    say("prefill bwd", dict(d=d, N=N, counts=counts, rows=rows, top_k=top_k))
    P = synth.pool(counts, N, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    plan = ops.row_plan(lib, rows)
    M_ = sum(rows)
    q = synth.queries(M_, d, device="cpu", seed=17)
    gen = torch.Generator().manual_seed(7)
    g_up = torch.randn(M_, d, generator=gen)
    dw_ext = torch.randn(M_, lib.cmax, generator=gen)
    qd = q.to(dev).requires_grad_(True)
    r, w = ops.library_read(qd, lib, plan, top_k=top_k)
    loss = (r * g_up.to(dev)).sum() + (w * dw_ext.to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    dq = qd.grad.cpu()
    off = 0
    for g, T in enumerate(rows):
        K, M, S = P.library(g)
        C = K.shape[0]
        ref, _ = O.read_dq(q[off:off + T].double().view(1, T, d), K.double(), M, S.double(),
                           g_up[off:off + T].double().view(1, T, d), 12.0, 10.0, top_k,
                           dw_ext=dw_ext[off:off + T, :C].double().view(1, T, C))
        rn, rm = _rel(dq[off:off + T], ref[0])
        assert rn <= 1e-2 and rm <= 1e-2, (g, rn, rm)
        off += T


def test_prefill_requires_tileable_shapes(dev):
    say("prefill shape guard")
    P = synth.pool([3], 40, 64, device="cpu")
    lib = _lib(P, dev)
    plan = ops.row_plan(lib, [5])
    with pytest.raises(ValueError):
        ops.prefill_forward(torch.zeros(5, 64, device=dev), torch.zeros(5, 3, device=dev), lib, plan)


@pytest.mark.parametrize("variant", ["linear", "untied", "untied_linear"])
def test_prefill_variants_fwd_bwd(dev, variant):
    """Linear read (scores modes 2/3) and untied values (V pages in the readout, K in the dQ
    readout) vs the fp64 oracle forward and its autograd."""
    say("prefill variant", variant)
    d, N, C, T, top_k = 256, 192, 5, 70, 2
    soft = "linear" not in variant
    g = torch.Generator().manual_seed(21)
    rows = [torch.nn.functional.normalize(torch.randn(n, d, generator=g), dim=-1) for n in (192, 40, 1, 130, 77)]
    K, M, S = O.library_tensors(rows)
    V = None
    if "untied" in variant:
        V = torch.nn.functional.normalize(torch.randn(K.shape, generator=g), dim=-1) * M.unsqueeze(-1)
    lib = ops.PagedLibrary.from_padded(K, M, S, device=dev, V=V)
    q = synth.queries(T, d, device="cpu", seed=23)
    g_up = torch.randn(T, d, generator=g)
    qd = q.to(dev).requires_grad_(True)
    r, w = ops.library_read(qd, lib, lib.plan([T]), top_k=top_k, read_softmax=soft)
    (r * g_up.to(dev)).sum().backward()
    qo = q.double().view(1, T, d).requires_grad_(True)
    ref, _ = O.branch_read(qo, K.double(), M, S.double(), top_k=top_k, read_softmax=soft,
                           V=None if V is None else V.double())
    (ref[0] * g_up.double()).sum().backward()
    rn, rm = _rel(r.detach(), ref[0].detach())
    assert rn <= 1e-2 and (r.detach().cpu().double() - ref[0].detach()).abs().max() <= 2e-3, (rn, rm)
    rn, rm = _rel(qd.grad, qo.grad[0])
    assert rn <= 1e-2 and rm <= 1e-2, (rn, rm)


@pytest.mark.parametrize("counts,rows,top_k", [([32, 7, 130], [300, 64, 129], 0), ([32, 7, 130], [300, 0, 65], 5),
                                               ([1, 64], [70, 1], 1)])
@pytest.mark.parametrize("d", [256, 456])
def test_route_rows_matches_per_row_kernel(dev, counts, rows, top_k, d):
    """The many-row routing kernel gives the per-row kernel's routing: identical kept chunks
    (rows whose fp64 top-k gap is below 1e-5 are exempt) and weights within 1e-6; its fp16 copy
    of q is the cast.  d = 456 ends in a partial k-step of 72 columns."""
    say("route rows", dict(counts=counts, rows=rows, top_k=top_k, d=d))
    P = synth.pool(counts, 64, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    plan = ops.row_plan(lib, rows)
    q = synth.queries(sum(rows), d, device="cpu", seed=31)
    qg = ops._plan_groups(plan)
    w1, i1, s1 = ops.route_topk(q.to(dev), lib, qg.to(dev), top_k=top_k)
    w2, i2, s2, qh = ops.route_topk_rows(q.to(dev), lib, plan, top_k=top_k, emit_f16=True)
    assert (w1 - w2).abs().max().item() <= 1e-6
    assert torch.equal(qh, ops.cast_f16(q.to(dev)))
    i1, i2 = i1.cpu(), i2.cpu()
    off = 0
    for g, T in enumerate(rows):
        K, M, S = P.library(g)
        gap = O.boundary_gap(q[off:off + T].double(), S.double(), top_k)
        ok = gap > 1e-5
        assert torch.equal(i1[off:off + T][ok], i2[off:off + T][ok]), g
        off += T


@pytest.mark.parametrize("counts,rows", [([32, 7, 130], [300, 64, 129]), ([3], [33]), ([40, 2], [1, 97])])
def test_route_rows_fp16_rows_are_the_cast(dev, counts, rows):
    """The routing pass's fp16 copy of q (emit_f16) equals cast_f16 bit for bit on every row (ragged
    row tiles, several chunk tiles per row tile), and prefill_forward gives the same bits with it
    as with its own cast; library_read, which shares the copy between routing and read, equals
    the two calls."""
    say("route rows fp16 rows", dict(counts=counts, rows=rows))
    d = 128
    P = synth.pool(counts, 64, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    plan = ops.row_plan(lib, rows)
    q = synth.queries(sum(rows), d, device=dev, seed=5)
    w, _, _, qh = ops.route_topk_rows(q, lib, plan, top_k=0, emit_f16=True)
    assert torch.equal(qh, ops.cast_f16(q))
    r1, p1 = ops.prefill_forward(q, w, lib, plan, qh=qh)
    r2, p2 = ops.prefill_forward(q, w, lib, plan)
    assert torch.equal(r1, r2)
    u1, u2 = ops.unpack_p(p1, q.shape[0]), ops.unpack_p(p2, q.shape[0])
    off = 0
    for g, T in enumerate(rows):                 # p is written for each library's own chunks only
        n = counts[g] * 64
        assert torch.equal(u1[off:off + T, :n], u2[off:off + T, :n]), g
        off += T
    if sum(rows) >= ops.ROUTE_ROWS_MIN:
        r3, w3 = ops.library_read(q, lib, plan)
        assert torch.equal(r3, r2) and torch.equal(w3, w)


def test_prefill_single_slot_chunks(dev):
    """Chunks of 1 and 3 valid slots next to a full one, softmax and linear, forward and dQ."""
    say("prefill 1-slot chunks")
    d, N, T = 128, 64, 40
    g = torch.Generator().manual_seed(41)
    rows = [torch.nn.functional.normalize(torch.randn(n, d, generator=g), dim=-1) for n in (1, 64, 3)]
    K, M, S = O.library_tensors(rows)
    lib = ops.PagedLibrary.from_padded(K, M, S, device=dev, pad_to=64)
    q = synth.queries(T, d, device="cpu", seed=43)
    g_up = torch.randn(T, d, generator=g)
    for soft in (True, False):
        qd = q.to(dev).requires_grad_(True)
        r, w = ops.library_read(qd, lib, lib.plan([T]), top_k=2, read_softmax=soft)
        (r * g_up.to(dev)).sum().backward()
        qo = q.double().view(1, T, d).requires_grad_(True)
        ref, _ = O.branch_read(qo, K.double(), M, S.double(), top_k=2, read_softmax=soft)
        (ref[0] * g_up.double()).sum().backward()
        rn, _ = _rel(r.detach(), ref[0].detach())
        assert rn <= 1e-2 and (r.detach().cpu().double() - ref[0].detach()).abs().max() <= 2e-3, soft
        rn, rm = _rel(qd.grad, qo.grad[0])
        assert rn <= 1e-2 and rm <= 1e-2, (soft, rn, rm)


@pytest.mark.parametrize("M,d,ldx", [(1, 8, 8), (37, 64, 68), (300, 2048, 2048), (5, 4104, 4112), (9000, 32, 36)])
def test_cast_rows_f16_is_torch_rounding(dev, M, d, ldx):
    """xenc_cast_rows_f16 on strided fp32 rows equals torch's fp16 rounding bit for bit: rows past
    one workgroup per row (M > 8192), rows longer than one pass of the workgroup's threads
    (d / 4 > 1024), padded strides, and values past fp16's range and in its subnormals."""
    say("cast rows f16", dict(M=M, d=d, ldx=ldx))
    g = torch.Generator().manual_seed(M * 7 + d)
    base = torch.randn(M, ldx, generator=g) * torch.logspace(-9, 6, ldx)[None, :]
    x = base.to(dev)[:, :d]
    y = ops.cast_f16(x)
    assert y.shape == (M, d) and y.is_contiguous()
    assert torch.equal(y.view(torch.int16).cpu(), base[:, :d].half().view(torch.int16))
