"""GPU: reads of pages longer than 512 slots on the MFMA path (sub-pages joined through their
log-sum-exp, ops.read_sub_pages): forward and autograd against the fp64 oracle.

- the injector path the reference runs with any skill length: XEncInjector over a skill of 1024
  rows and a prompt of 2 x 12 tokens (more rows than the decode path takes), forward and the
  interface gradients (xenc/injector.py:100-118, 185-197, 239-265);
- ops.library_read (route + read, autograd through both) on pools of 1024- and 640-slot pages
  with ragged valid counts, against O.branch_read and the closed-form O.read_dq;
- ops.read_rows with untied values and the linear read, gradients in q and w against fp64
  autograd of O.read.

Bars: those of the MFMA prefill read (fp16 operands, fp32 accumulation): max-abs 2e-3 and
relative 1e-2 on r; relative 1e-2 (norm and largest entry) on gradients."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops, synth
from kv_skill_v2_amd.depth import DEPTHS, injection_layers
from kv_skill_v2_amd.injector import XEncInjector
from kv_skill_v2_amd.interface import ModelInterface
from kv_skill_v2_amd.library import Library
from tiny import TinyLM, close, oracle_forward, randomize, skill_rho, x_in

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _lib(P, dev, V=None):
    return ops.PagedLibrary(P.pages.to(dev), P.chunk_page.to(dev), P.chunk_nvalid.to(dev), P.chunk_ptr.to(dev),
                            P.S.to(dev), n_chunks=P.n_chunks, nvalid=P.nvalid, values=V)


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item(), ((a - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("read_softmax", [True, False])
def test_injector_skill_of_1024_rows(dev, read_softmax):
    say("XEncInjector 1024-row skill", dict(read_softmax=read_softmax))
    reader = TinyLM(d=32, n_layers=8).to(dev)
    layers = injection_layers(reader, DEPTHS)
    itf = ModelInterface(32, 64, layers).to(dev)
    randomize(itf, seed=9)
    skill = skill_rho(64, DEPTHS, n=1024, seed=5)
    x = x_in(32, T=12).to(dev)
    inj = XEncInjector(reader, itf, read_softmax=read_softmax)
    inj.load(skill)
    pool = inj._skill_pool(layers[0], dev)
    assert pool.slots_per_page == 1024
    g_up = torch.randn(2, 12, 32, generator=torch.Generator().manual_seed(3))
    itf.zero_grad()
    out = reader(x)
    (out * g_up.to(dev)).sum().backward()
    inj.detach()
    lib1 = Library([skill], layers, DEPTHS)     # the one-chunk form of the same skill (oracle operands)
    tensors = {li: (lib1.K[li].cpu(), lib1.mask[li].cpu(), lib1.S[li].cpu()) for li in lib1.layers}
    ref, (it, _) = oracle_forward(reader, x, itf, tensors, read_softmax=read_softmax, grad=True)
    ok, err, rn = close(out, ref)
    assert ok, (err, rn)
    (ref * g_up.double()).sum().backward()
    ours, theirs = dict(itf.named_parameters()), dict(it.named_parameters())
    for name in ("A.weight", "B.weight", "gate_w", "gate_b", "log_gain"):
        ok, err, rn = close(ours[name].grad, theirs[name].grad, rel=2e-2, atol=5e-3)
        assert ok, (name, err, rn)


@pytest.mark.parametrize("N,counts,rows,top_k", [(1024, [3], [20], 0), (640, [4, 2], [33, 17], 2),
                                                 (1024, [2, 5], [9, 130], 3)])
def test_library_read_large_pages(dev, N, counts, rows, top_k):
    say("library_read large pages", dict(N=N, counts=counts, rows=rows, top_k=top_k))
    d = 128
    P = synth.pool(counts, N, d, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    assert not ops.prefill_ok(lib)
    plan = ops.row_plan(lib, rows)
    M_ = sum(rows)
    q = synth.queries(M_, d, device="cpu", seed=19)
    qd = q.to(dev).requires_grad_(True)
    r, w = ops.library_read(qd, lib, plan, top_k=top_k)
    g = torch.randn(M_, d, generator=torch.Generator().manual_seed(4))
    (r * g.to(dev)).sum().backward()
    off = 0
    for gi, T in enumerate(rows):
        K, Mk, S = P.library(gi)
        qg = q[off:off + T].double().view(1, T, d)
        ref, _ = O.branch_read(qg, K.double(), Mk, S.double(), top_k=top_k)
        err = (r[off:off + T].detach().double().cpu() - ref[0]).abs().max().item()
        rel = ((r[off:off + T].detach().double().cpu() - ref[0]).norm() / ref.norm()).item()
        assert err <= 2e-3 and rel <= 1e-2, (gi, err, rel)
        dq, _ = O.read_dq(qg, K.double(), Mk, S.double(), g[off:off + T].double().view(1, T, d), top_k=top_k)
        rn, rm = _rel(qd.grad[off:off + T], dq[0])
        assert rn <= 1e-2 and rm <= 1e-2, (gi, rn, rm)
        off += T


@pytest.mark.parametrize("read_softmax,untied", [(True, True), (False, False), (False, True)])
def test_read_rows_large_pages_grads(dev, read_softmax, untied):
    say("read_rows large pages", dict(read_softmax=read_softmax, untied=untied))
    d, N, C, M_ = 128, 1024, 3, 12
    P = synth.pool([C], N, d, device="cpu", tail_lo=1)
    K, Mk, S = P.library(0)
    gen = torch.Generator().manual_seed(8)
    V = torch.nn.functional.normalize(torch.randn(K.shape, generator=gen), dim=-1).half() if untied else None
    Vp = None
    if untied:
        Vp = torch.zeros_like(P.pages)
        Vp[P.chunk_page.long()] = V.masked_fill(~Mk.unsqueeze(-1), 0.0)
    lib = _lib(P, dev, None if Vp is None else Vp.to(dev))
    q = synth.queries(M_, d, device="cpu", seed=23)
    w = torch.softmax(torch.randn(M_, C, generator=gen), -1)
    qd = q.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    idx = torch.arange(C, dtype=torch.int32).repeat(M_, 1).to(dev)
    r = ops.read_rows(qd, wd, idx, wd.detach(), lib, 12.0, read_softmax)
    g = torch.randn(M_, d, generator=gen)
    (r * g.to(dev)).sum().backward()
    q64 = q.double().view(1, M_, d).requires_grad_(True)
    w64 = w.double().view(1, M_, C).requires_grad_(True)
    ref, _ = O.read(q64, K.double(), Mk, w64, 12.0, read_softmax, None if V is None else V.double())
    (ref * g.double().view(1, M_, d)).sum().backward()
    err = (r.detach().double().cpu() - ref[0].detach()).abs().max().item()
    rel = ((r.detach().double().cpu() - ref[0].detach()).norm() / ref.detach().norm()).item()
    assert err <= 2e-3 and rel <= 1e-2, (err, rel)
    for ours, theirs, name in ((qd.grad, q64.grad[0], "dq"), (wd.grad, w64.grad[0], "dw")):
        rn, rm = _rel(ours, theirs)
        assert rn <= 1e-2 and rm <= 1e-2, (name, rn, rm)


def test_sub_pages_layout(dev):
    """The re-paged pool: sub-chunk j of chunk c holds its slots 512 j .. and the valid counts,
    parents and linear-read ratios follow the chunk's valid count."""
    say("sub-page layout")
    P = synth.pool([3, 2], 1024, 64, device="cpu", tail_lo=1)
    lib = _lib(P, dev)
    sp = lib.sub_pages()
    assert sp.lib.slots_per_page == ops.SUB_SPAN
    c_sub = 0
    for gi, nch in enumerate(P.n_chunks):
        base = sum(P.n_chunks[:gi])
        j_local = 0
        for c in range(nch):
            n = P.nvalid[base + c]
            for j in range(-(-n // 512)):
                nj = min(512, n - 512 * j)
                assert sp.lib.nvalid[c_sub] == nj
                src = P.pages[int(P.chunk_page[base + c]), 512 * j:512 * j + nj]
                assert torch.equal(sp.lib.pages[c_sub, :nj].cpu(), src)
                assert int(sp.parent[gi, j_local]) == c and bool(sp.valid[gi, j_local])
                assert abs(float(sp.ratio[gi, j_local]) - (nj / n) ** 0.5) < 1e-6
                c_sub += 1
                j_local += 1
        assert not sp.valid[gi, j_local:].any()
