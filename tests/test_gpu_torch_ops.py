"""GPU: the torch.ops.xenc operators (kv_skill_v2_amd/torch_ops.py) under torch.library.opcheck
(schema and mutation declarations, fake / meta kernels against the real outputs, autograd
registration, and AOT dispatch with dynamic shapes including the backward), plus a HIP graph
captured through torch.ops and replayed with new query rows.

The operators replace LibraryInjector.route and the read of _branch (xenc/injector.py:220-265),
and DecodeReader.__call__ (xenc/d23_read_kernels.py:145-160)."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops, synth
from kv_skill_v2_amd.torch_ops import kept_width

pytestmark = pytest.mark.gpu

CHECKS = ("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_dynamic")


def say(*a):
    print("[case]", *a, flush=True)


def _pool(dev, counts=(5, 3), N=128, d=256, seed=0):
    P = synth.pool(list(counts), N, d, device="cpu", tail_lo=1)
    return P, ops.PagedLibrary(P.pages.to(dev), P.chunk_page.to(dev), P.chunk_nvalid.to(dev),
                               P.chunk_ptr.to(dev), P.S.to(dev), n_chunks=P.n_chunks, nvalid=P.nvalid)


def test_opcheck_route_and_decode_read(dev):
    say("opcheck route_topk / library_read / route_read")
    P, lib = _pool(dev)
    q = synth.queries(6, lib.d, device=dev, seed=3)
    qg = torch.tensor([0, 1, 1, 0, 1, 0], dtype=torch.int32, device=dev)
    kk = kept_width(2, lib.cmax)
    args = (q, lib.S, lib.chunk_ptr, qg, 2, 10.0, lib.cmax, kk)
    torch.library.opcheck(torch.ops.xenc.route_topk.default, args, test_utils=CHECKS)
    _, idx, wsel = torch.ops.xenc.route_topk(*args)
    ws, rows = ops._WORKSPACES.get(dev, torch.cuda.current_stream(dev).cuda_stream, 6, kk, 2, lib.d)
    rargs = (q, lib.pages, lib.chunk_page, lib.chunk_nvalid, lib.chunk_ptr, qg, idx, wsel, 12.0, True, 2, ws, rows)
    torch.library.opcheck(torch.ops.xenc.library_read.default, rargs, test_utils=CHECKS)
    fargs = (q, lib.S, lib.pages, lib.chunk_page, lib.chunk_nvalid, lib.chunk_ptr, qg, 2, 10.0, lib.cmax, kk, 12.0,
             True, 2, ws, rows)
    torch.library.opcheck(torch.ops.xenc.route_read.default, fargs, test_utils=CHECKS)
    r = torch.ops.xenc.library_read(*rargs).cpu().double()
    for m, g in enumerate(qg.tolist()):
        K, M, S = P.library(g)
        ref, _ = O.branch_read(q[m].cpu().double().view(1, 1, -1), K.double(), M, S.double(), top_k=2)
        assert float((r[m] - ref.view(-1)).abs().max()) < 2e-3


def _close(a, b, rel=1e-5):
    """Equal up to fp32 rounding of a reordered sum: max-abs difference within rel of max |b|."""
    return float((a - b).abs().max()) <= rel * float(b.abs().max())


def test_opcheck_prefill_and_routing_with_autograd(dev):
    say("opcheck route_rows / library_prefill_fwd / bwd / route_backward_")
    P, lib = _pool(dev, counts=(3, 2), N=128, d=128)
    plan = ops.row_plan(lib, [70, 66])
    q = synth.queries(plan.M, lib.d, device=dev, seed=4).requires_grad_(True)
    rargs = (q, lib.S, lib.chunk_ptr, plan.row_ptr, plan.logit_tiles, plan.route_tiles, plan.n_logit, plan.n_route,
             0, 10.0, lib.cmax, kept_width(0, lib.cmax), True)
    torch.library.opcheck(torch.ops.xenc.route_rows.default, rargs, test_utils=CHECKS)
    w, _, _, qh = torch.ops.xenc.route_rows(*rargs)
    w = w.detach().requires_grad_(True)
    operands = ops._prefill_operands(lib, plan)
    fargs = (q, qh, w, *operands, 12.0, True, True)
    torch.library.opcheck(torch.ops.xenc.library_prefill_fwd.default, fargs, test_utils=CHECKS)
    r, p = torch.ops.xenc.library_prefill_fwd(*fargs)
    g = torch.randn(plan.M, lib.d, generator=torch.Generator(device=dev).manual_seed(1), device=dev)
    bargs = (g, w.detach(), p, *operands[2:], 12.0, True)
    torch.library.opcheck(torch.ops.xenc.library_prefill_bwd_dq.default, bargs, test_utils=CHECKS)
    dq = torch.zeros(plan.M, lib.d, device=dev)
    gargs = (dq, w.detach(), torch.randn_like(w), None, lib.S, lib.chunk_ptr, plan.row_ptr, plan.route_tiles,
             plan.n_route, 10.0)
    torch.library.opcheck(torch.ops.xenc.route_backward_.default, gargs,
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))
    # the backward with the routing term folded into the readout == bwd_dq + route_backward_
    dw_ext = torch.randn_like(w)
    xargs = (g, w.detach(), p, dw_ext, lib.S, *operands[2:], 12.0, True, 10.0)
    torch.library.opcheck(torch.ops.xenc.library_prefill_bwd_routed.default, xargs,
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))
    dq_x = torch.ops.xenc.library_prefill_bwd_routed(*xargs)
    dq_r, gamma = torch.ops.xenc.library_prefill_bwd_dq(*bargs)
    torch.ops.xenc.route_backward_(dq_r, w.detach(), gamma, dw_ext, lib.S, lib.chunk_ptr, plan.row_ptr,
                                   plan.route_tiles, plan.n_route, 10.0)
    assert _close(dq_x, dq_r), float((dq_x - dq_r).abs().max())
    # routing + read as one autograd node: schema, fakes, registered autograd ...
    cargs = (q, lib.S, lib.chunk_ptr, plan.row_ptr, plan.logit_tiles, plan.route_tiles, plan.n_logit, plan.n_route,
             2, 10.0, lib.cmax, kept_width(2, lib.cmax), *operands[:4], lib.chunk_page, lib.chunk_nvalid,
             plan.score_tiles, plan.readout_tiles, plan.n_score, plan.n_readout, lib.slots_per_page, 12.0, True, True)
    torch.library.opcheck(torch.ops.xenc.library_read_routed.default, cargs, test_utils=CHECKS)
    # ... and the same values (bit for bit) and gradients (to fp32 rounding: the routing term is
    # summed in another order) as the two operators, for a loss on both r and w (the gradient
    # reaching w from elsewhere enters the routing term)
    qa = q.detach().clone().requires_grad_(True)
    qb = q.detach().clone().requires_grad_(True)
    ra, wa, *_ = torch.ops.xenc.library_read_routed(qa, *cargs[1:])
    ((ra * g).sum() + 3.0 * (wa * wa).sum()).backward()
    wb, _, _, qhb = torch.ops.xenc.route_rows(qb, *rargs[1:8], 2, 10.0, lib.cmax, kept_width(2, lib.cmax), True)
    rb, _ = torch.ops.xenc.library_prefill_fwd(qb, qhb, wb, *operands, 12.0, True, True)
    ((rb * g).sum() + 3.0 * (wb * wb).sum()).backward()
    assert torch.equal(ra, rb) and torch.equal(wa, wb)
    assert _close(qa.grad, qb.grad), float((qa.grad - qb.grad).abs().max())
    # autograd through both operators equals the oracle's closed-form dq
    r, w2 = ops.library_read(q, lib, plan)
    (r * g).sum().backward()
    off = 0
    for gi, T in enumerate(plan.rows):
        K, M, S = P.library(gi)
        qs = q[off:off + T].detach().cpu().double().view(1, T, -1)
        ref_dq, _ = O.read_dq(qs, K.double(), M, S.double(), g[off:off + T].cpu().double().view(1, T, -1))
        got = q.grad[off:off + T].cpu().double()
        rel = float(((got - ref_dq[0]).norm(dim=-1) / ref_dq[0].norm(dim=-1)).max())
        assert rel < 1e-2, (gi, rel)
        off += T


def test_opcheck_paged_decode_joint(dev):
    say("opcheck paged_decode_joint")
    from kv_skill_v2_amd.decode_reader import DecodeReader
    gen = torch.Generator().manual_seed(5)
    N, hq, hkv, d, bs = 3, 16, 4, 128, 16
    op_k, op_v = (torch.randn(30, bs, hkv, d, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2))
    own_k, own_v = (torch.randn(10, bs, hkv, d, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2))
    q = torch.randn(N, hq, d, generator=gen).to(torch.bfloat16).to(dev)
    op_bt = torch.stack([torch.randperm(30, generator=gen)[:12] for _ in range(N)]).int().to(dev)
    own_bt = torch.stack([torch.randperm(10, generator=gen)[:3] for _ in range(N)]).int().to(dev)
    op_len = torch.tensor([150, 1, 190], dtype=torch.int32, device=dev)
    own_len = torch.tensor([3, 40, 1], dtype=torch.int32, device=dev)
    dec = DecodeReader(4, hq, hkv, d, max_keys=256, device=dev, chunk=64)
    out = torch.empty(N, hq, d, device=dev)
    args = (q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, d ** -0.5, dec.S, dec.chunk,
            dec.workspace, dec.max_n, out)
    torch.library.opcheck(torch.ops.xenc.paged_decode_joint.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))
    torch.ops.xenc.paged_decode_joint(*args)
    ref = O.decode_read_ref(*[t.cpu() for t in (q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len)],
                            d ** -0.5)
    assert float((out.cpu().double() - ref.double()).norm() / ref.double().norm()) < 2e-3


def test_graph_capture_through_torch_ops(dev):
    """route + read captured once through torch.ops.xenc, replayed for new query rows written into
    the captured input; every replay equals the eager operators bit for bit, with eager work and
    synchronisation between replays."""
    say("graph capture through torch.ops")
    P, lib = _pool(dev, counts=(9, 4, 6), N=256, d=512)
    M = 5
    qg = torch.tensor([0, 2, 1, 2, 0], dtype=torch.int32, device=dev)
    q_in = synth.queries(M, lib.d, device=dev, seed=8)

    def step(q):
        _, idx, wsel = ops.route_topk(q, lib, qg, top_k=3)
        return ops.library_read_decode(q, lib, idx, wsel, qg)

    step(q_in)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(q_in)
    torch.cuda.current_stream().wait_stream(s)
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        r_g = step(q_in)
    for seed in (11, 12, 13):
        q_new = synth.queries(M, lib.d, device=dev, seed=seed)
        q_in.copy_(q_new)
        gph.replay()
        torch.cuda.synchronize()
        ref = step(q_new.clone())
        torch.cuda.synchronize()
        assert torch.equal(r_g, ref), seed


def test_graph_capture_of_prefill_training_step(dev):
    """A whole training step of the routed MFMA read (xenc::library_read_routed forward and its
    backward through autograd) captured once in a HIP graph, as whole-network capture does it
    (grads set to None before the capture), then replayed for new query rows written into the
    captured leaf: r and q.grad of every replay equal an eager step bit for bit, with eager work
    and synchronisation between the replays."""
    say("graph capture of a prefill training step")
    P, lib = _pool(dev, counts=(5, 3), N=128, d=256)
    plan = ops.row_plan(lib, [80, 70])
    g_up = torch.randn(plan.M, lib.d, generator=torch.Generator(device=dev).manual_seed(3), device=dev)
    q_leaf = synth.queries(plan.M, lib.d, device=dev, seed=9).requires_grad_(True)

    def step(q):
        r, w = ops.library_read(q, lib, plan, top_k=2)
        ((r * g_up).sum() + (w * w).sum()).backward()
        return r

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            q_leaf.grad = None
            step(q_leaf)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    q_leaf.grad = None
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        r_g = step(q_leaf)
    for seed in (21, 22, 23):
        q_new = synth.queries(plan.M, lib.d, device=dev, seed=seed)
        with torch.no_grad():
            q_leaf.copy_(q_new)
        gph.replay()
        torch.cuda.synchronize()
        q_ref = q_new.clone().requires_grad_(True)
        r_ref = step(q_ref)
        torch.cuda.synchronize()
        assert torch.equal(r_g, r_ref), seed
        assert torch.equal(q_leaf.grad, q_ref.grad), (seed, float((q_leaf.grad - q_ref.grad).abs().max()))
