"""Parity at the benchmark configurations' full sizes.

Multi-depth selector decode (8 depth Libraries of 64 x 512 slots, d_s 2560, 32 tokens, selector
top-2, routing top-8, write-back to d_r 5120): the step `bench.py --workload multi_depth` times
(kv_skill_v2_amd.multi_depth.MultiDepthDecode) against the fp64 oracle computed the reference's
way: the branch at EVERY candidate depth, each over all 64 chunks (xenc/injector.py:231-273),
then the selector weighting of every depth's update (xenc/selector.py:95-110), summed per token;
the same step at reduced sizes with one to three kept depths, unequal depth libraries and dense
routing.

Prefill (4 documents x 2048 rows x 32 chunks of 512 slots, d_s 2048, dense routing): the
forward r and the dQ backward of the composition `bench.py --workload prefill` times, over the
full tiling, checked on a row sample of every document (rows spread over all 16 row tiles) against
the oracle's branch_read and closed-form read_dq in fp64 (each row's r and dq depend only on that
row's q and upstream gradient).

Bars: routed chunk indices bit-exact (rows whose fp64 top-k boundary gap is below the fp32
rounding of the dots are reported, not failed); outputs max-abs 2e-3 and relative 1e-2."""

from __future__ import annotations

import math

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops, synth
from kv_skill_v2_amd.multi_depth import MultiDepthDecode
from kv_skill_v2_amd.selector import rms_norm

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def test_multi_depth_step_full_shape(dev):
    c = synth.MULTI_DEPTH
    say("multi-depth step, full shape", c)
    P, z, q_all, h, BwT = synth.multi_depth_workload(dev)
    Bw = BwT.transpose(1, 2).contiguous()
    del BwT
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    B, L, d, dr, k, ks = c["B"], c["depths"], c["d"], c["d_r"], c["top_k"], c["k_sel"]
    gen = torch.Generator().manual_seed(21)
    gate_w = (torch.randn(dr, generator=gen) * 0.02).to(dev)
    gate_b = torch.linspace(-2.0, 1.0, L).to(dev)
    log_gain = torch.linspace(-0.5, 0.5, L).to(dev)
    log_alpha = torch.tensor(math.log(0.02), device=dev)
    hn = rms_norm(h)
    md = MultiDepthDecode(lib, Bw, gate_w, gate_b, log_gain, log_alpha, k_sel=ks, top_k=k)
    out, idx, depth = md(z, q_all, h, hn)
    torch.cuda.synchronize()
    out, idx, depth = out.double().cpu(), idx.cpu(), depth.cpu()

    zc, hc, hnc = z.double().cpu(), h.double().cpu(), hn.double().cpu()
    wsel = O.selector_weights(zc, ks)                                   # [B, L], ties to the lower depth
    ref = torch.zeros(B, dr, dtype=torch.float64)
    near = 0
    for l in range(L):
        K, M, S = P.library(l)
        K, M, S = K.double().cpu(), M.cpu(), S.double().cpu()
        ql = q_all[l].double().cpu()
        r_l, _ = O.branch_read(ql.view(B, 1, d), K, M, S, top_k=k)      # every chunk, every token
        d_l = O.epilogue(hnc.view(B, 1, dr), r_l, Bw[l].double().cpu(), None, gate_w.double().cpu(),
                         gate_b[l].double().cpu(), log_gain[l].double().cpu())
        ref += O.selector_apply(d_l.view(B, dr), hc, wsel[:, l], math.log(0.02))
        # routed chunks of the rows that kept this depth
        rows = [i for i in range(B * ks) if int(depth[i]) == l]
        if rows:
            tok = [i // ks for i in rows]
            logit = ql[tok] @ S.T * 10.0
            want = O.topk_order(logit, k)
            gap = O.boundary_gap(ql[tok], S, k)
            for j, i in enumerate(rows):
                if not torch.equal(idx[i].long(), want[j]):
                    assert float(gap[j]) < 1e-6, (l, tok[j], idx[i].tolist(), want[j].tolist())
                    near += 1
    del K
    # kept depths: the selector's top-2 per token, in rank order
    assert torch.equal(depth.view(B, ks).long(), O.topk_order(zc, ks))
    err = (out - ref).abs().max().item()
    rel = ((out - ref).norm() / ref.norm()).item()
    say("max-abs", err, "rel", rel, "near-tie rows", near)
    assert err <= 2e-3 and rel <= 1e-2
    row_rel = ((out - ref).norm(dim=-1) / ref.norm(dim=-1)).max().item()
    assert row_rel <= 1e-2, row_rel


@pytest.mark.parametrize("chunks,B,ks,k", [([5, 12, 64, 3, 20], 24, 3, 4),
                                            ([16, 9, 30, 1], 40, 1, 8),
                                            ([64] * 6, 20, 2, 0)])
def test_multi_depth_step_reduced_shapes(dev, chunks, B, ks, k):
    """The multi-depth step (MultiDepthDecode) at reduced sizes against the fp64 oracle computed
    the reference's way (every depth read over all its chunks, then the selector weighting): one,
    two or three kept depths, depth libraries of unequal chunk counts (one of a single chunk),
    routing top-k below, at and above a library's chunk count and dense (k = 0), runs that the
    read groups by page and runs it does not (k_sel 1 with few rows per depth)."""
    L, N, d, dr = len(chunks), 64, 256, 96
    say("multi-depth step, reduced", dict(chunks=chunks, B=B, ks=ks, k=k))
    P = synth.pool(chunks, N, d, device=dev)
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    gen = torch.Generator().manual_seed(B + L + ks)
    z = torch.randn(B, L, generator=gen)
    q_all = torch.nn.functional.normalize(torch.randn(L, B, d, generator=gen), dim=-1)
    h = torch.randn(B, dr, generator=gen)
    Bw = torch.randn(L, dr, d, generator=gen) / d ** 0.5
    gate_w = torch.randn(dr, generator=gen) * 0.05
    gate_b = torch.linspace(-1.0, 1.0, L)
    log_gain = torch.linspace(-0.3, 0.3, L)
    log_alpha = math.log(0.02)
    hn = rms_norm(h)
    md = MultiDepthDecode(lib, Bw.to(dev), gate_w.to(dev), gate_b.to(dev), log_gain.to(dev),
                          torch.tensor(log_alpha, device=dev), k_sel=ks, top_k=k)
    out, idx, depth = md(z.to(dev), q_all.to(dev), h.to(dev), hn.to(dev))
    torch.cuda.synchronize()
    out, depth = out.double().cpu(), depth.cpu()
    zc, hc, hnc = z.double(), h.double(), hn.double()
    wsel = O.selector_weights(zc, ks)
    ref = torch.zeros(B, dr, dtype=torch.float64)
    for l in range(L):
        K, M, S = P.library(l)
        K, M, S = K.double().cpu(), M.cpu(), S.double().cpu()
        r_l, _ = O.branch_read(q_all[l].double().view(B, 1, d), K, M, S, top_k=k)
        d_l = O.epilogue(hnc.view(B, 1, dr), r_l, Bw[l].double(), None, gate_w.double(), gate_b[l].double(),
                         log_gain[l].double())
        ref += O.selector_apply(d_l.view(B, dr), hc, wsel[:, l], log_alpha)
    assert torch.equal(depth.view(B, ks).long(), O.topk_order(zc, ks))
    err = (out - ref).abs().max().item()
    row_rel = ((out - ref).norm(dim=-1) / ref.norm(dim=-1)).max().item()
    say("max-abs", err, "row-rel", row_rel)
    assert err <= 2e-3 and row_rel <= 1e-2


def test_prefill_full_shape_row_sample(dev):
    G, T, C, N, d = 4, 2048, 32, 512, 2048
    say("prefill full shape", dict(G=G, T=T, C=C, N=N, d=d))
    P = synth.pool([C] * G, N, d, device=dev)
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    plan = ops.row_plan(lib, [T] * G)
    q = synth.queries(G * T, d, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    g_up = torch.randn(G * T, d, generator=gen, device=dev)
    with torch.no_grad():
        w, _, _, qh = ops.route_topk_rows(q, lib, plan, top_k=0, emit_f16=True)
        r, p = ops.prefill_forward(q, w, lib, plan, qh=qh)
        dq = ops.prefill_backward_routed(g_up, w, p, lib, plan, route_temp=10.0)
        # the same gradient through the read's dq and a separate pass adding the routing term
        dq2, gamma = ops.prefill_backward(g_up, w, p, lib, plan)
        ops.route_backward(w, gamma, lib, plan, 10.0, dq2)
    torch.cuda.synchronize()
    sep = float((dq - dq2).abs().max()) / float(dq2.abs().max())
    say("routed backward vs separate route pass, max-abs / max", sep)
    assert sep <= 1e-5
    # two rows in each 128-row tile, at varying offsets, plus the first and last row
    sample = sorted({0, T - 1} | {t * 128 + (37 * t + 5) % 128 for t in range(16)}
                    | {t * 128 + (91 * t + 64) % 128 for t in range(16)})
    for g in range(G):
        K, M, S = P.library(g)
        K, M, S = K.double().cpu(), M.cpu(), S.double().cpu()
        rows = torch.tensor(sample) + g * T
        qs = q[rows.to(dev)].double().cpu().view(1, -1, d)
        gs = g_up[rows.to(dev)].double().cpu().view(1, -1, d)
        ref_r, ref_w = O.branch_read(qs, K, M, S, top_k=0)
        ref_dq, _ = O.read_dq(qs, K, M, S, gs, top_k=0)
        got_r = r[rows.to(dev)].double().cpu()
        got_dq = dq[rows.to(dev)].double().cpu()
        got_w = w[rows.to(dev)].double().cpu()
        e_r = (got_r - ref_r[0]).abs().max().item()
        rel_r = ((got_r - ref_r[0]).norm(dim=-1) / ref_r[0].norm(dim=-1)).max().item()
        rel_dq = ((got_dq - ref_dq[0]).norm(dim=-1) / ref_dq[0].norm(dim=-1)).max().item()
        mx_dq = ((got_dq - ref_dq[0]).abs().max() / ref_dq[0].abs().max()).item()
        e_w = (got_w - ref_w[0]).abs().max().item()
        say("document", g, "r max-abs", e_r, "r row-rel", rel_r, "dq row-rel", rel_dq, "dq max-rel", mx_dq,
            "w max-abs", e_w)
        assert e_r <= 2e-3 and rel_r <= 1e-2
        assert rel_dq <= 1e-2 and mx_dq <= 1e-2
        assert e_w <= 1e-5
