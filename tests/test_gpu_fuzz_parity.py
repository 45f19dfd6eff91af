"""Seeded random shapes through the product's decode, prefill and op-B paths against the CPU oracle.

Each case draws its shape from a fixed seed (page size, d, chunk and row counts per library,
top-k, slot splits, softmax or linear read, how ragged the last page of a library is), so a
failure names a reproducible case.  The draws stay inside what the entry points accept and
keep the fp64 oracle's work to a few million multiply-adds per case.

Bar: routed indices bit-exact where the fp64 top-k boundary gap exceeds fp32 rounding (ties to
the lower index), weights within 1e-6; reads within max-abs 2e-3 / rel 1e-2 and, since slots are
fp16-exact and sums fp32, within 1e-4 max-abs; dQ within 1e-2 (norm- and max-relative)."""

from __future__ import annotations

import random

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops, synth

pytestmark = pytest.mark.gpu

GAP = 1e-6
MAX_ABS, REL, PRECISE = 2e-3, 1e-2, 1e-4


def say(*a):
    print("[case]", *a, flush=True)


def _lib(P, dev):
    return ops.PagedLibrary(P.pages.to(dev), P.chunk_page.to(dev), P.chunk_nvalid.to(dev), P.chunk_ptr.to(dev),
                            P.S.to(dev), n_chunks=P.n_chunks, nvalid=P.nvalid)


def _decode_case(i: int) -> dict:
    rng = random.Random(1000 + i)
    d = rng.choice([8, 24, 64, 136, 256, 520, 1024, 2048, 2560, 4096])
    N = rng.choice([1, 7, 32, 64, 100, 256, 512, 640])
    cap = max(1, min(70, 3_000_000 // (N * d)))
    G = rng.randint(1, 4)
    counts = [rng.randint(1, cap) for _ in range(G)]
    rows = [rng.randint(0, 6) for _ in range(G)]
    rows[rng.randrange(G)] += 1
    return dict(d=d, N=N, counts=counts, rows=rows, top_k=rng.choice([0, 1, 2, 3, 5, 8, 64]),
                nsplit=rng.choice([None, 1, 2, 3, 8, 16]), softmax=rng.random() < 0.75,
                tail_lo=rng.choice([1, max(1, N // 2), N]), shuffle_rows=rng.random() < 0.5, seed=50 + i)


def _decode_many_rows_case(i: int) -> dict:
    """Many rows sharing few libraries: the page-grouped read (rows ranked by page) and, from
    256 rows, the one-workgroup-per-row top-k."""
    rng = random.Random(3000 + i)
    G = rng.randint(1, 3)
    return dict(d=rng.choice([64, 128, 256]), N=rng.choice([32, 64, 128]),
                counts=[rng.randint(8, 40) for _ in range(G)], rows=[rng.randint(40, 150) for _ in range(G)],
                top_k=rng.choice([2, 4, 8]), nsplit=rng.choice([None, 1, 2]), softmax=rng.random() < 0.75,
                tail_lo=1, shuffle_rows=rng.random() < 0.5, seed=90 + i)


@pytest.mark.parametrize("case", [("shapes", i) for i in range(48)] + [("many_rows", i) for i in range(8)],
                         ids=lambda c: f"{c[0]}{c[1]}")
def test_decode_random_shapes(dev, case):
    kind, i = case
    c = _decode_case(i) if kind == "shapes" else _decode_many_rows_case(i)
    say("decode", kind, i, c)
    P = synth.pool(c["counts"], c["N"], c["d"], device="cpu", tail_lo=c["tail_lo"])
    lib = _lib(P, dev)
    groups = [g for g, n in enumerate(c["rows"]) for _ in range(n)]
    if c["shuffle_rows"]:
        random.Random(c["seed"]).shuffle(groups)
    M, d, top_k = len(groups), c["d"], c["top_k"]
    q = synth.queries(M, d, device="cpu", seed=c["seed"])
    qg = torch.tensor(groups, dtype=torch.int32, device=dev)
    w, idx, wsel, r = ops.route_read_decode(q.to(dev), lib, qg, top_k=top_k, read_temp=12.0,
                                            softmax=c["softmax"], nsplit=c["nsplit"])
    # the one-call operator equals route_topk + library_read_decode bit for bit
    w2, idx2, wsel2 = ops.route_topk(q.to(dev), lib, qg, top_k=top_k)
    r2 = ops.library_read_decode(q.to(dev), lib, idx2, wsel2, qg, read_temp=12.0, softmax=c["softmax"],
                                 nsplit=c["nsplit"])
    torch.cuda.synchronize()
    assert torch.equal(idx, idx2) and torch.equal(w, w2) and torch.equal(wsel, wsel2)
    assert torch.equal(r, r2)
    w, idx, wsel, r = w.cpu(), idx.cpu(), wsel.cpu(), r.double().cpu()
    for m, g in enumerate(groups):
        K, Mk, S = P.library(g)
        C = K.shape[0]
        qm = q[m:m + 1].double()
        wref = O.route(qm, S.double(), 10.0, top_k)[0]
        kept = C if (not top_k or top_k >= C) else top_k
        order = torch.arange(C) if kept == C else O.topk_order(qm @ S.double().T, top_k)[0]
        if kept == C or float(O.boundary_gap(qm, S.double(), top_k)[0]) > GAP:   # clear of a top-k tie
            assert idx[m, :kept].tolist() == order.tolist(), (m, idx[m].tolist(), order.tolist())
            assert float((w[m, :C].double() - wref).abs().max()) <= 1e-6, m
        assert bool((idx[m, kept:] == -1).all()), m
        assert float(w[m, C:].abs().sum()) == 0.0, m
        # the read, checked at the GPU's own routing (independent of near-ties)
        sel = idx[m, :kept].long()
        ref = O.read_routed(qm, K.double(), Mk, sel.view(1, -1), wsel[m, :kept].double().view(1, -1), 12.0,
                            c["softmax"])[0]
        err = float((r[m] - ref).abs().max())
        rel = float((r[m] - ref).norm() / ref.norm().clamp_min(1e-30))
        assert err <= MAX_ABS and rel <= REL and err <= PRECISE, (m, g, err, rel)


def _prefill_case(i: int) -> dict:
    rng = random.Random(2000 + i)
    d = rng.choice([64, 128, 192, 256, 512, 1024])
    N = rng.choice([64, 128, 192, 256, 512])
    G = rng.randint(1, 3)
    rows = [rng.choice([1, 17, 64, 100, 150]) for _ in range(G)]
    cap = max(1, min(12, 40_000_000 // (max(rows) * N * d)))
    counts = [rng.randint(1, cap) for _ in range(G)]
    return dict(d=d, N=N, counts=counts, rows=rows, top_k=rng.choice([0, 1, 2, 4]),
                tail_lo=rng.choice([1, N // 2, N]), seed=70 + i)


@pytest.mark.parametrize("i", range(16))
def test_prefill_random_shapes(dev, i):
    c = _prefill_case(i)
    say("prefill", i, c)
    P = synth.pool(c["counts"], c["N"], c["d"], device="cpu", tail_lo=c["tail_lo"])
    lib = _lib(P, dev)
    plan = ops.row_plan(lib, c["rows"])
    Mt, d, top_k = plan.M, c["d"], c["top_k"]
    q = synth.queries(Mt, d, device="cpu", seed=c["seed"])
    gen = torch.Generator().manual_seed(c["seed"])
    g_up = torch.randn(Mt, d, generator=gen)
    dw_ext = torch.randn(Mt, lib.cmax, generator=gen)
    qd = q.to(dev).requires_grad_(True)
    r, w = ops.library_read(qd, lib, plan, top_k=top_k)
    ((r * g_up.to(dev)).sum() + (w * dw_ext.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    r, w, dq = r.detach().double().cpu(), w.detach().double().cpu(), qd.grad.double().cpu()
    off = 0
    for g, T in enumerate(c["rows"]):
        K, Mk, S = P.library(g)
        C = K.shape[0]
        qs = q[off:off + T].double()
        ok = torch.ones(T, dtype=torch.bool)                   # rows clear of a top-k tie
        if top_k and top_k < C:
            ok = O.boundary_gap(qs, S.double(), top_k) > GAP
        ref_r, ref_w = O.branch_read(qs.view(1, T, d), K.double(), Mk, S.double(), top_k=top_k)
        ref_dq, _ = O.read_dq(qs.view(1, T, d), K.double(), Mk, S.double(), g_up[off:off + T].double().view(1, T, d),
                              12.0, 10.0, top_k, dw_ext=dw_ext[off:off + T, :C].double().view(1, T, C))
        a, b = r[off:off + T][ok], ref_r[0][ok]
        if a.numel():
            err = float((a - b).abs().max())
            rel = float((a - b).norm() / b.norm().clamp_min(1e-30))
            assert err <= MAX_ABS and rel <= REL, (g, err, rel)
            assert float((w[off:off + T, :C][ok] - ref_w[0][ok]).abs().max()) <= 1e-5, g
            x, y = dq[off:off + T][ok], ref_dq[0][ok]
            rn = float((x - y).norm() / y.norm().clamp_min(1e-30))
            rm = float((x - y).abs().max() / y.abs().max().clamp_min(1e-30))
            assert rn <= 1e-2 and rm <= 1e-2, (g, rn, rm)
        off += T


def _decode_reader_case(i: int) -> dict:
    rng = random.Random(4000 + i)
    G = rng.choice([1, 2, 3, 4, 8])
    d = rng.choice([x for x in (8, 64, 80, 128, 136, 256, 512) if G * x <= 4096])
    bs = rng.choice([1, 8, 16, 32])
    N = rng.randint(1, 10)
    op_blocks = rng.randint(1, max(1, 1024 // bs))
    own_blocks = rng.randint(1, max(1, 128 // bs))
    op_len = [rng.randint(0, op_blocks * bs) for _ in range(N)]
    own_len = [rng.randint(0 if o else 1, own_blocks * bs) for o in op_len]   # every row reads >= 1 key
    return dict(G=G, hkv=rng.choice([1, 2, 4]), d=d, bs=bs, N=N, op_blocks=op_blocks, own_blocks=own_blocks,
                op_len=op_len, own_len=own_len, dtype=rng.choice([torch.float16, torch.bfloat16]),
                chunk=rng.choice([None, 64, 128, 512]), seed=110 + i)


@pytest.mark.parametrize("i", range(16))
def test_decode_reader_random_layouts(dev, i):
    """Op B (DecodeReader's joint read over paged operator + own pools) on seeded random layouts
    against the oracle's decode_read_ref: relative error < 2e-3 (the reference test's bar,
    tests/test_d23_kernels.py:51-82 of the reference)."""
    from kv_skill_v2_amd.decode_reader import DecodeReader

    c = _decode_reader_case(i)
    say("op B", i, {k: (str(v) if k == "dtype" else v) for k, v in c.items()})
    g = torch.Generator().manual_seed(c["seed"])
    hkv, d, bs, N, dt = c["hkv"], c["d"], c["bs"], c["N"], c["dtype"]
    hq = c["G"] * hkv
    nb_op, nb_own = c["op_blocks"] + 3, c["own_blocks"] * N + 2
    op_k, op_v = (torch.randn(nb_op, bs, hkv, d, generator=g).to(dt) for _ in range(2))
    own_k, own_v = (torch.randn(nb_own, bs, hkv, d, generator=g).to(dt) for _ in range(2))
    q = torch.randn(N, hq, d, generator=g).to(dt)
    op_bt = torch.stack([torch.randperm(nb_op, generator=g)[:c["op_blocks"]] for _ in range(N)]).int()
    own_bt = torch.stack([torch.randperm(nb_own, generator=g)[:c["own_blocks"]] for _ in range(N)]).int()
    op_len = torch.tensor(c["op_len"], dtype=torch.int32)
    own_len = torch.tensor(c["own_len"], dtype=torch.int32)
    args = [q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len]
    max_keys = max(1, int((op_len + own_len).max()))
    dec = DecodeReader(N, hq, hkv, d, max_keys=max_keys, device=dev, chunk=c["chunk"])
    out = dec(*[a.to(dev) for a in args], d ** -0.5).double().cpu()
    ref = O.decode_read_ref(*args, d ** -0.5).double()
    rel = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
    assert rel < 2e-3, rel
