"""GPU: the LayerSelector kernels and the epilogue row scale against the oracle:
xenc_selector_weights vs selector_weights (xenc/selector.py:59-67; kept indices bit-exact incl.
ties, weights to 1e-6), xenc_selector_apply vs selector_apply (xenc/selector.py:106-110) for one
layer and summed over a token's selected layers, xenc_gate_scale vs the epilogue's gate * gain
(xenc/injector.py:59-69, 266-267), and the guards."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("B,n,k,ties", [(37, 8, 2, False), (5, 200, 5, False), (64, 8, 2, True),
                                        (9, 36, 1, True), (4, 256, 64, True)])
def test_selector_weights(dev, B, n, k, ties):
    say("selector weights", dict(B=B, n=n, k=k, ties=ties))
    g = torch.Generator().manual_seed(B * n + k)
    z = (torch.randint(-3, 4, (B, n), generator=g).float() if ties else torch.randn(B, n, generator=g))
    w, idx, w_sel = ops.selector_weights(z.to(dev), k)
    ref = O.selector_weights(z.double(), k)
    order = O.topk_order(z, k)
    assert torch.equal(idx.cpu().long(), order)
    assert float((w.cpu().double() - ref).abs().max()) < 1e-6
    assert float((w_sel.cpu().double() - ref.gather(1, order)).abs().max()) < 1e-6
    assert int((w.cpu() != 0).sum(1).min()) == k


def test_selector_weights_non_finite_logits(dev):
    """NaN, +inf and -inf logits: every kept index lies in [0, n) and the order is the oracle's
    (NaN ranks above +inf as torch.sort / topk rank it, ties to the lower index); rows of all
    NaN or all -inf included.  The weights of a row with a kept NaN are NaN, as the softmax of
    the reference gives."""
    say("selector weights, non-finite logits")
    nan, inf = float("nan"), float("inf")
    z = torch.randn(6, 8, generator=torch.Generator().manual_seed(4))
    z[0, 3] = nan
    z[1] = nan
    z[2] = -inf
    z[3, 5], z[3, 1] = inf, inf
    z[4, :4] = nan
    z[4, 6] = -inf
    z[5, 7] = -inf
    for k in (1, 2, 5, 8):
        w, idx, w_sel = ops.selector_weights(z.to(dev), k)
        idx = idx.cpu().long()
        assert int(idx.min()) >= 0 and int(idx.max()) < 8
        assert torch.equal(idx, O.topk_order(z, k)), k
        finite_rows = [r for r in range(6) if torch.isfinite(z[r].gather(0, idx[r])).all()]
        ref = O.selector_weights(z.double(), k)
        for r in finite_rows:
            assert float((w[r].cpu().double() - ref[r]).abs().max()) < 1e-6


def test_selector_apply_one_and_summed(dev):
    say("selector apply")
    g = torch.Generator().manual_seed(3)
    B, d, k = 32, 5120, 2
    h = torch.randn(B, d, generator=g)
    delta = torch.randn(B * k, d, generator=g) * 0.01
    w = torch.rand(B * k, generator=g)
    la = -3.9
    out1 = ops.selector_apply(delta[::2].contiguous().to(dev), h.to(dev), w[::2].contiguous().to(dev), la, k=1)
    ref1 = O.selector_apply(delta[::2].double(), h.double(), w[::2].double(), la)
    assert float((out1.cpu().double() - ref1).abs().max()) < 1e-6 * float(ref1.abs().max()) + 1e-9
    out2 = ops.selector_apply(delta.to(dev), h.to(dev), w.to(dev), la, k=k)
    ref2 = sum(O.selector_apply(delta[j::k].double(), h.double(), w[j::k].double(), la) for j in range(k))
    assert float((out2.cpu().double() - ref2).abs().max()) < 1e-6 * float(ref2.abs().max()) + 1e-9
    # the matched norm, closed form: with one layer and w = 1,
    # ||out|| / ||h|| = alpha * rel / (rel + 1e-6) * (||h|| + 1e-6) / ||h||, rel = ||delta|| / (||h|| + 1e-6)
    one = ops.selector_apply(delta[:B].contiguous().to(dev), h.to(dev), torch.ones(B, device=dev), la, k=1)
    hn_, dn_ = h.double().norm(dim=-1), delta[:B].double().norm(dim=-1)
    rel = dn_ / (hn_ + 1e-6)
    want = torch.tensor(la, dtype=torch.float64).exp() * rel / (rel + 1e-6) * (hn_ + 1e-6) / hn_
    ratio = one.cpu().double().norm(dim=-1) / hn_
    assert torch.allclose(ratio, want, rtol=1e-5)


def test_gate_scale_matches_epilogue(dev):
    say("gate scale")
    g = torch.Generator().manual_seed(5)
    T, d, n_pos = 20, 5120, 8
    hn = O.rms_norm(torch.randn(T, d, generator=g))
    gate_w = torch.randn(d, generator=g) / 50
    gate_b = torch.randn(n_pos, generator=g)
    log_gain = torch.randn(n_pos, generator=g) * 0.2
    row_token = torch.tensor([3, 3, 0, 19, 7, 7, 7])
    row_pos = torch.tensor([0, 5, 2, 7, 1, 3, 6])
    s = ops.gate_scale(hn.to(dev), gate_w.to(dev), gate_b.to(dev), log_gain.to(dev), 0.5,
                       row_token.to(dev), row_pos.to(dev))
    hd = hn.double()
    ref = torch.stack([0.5 * torch.exp(log_gain[p].double()) * torch.sigmoid(hd[t] @ gate_w.double() + gate_b[p].double())
                       for t, p in zip(row_token.tolist(), row_pos.tolist())])
    assert float((s.cpu().double() - ref).abs().max()) < 1e-6
    s_all = ops.gate_scale(hn.to(dev), gate_w.to(dev), gate_b[2:3].to(dev), log_gain[2:3].to(dev), 0.5)
    ref_all = 0.5 * torch.exp(log_gain[2].double()) * torch.sigmoid(hd @ gate_w.double() + gate_b[2].double())
    assert float((s_all.cpu().double() - ref_all).abs().max()) < 1e-6
    # against the oracle epilogue itself (B = identity, d = 64): delta = scale * r
    d2 = 64
    hn2 = O.rms_norm(torch.randn(T, d2, generator=g)).double()
    r2 = torch.randn(T, d2, generator=g).double()
    gw2 = torch.randn(d2, generator=g).double() / 8
    ep = O.epilogue(hn2, r2, torch.eye(d2, dtype=torch.float64), None, gw2, gate_b[4].double(),
                    log_gain[4].double(), 0.7)
    s2 = ops.gate_scale(hn2.float().to(dev), gw2.float().to(dev), gate_b[4:5].to(dev), log_gain[4:5].to(dev), 0.7)
    assert float((s2.cpu().double().unsqueeze(-1) * r2 - ep).abs().max()) < 1e-5


@pytest.mark.parametrize("B,L,k,d,d_r,ties,vec4", [(32, 8, 2, 2560, 5120, False, True),
                                                   (7, 8, 3, 36, 20, True, True),
                                                   (5, 12, 2, 30, 18, False, False)])
def test_multi_depth_prepare_equals_separate_calls(dev, B, L, k, d, d_r, ties, vec4):
    """xenc_multi_depth_prepare: the selector outputs, the gathered query rows and the row scales
    equal xenc_selector_weights, q_all[top, token] and xenc_gate_scale bit for bit (also with
    tied logits, a strided q_all and rows whose sizes force the scalar copy / dot)."""
    say("multi-depth prepare", dict(B=B, L=L, k=k, d=d, d_r=d_r, ties=ties, vec4=vec4))
    g = torch.Generator().manual_seed(B * L + d)
    z = (torch.randint(-2, 3, (B, L), generator=g).float() if ties else torch.randn(B, L, generator=g)).to(dev)
    q_big = torch.randn(L, B, d + (0 if vec4 else 3), generator=g).to(dev)
    q_all = q_big[:, :, :d]                       # strided over tokens and depths when padded
    hn = torch.randn(B, d_r, generator=g).to(dev)
    gate_w = (torch.randn(d_r, generator=g) / d_r ** 0.5).to(dev)
    gate_b = torch.randn(L, generator=g).to(dev)
    log_gain = (0.1 * torch.randn(L, generator=g)).to(dev)
    w, top, wtop, q_rows, scale = ops.multi_depth_prepare(z, k, q_all, hn, gate_w, gate_b, log_gain, 0.7)
    w2, top2, wtop2 = ops.selector_weights(z, k)
    assert torch.equal(w, w2) and torch.equal(top, top2) and torch.equal(wtop, wtop2)
    depth = top.reshape(-1).long()
    token = torch.arange(B, device=dev).repeat_interleave(k)
    assert torch.equal(q_rows, q_all[depth, token])
    scale2 = ops.gate_scale(hn, gate_w, gate_b, log_gain, 0.7, token.int(), depth.int())
    assert torch.equal(scale, scale2)
    with pytest.raises(ValueError):
        ops.multi_depth_prepare(z, k, q_all, hn, gate_w, gate_b[:-1], log_gain, 0.7)


@pytest.mark.parametrize("B,chunks,k,top_k,d,ties", [(32, [64] * 8, 2, 8, 2560, False),
                                                     (7, [5, 33, 64, 1, 12], 3, 4, 264, True),
                                                     (3, [9, 17, 2, 40], 1, 0, 64, False),
                                                     (12, [64, 30, 7], 2, 64, 520, True)])
def test_multi_depth_prepare_route_equals_separate_calls(dev, B, chunks, k, top_k, d, ties):
    """xenc_multi_depth_prepare_route: every output equals xenc_multi_depth_prepare followed by
    xenc_route_topk of its q_rows (the depth of each row as its library) bit for bit: the dots
    of the fused launch take each row's depth from their own rank count of the logits, so tied
    logits, unequal libraries, dense routing (top_k 0 or >= the chunks) and d not a multiple of
    256 are the cases where that could part from the selection kernel."""
    L = len(chunks)
    say("multi-depth prepare + route", dict(B=B, chunks=chunks, k=k, top_k=top_k, d=d, ties=ties))
    P = synth.pool(chunks, 64, d, device=dev)
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    g = torch.Generator().manual_seed(B * L + d + k)
    z = (torch.randint(-1, 2, (B, L), generator=g).float() if ties else torch.randn(B, L, generator=g)).to(dev)
    q_all = torch.randn(L, B, d, generator=g).to(dev)
    d_r = 48
    hn = torch.randn(B, d_r, generator=g).to(dev)
    gate_w = (torch.randn(d_r, generator=g) / d_r ** 0.5).to(dev)
    gate_b = torch.randn(L, generator=g).to(dev)
    log_gain = (0.1 * torch.randn(L, generator=g)).to(dev)
    got = ops.multi_depth_prepare_route(z, k, q_all, hn, gate_w, gate_b, log_gain, lib, top_k=top_k,
                                        route_temp=10.0, gain_scale=0.7)
    w, top, wtop, q_rows, scale = ops.multi_depth_prepare(z, k, q_all, hn, gate_w, gate_b, log_gain, 0.7)
    wr, idx, wsel = ops.route_topk(q_rows, lib, top.reshape(-1), top_k=top_k, route_temp=10.0)
    for a, b, name in zip(got, (w, top, wtop, q_rows, scale, wr, idx, wsel),
                          ("w", "top", "wtop", "q_rows", "scale", "w_route", "idx", "w_sel")):
        assert a.shape == b.shape and torch.equal(a, b), name
    with pytest.raises(ValueError):
        ops.multi_depth_prepare_route(z, k, q_all[:, :, :-8], hn, gate_w, gate_b, log_gain, lib)


def test_selector_guards(dev):
    say("selector guards")
    with pytest.raises(ValueError):
        ops.selector_weights(torch.randn(2, 300, device=dev), 2)      # n > 256
    with pytest.raises(ValueError):
        ops.selector_weights(torch.randn(2, 4, device=dev), 5)        # k > n
    with pytest.raises(ValueError):
        ops.selector_apply(torch.randn(3, 8, device=dev), torch.randn(2, 8, device=dev),
                           torch.ones(4, device=dev), 0.0, k=2)
