"""GPU: the drop-in injectors (LibraryInjector / XEncInjector) on a small reader, through the HIP
route / read kernels, against a CPU fp64 re-run of the same forward through the oracle.
Mirrors tests/test_library.py, tests/test_d6_force_attn.py, tests/test_attn_harvest.py:129-168 and
the selector hook tests of the reference.  Pages are fp16, so outputs meet the fp16 bar
(relative 1e-2 on the norm, max-abs 2e-3 of the output scale); the reference's 1e-5 checks
between two fp32 torch paths become checks between the HIP path and the fp64 oracle."""

from __future__ import annotations

import pytest
import torch

import kv_skill_v2_amd.injector as xi
from kv_skill_v2_amd import ops
from kv_skill_v2_amd.depth import DEPTHS, for_reader, injection_layers
from kv_skill_v2_amd.injector import LibraryInjector, XEncInjector, itf_gain, itf_gate, itf_write, rms_norm
from kv_skill_v2_amd.interface import ModelInterface
from kv_skill_v2_amd.library import Library
from kv_skill_v2_amd.selector import LayerSelector
from tiny import TinyLM, close, oracle_forward, randomize, skill_rho, x_in

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _setup(d=32, d_s=24, ns=(5, 9, 3), seed_itf=3, dev="cuda"):
    reader = TinyLM(d=d, n_layers=8).to(dev)
    layers = injection_layers(reader, DEPTHS)
    itf = ModelInterface(d, d_s, layers).to(dev)
    randomize(itf, seed=seed_itf)
    skills = [skill_rho(d_s, DEPTHS, n=n, seed=i) for i, n in enumerate(ns)]
    lib = Library(skills, layers, DEPTHS)
    return reader, layers, itf, skills, lib


def _tensors(lib):
    return {li: (lib.K[li].cpu(), lib.mask[li].cpu(), lib.S[li].cpu(),
                 None if lib.V is None else lib.V[li].cpu()) for li in lib.layers}


def test_noop_at_init_and_guards(dev):
    say("noop + guards")
    reader = TinyLM(d=40, n_layers=8).to(dev)
    layers = injection_layers(reader, DEPTHS)
    itf = ModelInterface(40, 24, layers).to(dev)
    x = x_in(40).to(dev)
    with torch.no_grad():
        bare = reader(x)
    inj = XEncInjector(reader, itf)
    inj.load(skill_rho(24, DEPTHS))
    assert sorted(inj.skill.K) == layers
    with torch.no_grad():
        assert torch.equal(reader(x), bare), "zero-init B must be a no-op"
    assert len(inj.mag_terms) == len(layers) and all(float(m) == 0 for m in inj.mag_terms)
    with pytest.raises(ValueError):
        inj.load(skill_rho(32, DEPTHS))
    s = for_reader(skill_rho(24, DEPTHS), reader)
    s.K.pop(layers[-1])
    with pytest.raises(KeyError):
        inj.load(s)
    inj.detach()
    lib = Library([skill_rho(24, DEPTHS, n=n, seed=n) for n in (5, 9, 3)], layers, DEPTHS)
    linj = LibraryInjector(reader, itf)
    linj.load_library(lib)
    with torch.no_grad():
        assert torch.equal(reader(x), bare)
    with pytest.raises(ValueError):
        linj.load_library(Library([skill_rho(16, DEPTHS)], layers, DEPTHS))
    lib2 = Library([skill_rho(24, DEPTHS)], layers[:3] + [5], DEPTHS)
    with pytest.raises(KeyError):
        linj.load_library(lib2)
    linj.detach()


@pytest.mark.parametrize("read_softmax", [True, False])
@pytest.mark.parametrize("top_k", [0, 2])
@pytest.mark.parametrize("T", [1, 7, 40])
def test_library_forward_matches_oracle(dev, read_softmax, top_k, T):
    """T=1 and T=7 (B=2: 2 and 14 rows) take the split-K decode path, T=40 the MFMA path."""
    say("library fwd", dict(read_softmax=read_softmax, top_k=top_k, T=T))
    reader, layers, itf, skills, lib = _setup(ns=(5, 9, 3, 12))
    x = x_in(32, T=T).to(dev)
    inj = LibraryInjector(reader, itf, read_softmax=read_softmax, top_k=top_k)
    inj.load_library(lib)
    with torch.no_grad():
        out = reader(x)
        bare_inj = inj.mag_terms[-1]
    ref, _ = oracle_forward(reader, x, itf, _tensors(lib), top_k=top_k, read_softmax=read_softmax)
    ok, err, rn = close(out, ref)
    assert ok, (err, rn)
    assert float(bare_inj) > 0
    inj.detach()


def test_one_chunk_equals_single_skill(dev):
    """A one-chunk Library reads exactly what the single-skill injector reads (tests/test_library.py:91-123)."""
    say("one chunk == single skill")
    reader = TinyLM(d=32, n_layers=8).to(dev)
    layers = injection_layers(reader, DEPTHS)
    skill = skill_rho(32, DEPTHS, n=11, seed=4)
    x = x_in(32).to(dev)
    for read_softmax in (False, True):
        itf = ModelInterface(32, 32, layers).to(dev)
        randomize(itf, seed=7)
        ext = XEncInjector(reader, itf, read_softmax=read_softmax)
        ext.load(skill)
        with torch.no_grad():
            ref = reader(x)
        ext.detach()
        lib_inj = LibraryInjector(reader, itf, read_softmax=read_softmax)
        lib_inj.load_library(Library([skill], layers, DEPTHS))
        with torch.no_grad():
            out = reader(x)
        lib_inj.detach()
        with torch.no_grad():
            bare = reader(x)
        assert (ref - bare).abs().max() > 1e-3
        assert (out - ref).abs().max().item() < 1e-5, read_softmax
        for a, b in zip(ext.mag_terms, lib_inj.mag_terms):
            assert abs(float(a) - float(b)) < 1e-5
        lib1 = Library([skill], layers, DEPTHS)
        oref, _ = oracle_forward(reader, x, itf, _tensors(lib1), read_softmax=read_softmax)
        ok, err, rn = close(out, oref)
        assert ok, (read_softmax, err, rn)


def test_routing_topk_bookkeeping(dev):
    say("route_terms / last_route")
    reader, layers, itf, skills, _ = _setup(ns=(4, 5, 6, 7, 8), seed_itf=3)
    lib = Library([skill_rho(24, DEPTHS, n=4 + i, seed=i) for i in range(5)], layers, DEPTHS)
    assert lib.n_chunks == 5 and lib.K[layers[0]].shape == (5, 8, 24)
    for top_k in (0, 2):
        inj = LibraryInjector(reader, itf, top_k=top_k)
        inj.load_library(lib)
        reader(x_in(32).to(dev))                 # grad enabled -> route_terms recorded
        assert len(inj.route_terms) == len(layers)
        for li, w in inj.route_terms:
            assert w.shape == (2, 7, 5)
            assert torch.allclose(w.sum(-1), torch.ones(2, 7, device=dev), atol=1e-6)
            assert bool(((w > 0).sum(-1) == (2 if top_k else 5)).all())
            assert w.requires_grad
        assert torch.equal(inj.last_route, inj.route_terms[-1][1].detach())
        inj.unload()
        assert not inj.route_terms and not inj.mag_terms and inj.last_route is None
        inj.detach()


@pytest.mark.parametrize("top_k", [0, 2])
def test_training_gradients_match_oracle(dev, top_k):
    """Interface gradients (A through the MFMA read's dQ and the route backward; B, gate, gain)
    vs autograd on the oracle forward in fp64."""
    say("training grads", dict(top_k=top_k))
    reader, layers, itf, skills, lib = _setup(ns=(20, 64, 33), seed_itf=5)
    x = x_in(32, T=9).to(dev)
    g_up = torch.randn(2, 9, 32, generator=torch.Generator().manual_seed(7))
    itf.zero_grad()
    inj = LibraryInjector(reader, itf, top_k=top_k)
    inj.load_library(lib)
    out = reader(x)
    (out * g_up.to(dev)).sum().backward()
    inj.detach()
    ref_out, (it, _) = oracle_forward(reader, x, itf, _tensors(lib), top_k=top_k, grad=True)
    assert close(out, ref_out)[0]
    (ref_out * g_up.double()).sum().backward()
    ours, theirs = dict(itf.named_parameters()), dict(it.named_parameters())
    for name in ("A.weight", "B.weight", "gate_w", "gate_b", "log_gain"):
        ok, err, rn = close(ours[name].grad, theirs[name].grad)      # rel 1e-2, max-abs 2e-3
        print(f"[grad] top_k={top_k} {name}: max-abs {err:.3g} rel {rn:.3g}", flush=True)
        assert ok, (top_k, name, err, rn)


def test_route_terms_backward(dev):
    """A loss on route_terms reaches the query map through the route backward kernel."""
    say("route_terms backward")
    reader, layers, itf, skills, lib = _setup(ns=(20, 64, 33), seed_itf=5)
    inj = LibraryInjector(reader, itf, top_k=2)
    inj.load_library(lib)
    reader(x_in(32, T=9).to(dev))
    itf.zero_grad()
    sum((w * w).sum() for _, w in inj.route_terms).backward()
    g = itf.A.weight.grad
    assert g is not None and torch.isfinite(g).all() and g.abs().sum() > 0
    inj.detach()


def test_untied_values_match_oracle(dev):
    """An untied Library reads its values (tests/test_attn_harvest.py:129-149)."""
    say("untied values")
    reader, layers, itf, skills, _ = _setup(ns=(6, 9, 4))
    g = torch.Generator().manual_seed(11)
    for s in skills:
        s.V = {r: torch.nn.functional.normalize(torch.randn(k.shape, generator=g), dim=-1) for r, k in s.K.items()}
    lib = Library(skills, layers, DEPTHS)
    assert lib.V is not None
    x = x_in(32).to(dev)
    inj = LibraryInjector(reader, itf)
    inj.load_library(lib)
    with torch.no_grad():
        out = reader(x)
    inj.detach()
    ref, _ = oracle_forward(reader, x, itf, _tensors(lib))
    ok, err, rn = close(out, ref)
    assert ok, (err, rn)
    tied, _ = oracle_forward(reader, x, itf, {li: t[:3] for li, t in _tensors(lib).items()})
    assert (tied.cuda() - out).abs().max() > 1e-3, "values must change the read"


def test_force_attn(dev):
    """tests/test_d6_force_attn.py:37-105: None is the identity, a one-hot map reads that slot,
    the per-layer dict form, the shape guard, and norm matching."""
    say("force_attn")
    reader, layers, itf, skills, lib = _setup(ns=(5, 9, 3))
    x = x_in(32).to(dev)
    inj = LibraryInjector(reader, itf)
    inj.load_library(lib)
    with torch.no_grad():
        a = reader(x)
        inj.force_attn = None
        assert torch.equal(a, reader(x))
    li = layers[1]
    C, N = lib.mask[li].shape
    fa = torch.zeros(C, N)
    fa[1, 4] = 1.0
    inj.force_attn = fa
    h = torch.randn(2, 7, 32, generator=torch.Generator().manual_seed(3)).to(dev)
    with torch.no_grad():
        d = inj._branch(h, li)
        hn = rms_norm(h.float())
        ref = itf_gain(itf, li, hn) * itf_gate(itf, hn, li) * itf_write(itf, lib.K[li][1, 4].expand(2, 7, -1))
    assert (d - ref).abs().max() < 1e-5
    inj.force_attn = {l: torch.zeros(lib.mask[l].shape) for l in layers}
    with torch.no_grad():
        assert inj._branch(h, li).abs().max() == 0
    inj.force_attn = torch.zeros(C, N + 1)
    with pytest.raises(ValueError):
        inj._branch(h, li)
    li = layers[0]
    h = torch.randn(1, 5, 32, generator=torch.Generator().manual_seed(9)).to(dev)
    M = lib.mask[li]
    fa = torch.zeros(M.shape)
    fa[0, :2] = 0.5
    captured = []
    orig = xi.write_delta
    xi.write_delta = lambda itf_, hn_, r, *a, **k: (captured.append(r), orig(itf_, hn_, r, *a, **k))[1]
    try:
        with torch.no_grad():
            inj.force_attn, inj.force_norm_match = fa, True
            inj._branch(h, li)
            inj.force_attn = None
            inj._branch(h, li)
    finally:
        xi.write_delta = orig
    r_forced, r_comp = captured
    assert torch.allclose(r_forced.norm(dim=-1), r_comp.norm(dim=-1), atol=1e-4)
    inj.detach()


def test_record_and_training_attn(dev):
    say("record_attn / training_attn")
    reader, layers, itf, skills, lib = _setup(ns=(5, 9, 3))
    x = x_in(32).to(dev)
    inj = LibraryInjector(reader, itf, top_k=2)
    inj.load_library(lib)
    inj.record_attn = True
    with torch.no_grad():
        reader(x)
    assert sorted(inj.last_attn) == layers
    for li in layers:
        la = inj.last_attn[li]
        C, N = lib.mask[li].shape
        assert la.shape == (C, N) and la.device.type == "cpu"
        assert abs(float(la.sum()) - 1.0) < 1e-5 and float(la[~lib.mask[li].cpu()].abs().max()) == 0
    inj.record_attn = False
    inj.training_attn, inj.attn_pos = True, 3
    reader(x)
    assert len(inj.attn_terms) == len(layers) and all(t.requires_grad for t in inj.attn_terms)
    sum(t.sum() for t in inj.attn_terms).backward()
    assert itf.A.weight.grad is not None
    inj.detach()


class _CountingSelector:
    def __init__(self):
        self.resets, self.applied = 0, []

    def reset(self):
        self.resets += 1

    def apply(self, delta, h, li):
        self.applied.append(li)
        return 0.5 * delta


def test_selector_hooks(dev):
    say("selector hooks")
    reader, layers, itf, skills, lib = _setup(d_s=32, ns=(6, 6, 6), seed_itf=2)
    x = x_in(32).to(dev)
    base = LibraryInjector(reader, itf)
    base.load_library(lib)
    with torch.no_grad():
        full = reader(x)
    base.detach()
    sel = _CountingSelector()
    inj = LibraryInjector(reader, itf, selector=sel)
    inj.load_library(lib)
    with torch.no_grad():
        reader(x)
        reader(x)
        halved = reader(x)
    assert sel.resets == 3 and sel.applied == layers * 3
    assert (halved - full).abs().max() > 1e-4
    inj.detach()


@pytest.mark.parametrize("T", [1, 24])
def test_layer_selector_matches_oracle(dev, T):
    """A real LayerSelector over the injection layers: the injector reads only the rows that
    select a layer; the output equals the oracle forward that reads every row."""
    say("layer selector", dict(T=T))
    reader, layers, itf, skills, lib = _setup(ns=(7, 12, 30), seed_itf=4)
    torch.manual_seed(1)
    sel = LayerSelector(32, layers, k=2, alpha_init=0.05).to(dev)
    randomize(sel, seed=12, scale=1.0)
    x = x_in(32, T=T, B=3).to(dev)
    inj = LibraryInjector(reader, itf, selector=sel, top_k=2)
    inj.load_library(lib)
    with torch.no_grad():
        out = reader(x)
    inj.detach()
    ref, _ = oracle_forward(reader, x, itf, _tensors(lib), top_k=2, selector=sel)
    ok, err, rn = close(out, ref)
    assert ok, (err, rn)


def test_selector_decode_step_graph_replay(dev):
    """A T = 1 decode forward with a LayerSelector (selector weights, routed read of the selected
    rows only, fused write-back, matched-norm apply) has no host synchronisation: it captures in
    one HIP graph, and every replay with new input rows equals the eager forward bit for bit and
    the fp64 oracle forward within the fp16 bar."""
    say("selector decode step in a HIP graph")
    reader, layers, itf, skills, lib = _setup(ns=(7, 12, 30), seed_itf=4)
    torch.manual_seed(1)
    sel = LayerSelector(32, layers, k=2, alpha_init=0.05).to(dev)
    randomize(sel, seed=12, scale=1.0)
    inj = LibraryInjector(reader, itf, selector=sel, top_k=2)
    inj.load_library(lib)
    x_static = x_in(32, T=1, B=3, seed=20).to(dev)
    with torch.no_grad():
        reader(x_static)                              # pools built, workspaces allocated
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            reader(x_static)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_graph = reader(x_static)
        for seed in (21, 22, 23):
            x_new = x_in(32, T=1, B=3, seed=seed).to(dev)
            x_static.copy_(x_new)
            graph.replay()
            torch.cuda.synchronize()
            eager = reader(x_new.clone())
            torch.cuda.synchronize()
            assert torch.equal(y_graph, eager), seed
            ref, _ = oracle_forward(reader, x_new, itf, _tensors(lib), top_k=2, selector=sel)
            ok, err, rn = close(y_graph, ref)
            assert ok, (seed, err, rn)
    inj.detach()


def test_unload_restores_bare(dev):
    say("unload")
    reader, layers, itf, skills, lib = _setup()
    x = x_in(32).to(dev)
    with torch.no_grad():
        bare = reader(x)
    inj = LibraryInjector(reader, itf, top_k=2)
    inj.load_library(lib)
    with torch.no_grad():
        y = reader(x)
    assert torch.isfinite(y).all() and (y - bare).abs().max() > 1e-4
    inj.unload()
    with torch.no_grad():
        assert torch.equal(reader(x), bare)
    inj.detach()


def test_branch_read_dispatch_agrees(dev):
    """The decode and MFMA paths give the same read for the same rows (fp16 bar)."""
    say("dispatch agreement")
    _, layers, _, skills, lib = _setup(ns=(40, 512, 129))
    pl = lib.paged(layers[0], dev)
    q = torch.nn.functional.normalize(torch.randn(8, 24, generator=torch.Generator().manual_seed(4)), dim=-1).to(dev)
    for soft in (True, False):
        with torch.no_grad():
            r_dec, w_dec = ops.branch_read(q, pl, 2, read_softmax=soft)
        qg = q.clone().requires_grad_(True)
        r_mfma, w_mfma = ops.branch_read(qg, pl, 2, read_softmax=soft)
        assert torch.equal(w_dec, w_mfma.detach())
        ok, err, rn = close(r_dec, r_mfma, rel=5e-3)
        assert ok, (soft, err, rn)
