"""GPU: D8 slot top-k selection read (xenc/topk_read.py) on the HIP kernels, against the oracle and
the reference's own checks (tests/test_topk_read.py):
  kernels   select_scores vs the fp64 oracle; top-k bit-exact vs a stable sort (ties to the lower
            index) incl. heavy ties, -inf and k up to 1024 of 100k; gathered pages == the slots;
  (a)       selection == a hand computation on a transformers Llama reader (the bare reader's
            queries at the selection layer, GQA max over heads, top-k over valid slots);
  (b)       k >= valid slots: exactly LibraryInjector; the restricted read over ALL slots of one
            chunk == the standard one-chunk read; no-op at init (B = 0);
  (c)       the layer update == the oracle's topk_read + epilogue, decode and prefill paths, and
            the interface gradient of a training step matches the fp64 oracle's;
  (d)       decode reuse: one selection pass for a generate() call with the KV cache."""

from __future__ import annotations

import copy

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import ops
from kv_skill_v2_amd.depth import DEPTHS, decoder_layers, injection_layers
from kv_skill_v2_amd.injector import LibraryInjector
from kv_skill_v2_amd.interface import ModelInterface
from kv_skill_v2_amd.library import Library
from kv_skill_v2_amd.topk_read import (TopKLibraryInjector, TopKSelector, attach_sel_keys, reader_queries,
                                       sel_layer_for)
from tiny import close, randomize, skill_rho

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")

D_R, D_S, NKV, HD = 64, 32, 2, 16


def say(*a):
    print("[case]", *a, flush=True)


def _reader(dev):
    cfg = transformers.LlamaConfig(vocab_size=128, hidden_size=D_R, intermediate_size=128, num_hidden_layers=8,
                                   num_attention_heads=4, num_key_value_heads=NKV, max_position_embeddings=256)
    torch.manual_seed(0)
    return transformers.LlamaForCausalLM(cfg).to(dev).float()


def _lib(layers, ns=(16, 16, 9), seed=0):
    skills = [skill_rho(D_S, DEPTHS, n=n, seed=seed + i) for i, n in enumerate(ns)]
    lib = Library(skills, layers, DEPTHS)
    g = torch.Generator().manual_seed(seed + 100)
    ac = {"chunks": [{"K": {0.5: torch.randn(n, NKV * HD, generator=g)}} for n in ns]}
    return attach_sel_keys(lib, ac, 0.5)


def _itf(layers, dev, zero_B=False):
    itf = ModelInterface(D_R, D_S, layers).to(dev)
    randomize(itf, seed=21, scale=0.3)
    if zero_B:
        with torch.no_grad():
            itf.B.weight.zero_()
    return itf


# ------------------------------------------------------------------ kernels
def test_select_scores_and_topk_kernels(dev):
    say("D8 kernels")
    g = torch.Generator().manual_seed(1)
    B, n_q, n_kv, hd, S = 3, 8, 2, 64, 5000
    q = torch.randn(B, n_q, hd, generator=g)
    keys = torch.randn(S, n_kv, hd, generator=g)
    valid = torch.rand(S, generator=g) > 0.1
    for pool in ("max", "mean"):
        s = ops.select_scores(q.to(dev), keys.to(dev), valid.to(dev), pool).cpu()
        ref = O.select_scores(q.double(), keys.double(), valid, pool)
        fin = torch.isfinite(ref)
        assert torch.equal(torch.isfinite(s), fin)
        assert float((s[fin].double() - ref[fin]).abs().max()) < 1e-4
    # top-k: exact against a stable descending sort, with heavy ties and -inf
    for S2, k, seed in ((1000, 7, 2), (100_000, 1024, 3), (4096, 1, 4), (300, 300, 5), (50_000, 333, 6)):
        gg = torch.Generator().manual_seed(seed)
        sc = torch.randint(-20, 20, (4, S2), generator=gg).float() / 4      # many ties
        sc[:, ::17] = float("-inf")
        sc[1] = torch.randn(S2, generator=gg)
        idx, vals = ops.topk_rows(sc.to(dev), k)
        want = O.topk_order(sc, k)
        assert torch.equal(idx.cpu().long(), want), (S2, k)
        assert torch.equal(vals.cpu(), sc.gather(-1, want))


def test_gather_library_pages(dev):
    say("D8 gather")
    layers = [2, 4, 6, 7]
    lib = _lib(layers)
    pl = lib.paged(layers[1], dev)
    N = lib.mask[layers[1]].shape[1]
    idx = torch.tensor([[17, 0, 40, 3, 31], [5, 6, 7, 8, 9]], device=dev)
    sel = ops.gather_library(pl, idx, N)
    K = lib.K[layers[1]].reshape(-1, D_S)
    for g_ in range(2):
        for j, f in enumerate(idx[g_].tolist()):
            assert torch.equal(sel.pages[g_, j, :D_S].float().cpu(), K[f].half().float().cpu())
        assert float(sel.pages[g_, 5:].abs().max()) == 0.0
    assert sel.n_chunks == [1, 1] and sel.nvalid == [5, 5] and sel.slots_per_page == 64


# ------------------------------------------------------------------ (a) selection
def _sel_input(reader, sel_layer, ids):
    got = {}
    att = decoder_layers(reader)[sel_layer].self_attn

    def cap(mod, args, kwargs):
        got.setdefault("x", (kwargs["hidden_states"] if "hidden_states" in kwargs else args[0]).detach().clone())

    h = att.register_forward_pre_hook(cap, with_kwargs=True)
    with torch.no_grad():
        reader(ids)
    h.remove()
    return got["x"]


def test_selection_matches_hand_computation(dev):
    say("D8 (a) selection")
    reader = _reader(dev)
    layers = injection_layers(reader, DEPTHS)
    sel_layer = sel_layer_for(reader, 0.5)
    lib = _lib(layers)
    inj = TopKLibraryInjector(reader, _itf(layers, dev), TopKSelector(reader, sel_layer, k=7), read_temp=12.0)
    inj.load_library(lib)
    ids = torch.randint(0, 128, (2, 13), generator=torch.Generator().manual_seed(3)).to(dev)
    with torch.no_grad():
        reader(ids)
    idx = inj.last_idx
    assert idx.shape == (2, 7) and inj.n_select_passes == 1
    valid = lib.mask[layers[0]].reshape(-1).cpu()
    assert valid[idx.cpu()].all()
    inj.enabled = False                          # the bare reader's selection-layer input
    x = _sel_input(reader, sel_layer, ids)
    inj.enabled = True
    with torch.no_grad():
        q = reader_queries(decoder_layers(reader)[sel_layer].self_attn, x, inj.tk.geo)[:, :, -1]
    s = O.select_scores(q.double().cpu(), lib.sel_K.reshape(-1, NKV, HD).double().cpu(), valid)
    srt = torch.sort(s, dim=-1, descending=True, stable=True).values
    assert float((srt[:, 6] - srt[:, 7]).abs().min()) > 1e-4      # no near-tie at the cut
    assert torch.equal(idx.cpu(), O.topk_order(s, 7))
    assert inj.tk.last_scores.shape == (2, 48)
    inj.record_attn = True
    with torch.no_grad():
        reader(ids)
    for li in layers:
        A = inj.last_attn[li]
        assert A.shape == (3, 16) and abs(float(A.sum()) - 1) < 1e-5
        off = torch.ones(48, dtype=torch.bool)
        off[idx[0].cpu()] = False
        assert float(A.reshape(-1)[off].abs().sum()) == 0.0
    inj.unload()
    assert inj.last_idx is None
    inj.detach()


# ------------------------------------------------------------------ (b) equivalences
def test_full_k_one_chunk_and_noop(dev):
    say("D8 (b) equivalences")
    reader = _reader(dev)
    layers = injection_layers(reader, DEPTHS)
    sel_layer = sel_layer_for(reader, 0.5)
    ids = torch.randint(0, 128, (1, 9), generator=torch.Generator().manual_seed(4)).to(dev)
    itf = _itf(layers, dev)
    ref_inj = LibraryInjector(reader, itf, read_temp=12.0)
    ref_inj.load_library(_lib(layers))
    with torch.no_grad():
        ref = reader(ids).logits
    ref_inj.detach()
    inj = TopKLibraryInjector(reader, itf, TopKSelector(reader, sel_layer, k=10_000), read_temp=12.0)
    inj.load_library(_lib(layers))
    with torch.no_grad():
        out = reader(ids).logits
    assert inj.n_select_passes == 0 and torch.equal(out, ref)
    inj.detach()

    class _Flat(TopKLibraryInjector):
        @property
        def full_read(self):
            return False

    lib1 = lambda: _lib(layers, ns=(16,), seed=7)  # noqa: E731
    ref_inj = LibraryInjector(reader, itf, read_temp=12.0)
    ref_inj.load_library(lib1())
    with torch.no_grad():
        ref1 = reader(ids).logits
    ref_inj.detach()
    flat = _Flat(reader, itf, TopKSelector(reader, sel_layer, k=16), read_temp=12.0)
    flat.load_library(lib1())
    with torch.no_grad():
        out1 = reader(ids).logits
    assert flat.n_select_passes == 1 and flat.last_idx.shape == (1, 16)
    assert torch.allclose(out1, ref1, atol=1e-4), float((out1 - ref1).abs().max())
    flat.detach()

    with torch.no_grad():
        bare = reader(ids).logits
    inj0 = TopKLibraryInjector(reader, _itf(layers, dev, zero_B=True), TopKSelector(reader, sel_layer, k=5))
    inj0.load_library(_lib(layers))
    with torch.no_grad():
        out0 = reader(ids).logits
    assert inj0.n_select_passes == 1 and torch.equal(out0, bare)
    inj0.detach()


# ------------------------------------------------------------------ (c) update vs oracle, gradients
def _oracle_delta(itf, lib, li, h, idx, read_temp=12.0):
    hn = O.rms_norm(h.double().cpu())
    A = itf.A.weight.double().cpu()
    q = O.query(hn, A, None if itf.A.bias is None else itf.A.bias.double().cpu())
    r = O.topk_read(q, lib.K[li].double().cpu(), idx.cpu(), read_temp)
    p = itf._pos[li]
    return O.epilogue(hn, r, itf.B.weight.double().cpu(), None if itf.B.bias is None else itf.B.bias.double().cpu(),
                      itf.gate_w.double().cpu(), itf.gate_b[p].double().cpu(), itf.log_gain[p].double().cpu())


@pytest.mark.parametrize("T", [1, 40])
def test_update_matches_oracle(dev, T):
    """The injected update at a layer: T = 1 (decode kernel) and T = 40 (MFMA prefill kernels)."""
    say("D8 (c) update", dict(T=T))
    reader = _reader(dev)
    layers = injection_layers(reader, DEPTHS)
    lib = _lib(layers, ns=(64, 30, 64, 5))
    itf = _itf(layers, dev)
    inj = TopKLibraryInjector(reader, itf, TopKSelector(reader, sel_layer_for(reader, 0.5), k=20))
    inj.load_library(lib)
    idx = torch.randperm(int(lib.mask[layers[0]].sum()), generator=torch.Generator().manual_seed(2))[:20]
    flat_valid = lib.mask[layers[0]].reshape(-1).nonzero().squeeze(1)
    inj.tk.last_idx = flat_valid[idx].view(1, -1).to(dev)
    h = torch.randn(2, T, D_R, generator=torch.Generator().manual_seed(6)).to(dev)
    li = layers[2]
    with torch.no_grad():
        d = inj._branch(h, li)
    ref = _oracle_delta(itf, lib, li, h, inj.tk.last_idx.expand(2, -1))
    ok, err, rn = close(d, ref)
    assert ok, (err, rn)
    inj.detach()


def test_training_gradients_match_oracle(dev):
    say("D8 (c) gradients")
    reader = _reader(dev)
    layers = injection_layers(reader, DEPTHS)
    lib = _lib(layers, ns=(64, 30, 64))
    itf = _itf(layers, dev)
    inj = TopKLibraryInjector(reader, itf, TopKSelector(reader, sel_layer_for(reader, 0.5), k=24))
    inj.load_library(lib)
    li = layers[1]
    inj.tk.last_idx = lib.mask[li].reshape(-1).nonzero().squeeze(1)[3:27].view(1, -1).to(dev)
    h = torch.randn(1, 33, D_R, generator=torch.Generator().manual_seed(8)).to(dev)
    d = inj._branch(h, li)
    (d * torch.linspace(-1, 1, D_R, device=dev)).sum().backward()
    itf64 = copy.deepcopy(itf).double().cpu()
    for p in itf64.parameters():
        p.grad = None
    hn = O.rms_norm(h.double().cpu())
    q = O.query(hn, itf64.A.weight, itf64.A.bias)
    r = O.topk_read(q, lib.K[li].double().cpu(), inj.tk.last_idx.cpu(), 12.0)
    pos = itf64._pos[li]
    ref = O.epilogue(hn, r, itf64.B.weight, itf64.B.bias, itf64.gate_w, itf64.gate_b[pos], itf64.log_gain[pos])
    (ref * torch.linspace(-1, 1, D_R, dtype=torch.float64)).sum().backward()
    for (name, p), (_, p64) in zip(itf.named_parameters(), itf64.named_parameters()):
        if p64.grad is None:
            assert p.grad is None or float(p.grad.abs().max()) == 0.0, name
            continue
        ok, err, rn = close(p.grad, p64.grad)
        assert ok, (name, err, rn)
    inj.detach()


# ------------------------------------------------------------------ (d) decode reuse
def test_generate_reuses_the_selection(dev):
    say("D8 (d) decode reuse")
    reader = _reader(dev)
    layers = injection_layers(reader, DEPTHS)
    inj = TopKLibraryInjector(reader, _itf(layers, dev), TopKSelector(reader, sel_layer_for(reader, 0.5), k=6))
    inj.load_library(_lib(layers))
    ids = torch.randint(0, 128, (1, 10), generator=torch.Generator().manual_seed(9)).to(dev)
    with torch.no_grad():
        out = reader.generate(ids, max_new_tokens=5, do_sample=False, use_cache=True, pad_token_id=0)
    assert out.shape == (1, 15)
    assert inj.n_select_passes == 1
    first = inj.last_idx.clone()
    with torch.no_grad():                      # a new prompt selects again
        reader(torch.randint(0, 128, (1, 8), generator=torch.Generator().manual_seed(10)).to(dev))
    assert inj.n_select_passes == 2 and inj.last_idx.shape == first.shape
    inj.detach()
