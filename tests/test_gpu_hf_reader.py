"""GPU: the LibraryInjector inside a real transformers reader (a randomly initialised 8-layer
Llama built from its config, no download): prompt forward against the fp64 oracle-hooked copy,
a training step whose interface gradients match the oracle's, and greedy decoding with the KV
cache (one selector reset and one update per injected layer per forward, no route_terms without
grad), then a teacher-forced forward over the generated sequence against the oracle."""

from __future__ import annotations

import pytest
import torch

from kv_skill_v2_amd.depth import DEPTHS, injection_layers
from kv_skill_v2_amd.injector import LibraryInjector
from kv_skill_v2_amd.interface import ModelInterface
from kv_skill_v2_amd.library import Library
from kv_skill_v2_amd.selector import LayerSelector
from tiny import close, oracle_forward, randomize, skill_rho

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def say(*a):
    print("[case]", *a, flush=True)


def _reader(dev):
    cfg = transformers.LlamaConfig(vocab_size=128, hidden_size=64, intermediate_size=128,
                                   num_hidden_layers=8, num_attention_heads=4, num_key_value_heads=2,
                                   max_position_embeddings=256)
    torch.manual_seed(0)
    return transformers.LlamaForCausalLM(cfg).to(dev).float()


def _setup(dev, top_k=2, with_selector=True):
    reader = _reader(dev)
    layers = injection_layers(reader, DEPTHS)
    itf = ModelInterface(64, 32, layers).to(dev)
    randomize(itf, seed=21, scale=0.3)
    lib = Library([skill_rho(32, DEPTHS, n=n, seed=i) for i, n in enumerate((9, 40, 17, 64))], layers, DEPTHS)
    sel = None
    if with_selector:
        torch.manual_seed(3)
        sel = LayerSelector(64, layers, k=2, alpha_init=0.05).to(dev)
        randomize(sel, seed=5, scale=1.0)
    return reader, layers, itf, lib, sel


def _tensors(lib):
    return {li: (lib.K[li].cpu(), lib.mask[li].cpu(), lib.S[li].cpu()) for li in lib.layers}


def _logits(m, ids):
    return m(ids).logits


class _CountingSel:
    def __init__(self, inner):
        self.inner, self.resets = inner, 0

    def reset(self):
        self.resets += 1
        self.inner.reset()

    def selected_rows(self, h, li):
        return self.inner.selected_rows(h, li)

    def apply(self, delta, h, li):
        return self.inner.apply(delta, h, li)


def test_prompt_forward_and_training_step(dev):
    """No selector here: its matched-norm rescale makes the update independent of the gate and
    gain scalars, so their gradients vanish analytically and cannot be compared."""
    say("hf reader: forward + train step")
    reader, layers, itf, lib, sel = _setup(dev, with_selector=False)
    ids = torch.randint(0, 128, (2, 21), generator=torch.Generator().manual_seed(1))
    inj = LibraryInjector(reader, itf, top_k=2, selector=sel)
    inj.load_library(lib)
    logits = reader(ids.to(dev)).logits
    loss = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, 128), ids[:, 1:].reshape(-1).to(dev))
    itf.zero_grad()
    loss.backward()
    inj.detach()
    assert len(inj.route_terms) == len(layers) and all(w.requires_grad for _, w in inj.route_terms)
    ref, (it, _) = oracle_forward(reader, ids, itf, _tensors(lib), top_k=2, selector=sel, grad=True, call=_logits)
    ok, err, rn = close(logits, ref)
    assert ok, (err, rn)
    rloss = torch.nn.functional.cross_entropy(ref[:, :-1].reshape(-1, 128), ids[:, 1:].reshape(-1))
    rloss.backward()
    ours, theirs = dict(itf.named_parameters()), dict(it.named_parameters())
    for name in ("A.weight", "B.weight", "gate_w", "gate_b", "log_gain"):
        ok, err, rn = close(ours[name].grad, theirs[name].grad, rel=2e-2, atol=5e-3)
        assert ok, (name, err, rn)


def test_greedy_decode_with_cache(dev):
    say("hf reader: greedy decode")
    reader, layers, itf, lib, sel = _setup(dev)
    ids = torch.randint(0, 128, (2, 11), generator=torch.Generator().manual_seed(2)).to(dev)
    counting = _CountingSel(sel)
    inj = LibraryInjector(reader, itf, top_k=2, selector=counting)
    inj.load_library(lib)
    new = 5
    with torch.no_grad():
        out = reader.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False,
                              pad_token_id=0)
    assert out.shape == (2, 11 + new)
    forwards = counting.resets
    assert forwards == new                                 # prompt + new - 1 cached steps
    assert len(inj.mag_terms) == forwards * len(layers) and not inj.route_terms
    with torch.no_grad():
        full = reader(out).logits                          # teacher-forced over the whole sequence
    inj.detach()
    sel.reset()
    ref, _ = oracle_forward(reader, out, itf, _tensors(lib), top_k=2, selector=sel, call=_logits)
    ok, err, rn = close(full, ref)
    assert ok, (err, rn)
