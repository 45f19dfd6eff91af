"""GPU: the D18 multi-document read (xenc_d18_read, kv_skill_v2_amd/d18.py) against the fp64
oracle (d18_core / d18_lib_read, xenc/d18_library.py:34-96): the core over fp16 / bf16 / fp32
operators at several head shapes, row counts and own-row lengths; the routing modes (soft,
top-k with exact ties broken to the lower index, force, wfix, sharp beta); lib_read on a Qwen3.5
attention interface including the incremental form; and D18LibReader patched into a tiny Qwen3.5
reader (prefill + a decode step) against the same patch running the oracle."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd import d18, ops

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _case(Ns, T, P, Hkv, G, hd, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    D = len(Ns)
    qd = torch.randn(D, Hkv * G, T, hd, generator=g)
    qo = torch.randn(Hkv * G, T, hd, generator=g)
    docs = [(torch.randn(Hkv, n, hd, generator=g).to(dtype), torch.randn(Hkv, n, hd, generator=g).to(dtype))
            for n in Ns]
    Kown, Vown = torch.randn(Hkv, P + T, hd, generator=g), torch.randn(Hkv, P + T, hd, generator=g)
    return qd, qo, docs, Kown, Vown


def _oracle(qd, qo, docs, Kown, Vown, P, scale, **kw):
    D, Hq, T, hd = qd.shape
    Hkv = Kown.shape[0]
    return O.d18_core(qd.double().view(D, Hkv, Hq // Hkv, T, hd), qo.double().view(Hkv, Hq // Hkv, T, hd),
                      [(K.double(), V.double()) for K, V in docs], Kown.double(), Vown.double(), P, scale, **kw)


def _check(got, ref, tol):
    for key in ("o", "w", "r", "rmax"):
        a, b = got[key].double().cpu(), ref[key]
        err = float((a - b).abs().max())
        assert err <= tol * max(1.0, float(b.abs().max())), f"{key}: max-abs {err:.3g}"
    assert got["n"].cpu().tolist() == ref["n"].tolist()


@pytest.mark.parametrize("Ns,T,P,Hkv,G,hd,dtype,skip,top_k", [
    ([37], 1, 0, 2, 4, 128, torch.float16, 0, 0),
    ([20, 33, 7], 5, 9, 2, 2, 64, torch.bfloat16, 3, 0),
    ([50, 1, 64, 13, 9, 200], 3, 4, 1, 8, 128, torch.float32, 2, 2),
    ([300, 290], 2, 700, 4, 1, 256, torch.float16, 5, 1),
    ([16] * 10, 4, 0, 2, 3, 32, torch.bfloat16, 0, 4),
])
def test_d18_core_matches_oracle(dev, Ns, T, P, Hkv, G, hd, dtype, skip, top_k):
    say("d18 core", dict(Ns=Ns, T=T, P=P, Hkv=Hkv, G=G, hd=hd, dtype=str(dtype), skip=skip, top_k=top_k))
    qd, qo, docs, Kown, Vown = _case(Ns, T, P, Hkv, G, hd, dtype, sum(Ns) + T)
    scale = hd ** -0.5
    got = ops.d18_read(qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs], Kown.to(dev),
                       Vown.to(dev), scale, skip=skip, beta=1.3, top_k=top_k)
    _check(got, _oracle(qd, qo, docs, Kown, Vown, P, scale, skip=skip, beta=1.3, top_k=top_k), 2e-5)
    again = ops.d18_read(qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs], Kown.to(dev),
                         Vown.to(dev), scale, skip=skip, beta=1.3, top_k=top_k)
    assert all(torch.equal(got[k], again[k]) for k in ("o", "w", "r", "rmax"))


def test_d18_key_splits_and_decode_shape(dev):
    """Each unit's keys read in 1, 3 or 8 ranges by separate workgroups give the same result up to
    fp32 merge rounding (and each split count is deterministic); a decode-shaped call (one reader
    row, 6 documents of 2000 rows, G = 8, hd = 256, bf16 operators, auto split) matches the oracle."""
    say("d18 key splits / decode shape")
    qd, qo, docs, Kown, Vown = _case([300, 77, 129], 2, 40, 2, 4, 64, torch.float16, 11)
    dd = [(K.to(dev), V.to(dev)) for K, V in docs]
    res = [ops.d18_read(qd.to(dev), qo.to(dev), dd, Kown.to(dev), Vown.to(dev), 0.125, skip=3, nsplit=S)
           for S in (1, 3, 8)]
    for rr in res[1:]:
        for key in ("o", "w", "r", "rmax"):
            assert float((rr[key] - res[0][key]).abs().max()) < 1e-5, key
    _check(res[2], _oracle(qd, qo, docs, Kown, Vown, 40, 0.125, skip=3), 2e-5)
    qd, qo, docs, Kown, Vown = _case([2000] * 6, 1, 300, 1, 8, 256, torch.bfloat16, 12)
    got = ops.d18_read(qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs], Kown.to(dev),
                       Vown.to(dev), 256 ** -0.5, skip=4, top_k=2)
    _check(got, _oracle(qd, qo, docs, Kown, Vown, 300, 256 ** -0.5, skip=4, top_k=2), 2e-5)


def test_d18_repeated_calls_and_shape_changes(dev):
    """One call shape ten times in a row gives bit-identical results; a larger shape in between
    and the return to the first shape still match the oracle and the first results."""
    say("d18 repeated calls")

    def run(case, **kw):
        qd, qo, docs, Kown, Vown = case
        return ops.d18_read(qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs], Kown.to(dev),
                            Vown.to(dev), 0.1, skip=1, **kw)

    small = _case([40, 23], 1, 10, 2, 4, 128, torch.bfloat16, 21)
    big = _case([300, 120, 77], 3, 50, 2, 4, 128, torch.bfloat16, 22)
    first = run(small, nsplit=4)
    for _ in range(10):
        again = run(small, nsplit=4)
        assert all(torch.equal(first[k], again[k]) for k in ("o", "w", "r", "rmax"))
    _check(run(big, nsplit=5), _oracle(*big, 50, 0.1, skip=1), 2e-5)
    back = run(small, nsplit=4)
    assert all(torch.equal(first[k], back[k]) for k in ("o", "w", "r", "rmax"))
    _check(back, _oracle(*small, 10, 0.1, skip=1), 2e-5)


@pytest.mark.parametrize("dtype,nsplit", [(torch.bfloat16, 2), (torch.float16, 1), (torch.float32, 3)])
def test_d18_growing_scores_and_long_splits(dev, dtype, nsplit):
    """Keys whose scores climb along the document: row j of every document and of the own rows
    leans on the mean query direction with weight j / 4, so a query's score climbs by about 0.06 a
    key in log2 units (the queries project ~2 on that direction, scale 1/sqrt(128)): across a
    split of hundreds of keys the later tiles pass the running max by far more than 2^8, and the
    accumulators are rescaled mid-split; splits of up to 1,000 keys also run the multi-tile loop
    (several tiles per wave).  Against the fp64 oracle at the usual bar."""
    say("d18 growing scores", dict(dtype=str(dtype), nsplit=nsplit))
    g = torch.Generator().manual_seed(31)
    D, T, P, Hkv, G, hd = 2, 2, 700, 2, 4, 128
    Ns = [1000, 613]
    qd = torch.randn(D, Hkv * G, T, hd, generator=g)
    qo = torch.randn(Hkv * G, T, hd, generator=g)
    qdir = torch.nn.functional.normalize(qd.mean(dim=(0, 1, 2)), dim=0)
    odir = torch.nn.functional.normalize(qo.mean(dim=(0, 1)), dim=0)

    def climb(n, direction):
        base = torch.randn(Hkv, n, hd, generator=g) * 0.3
        ramp = (torch.arange(n, dtype=torch.float32) / 4.0).view(1, n, 1)
        return base + ramp * direction.view(1, 1, hd)

    docs = [(climb(n, qdir).to(dtype), torch.randn(Hkv, n, hd, generator=g).to(dtype)) for n in Ns]
    Kown, Vown = climb(P + T, odir), torch.randn(Hkv, P + T, hd, generator=g)
    scale = hd ** -0.5
    got = ops.d18_read(qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs], Kown.to(dev),
                       Vown.to(dev), scale, skip=5, nsplit=nsplit)
    ref = _oracle(qd, qo, docs, Kown, Vown, P, scale, skip=5)
    _check(got, ref, 2e-5)


def test_d18_routing_modes_and_ties(dev):
    """Documents 0 and 2 identical (same keys, same rotation): their route logits tie exactly, and
    top_k = 1 keeps the lower index as the oracle's stable top-k does; force, wfix and a sharp beta
    follow the oracle."""
    say("d18 routing modes")
    qd, qo, docs, Kown, Vown = _case([24, 24, 24, 24], 3, 5, 2, 2, 64, torch.float16, 7)
    docs[2] = docs[0]
    qd[2] = qd[0]
    scale = 0.125
    P = 5
    mk = lambda **kw: ops.d18_read(qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs],
                                   Kown.to(dev), Vown.to(dev), scale, skip=2, **kw)
    soft = mk()
    assert torch.equal(soft["r"][..., 0], soft["r"][..., 2])
    for kw in ({"top_k": 1}, {"top_k": 2}, {"force": 3}, {"wfix": torch.tensor([0.4, 0.3, 0.2, 0.1])},
               {"beta": 1e4}):
        _check(mk(**kw), _oracle(qd, qo, docs, Kown, Vown, P, scale, skip=2, **kw), 2e-5)
    hard = mk(top_k=1)
    w = hard["w"].cpu()
    assert bool(((w == 0) | (w == 1)).all()) and bool((w.sum(-1) == 1).all())
    assert not bool((w[..., 2] == 1).any()), "a tie must go to the lower index"


def test_d18_guards(dev):
    say("d18 guards")
    qd, qo, docs, Kown, Vown = _case([8, 8], 2, 0, 2, 2, 64, torch.float16, 1)
    args = (qd.to(dev), qo.to(dev), [(K.to(dev), V.to(dev)) for K, V in docs], Kown.to(dev), Vown.to(dev), 0.1)
    with pytest.raises(ValueError):
        ops.d18_read(*args, force=2)                                   # force >= D
    with pytest.raises(ValueError):
        ops.d18_read(qd[:, :, :, :48].contiguous().to(dev), qo[:, :, :48].contiguous().to(dev),
                     [(K[..., :48].contiguous().to(dev), V[..., :48].contiguous().to(dev)) for K, V in docs],
                     Kown[..., :48].contiguous().to(dev), Vown[..., :48].contiguous().to(dev), 0.1)   # hd 48
    with pytest.raises(RuntimeError):
        ops.d18_read(qd, qo, docs, Kown, Vown, 0.1)                    # CPU tensors: no CPU path
    with pytest.raises(RuntimeError):
        ops.d18_read(args[0].requires_grad_(), *args[1:])              # no backward


def _itf(dev):
    import d18_tiny
    return d18_tiny.TinyItf().to(dev), d18_tiny


def test_lib_read_matches_oracle_and_incremental(dev):
    say("d18 lib_read")
    itf, tiny = _itf(dev)
    li = 5
    ops_ = [(K.to(dev), V.to(dev)) for K, V in tiny.operators(itf, [20, 31, 17], seed=2)]
    x = torch.randn(7, 64, generator=torch.Generator().manual_seed(4)).to(dev)
    with torch.no_grad():
        got = d18.lib_read(itf, li, x, ops_, skip=2)
        ref = O.d18_lib_read(itf.cpu(), li, x.cpu(), [(K.cpu(), V.cpu()) for K, V in ops_], skip=2)
        itf.to(dev)
        for key in ("y", "o", "w", "r", "rmax"):
            err = float((got[key].double().cpu() - ref[key].double()).abs().max())
            assert err < 1e-4, f"{key}: {err:.3g}"
        assert got["n"].cpu().tolist() == [18.0, 29.0, 15.0]
        a = d18.lib_read(itf, li, x[:4], ops_, skip=2)
        b = d18.lib_read(itf, li, x[4:], ops_, skip=2, past=a["past"])
        assert float((torch.cat([a["y"], b["y"]]) - got["y"]).abs().max()) < 1e-5
        one = d18.lib_read(itf, li, x, ops_[1:2])
        f1 = d18.lib_read(itf, li, x, ops_, force=1)
        assert float((one["y"] - f1["y"]).abs().max()) < 1e-5
        # the route statistics: logsumexp bounds the max score, and exceeds it by at most log N_d
        assert bool((got["rmax"] <= got["r"] + 1e-5).all())
        assert bool((got["r"] - got["rmax"] <= got["n"].log().view(1, 1, 1, -1) + 1e-5).all())


def test_lib_reader_patch_matches_oracle_patch(dev, monkeypatch):
    """D18LibReader on a tiny Qwen3.5 reader (prefill of 6 rows, then one decode step) with the
    HIP lib_read == the same patch with lib_read replaced by the oracle's; off mode is the stock
    model; routes sum to 1 per head."""
    say("d18 reader patch")
    from transformers.models.qwen3_5 import modeling_qwen3_5 as M
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    itf, tiny = _itf(dev)
    cfg = Qwen3_5TextConfig(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                            intermediate_size=96, num_hidden_layers=6, vocab_size=128,
                            layer_types=["full_attention"] * 6)
    torch.manual_seed(0)
    reader = M.Qwen3_5ForCausalLM(cfg).float().to(dev).eval()
    op = {en: [(K.to(dev), V.to(dev)) for K, V in tiny.operators(itf, [25, 40], seed=en)] for en in tiny.LAYERS}
    rows = torch.randint(3, 100, (1, 6), generator=torch.Generator().manual_seed(1)).to(dev)

    def run(R):
        R.load(op, skip=1)
        R.mode = "lib"
        with torch.no_grad():
            a = reader(input_ids=rows, use_cache=True)
            b = reader(input_ids=torch.tensor([[7]], device=dev), past_key_values=a.past_key_values, use_cache=True)
        return a.logits, b.logits, {li: w.clone() for li, w in R.route.items()}

    R = d18.D18LibReader(reader, itf)
    a_hip, b_hip, route = run(R)
    R.detach()

    def oracle_lib_read(itf_, li, x, ops_, past=None, **kw):
        pk = ops.d18_pack(ops_)
        docs = list(zip(pk.K.cpu().split(pk.lengths, 1), pk.V.cpu().split(pk.lengths, 1)))
        o = O.d18_lib_read(itf_.cpu(), li, x.cpu(), docs,
                           past=None if past is None else (past[0].cpu(), past[1].cpu()), **kw)
        itf_.to(dev)
        return {k: (v.to(dev) if torch.is_tensor(v) else tuple(t.to(dev) for t in v)) for k, v in o.items()}

    monkeypatch.setattr(d18, "lib_read", oracle_lib_read)
    R2 = d18.D18LibReader(reader, itf)
    a_ref, b_ref, route_ref = run(R2)
    R2.detach()
    assert float((a_hip - a_ref).abs().max()) < 1e-4 and float((b_hip - b_ref).abs().max()) < 1e-4
    assert set(route) == set(tiny.LAYERS) and all(w.shape[-1] == 2 for w in route.values())
    assert all(abs(float(w.sum(-1).mean()) - 1) < 1e-5 for w in route.values())
    with torch.no_grad():
        stock = reader(input_ids=rows, use_cache=True).logits
    assert float((stock - a_hip).abs().max()) > 1e-5
