"""Host-side API: Library construction (R1/R2), LayerSelector (R10), the interface helpers and the
depth map, checked against the oracle and the reference tests' invariants
(tests/test_library.py:186-261, tests/test_selector.py:25-125, tests/test_interface.py).
CPU only: none of these calls a HIP kernel."""

from __future__ import annotations

import math

import pytest
import torch

import oracle as O
from kv_skill_v2_amd.depth import DEPTHS, DepthCollisionError, injection_layers, rho_layer_map
from kv_skill_v2_amd.interface import ModelInterface, load_interface, make_interface, save_interface
from kv_skill_v2_amd.library import Library
from kv_skill_v2_amd.selector import LayerSelector, rms_norm
from tiny import TinyLM, skill_rho

LAYERS8 = [2, 4, 6, 7]   # DEPTHS on an 8-layer reader


def _lib(skills, layers=LAYERS8, **kw):
    return Library(skills, layers, DEPTHS, **kw)


def test_depth_map():
    assert injection_layers(8, DEPTHS) == LAYERS8
    assert rho_layer_map(TinyLM(d=8, n_layers=8), DEPTHS) == dict(zip(DEPTHS, LAYERS8))
    assert injection_layers(36, DEPTHS) == [9, 18, 27, 35]
    with pytest.raises(DepthCollisionError):
        rho_layer_map(2, DEPTHS)
    with pytest.raises(ValueError):       # a collision is a ValueError too
        rho_layer_map(3, DEPTHS)


def test_library_matches_oracle():
    skills = [skill_rho(24, DEPTHS, n=n, seed=i) for i, n in enumerate((5, 9, 3, 9))]
    lib = _lib(skills)
    assert lib.n_chunks == 4 and lib.d_s == 24 and lib.layers == LAYERS8 and lib.V is None
    for li, rho in zip(LAYERS8, DEPTHS):
        K, M, S = O.library_tensors([s.K[rho] for s in skills])
        assert torch.equal(lib.K[li], K) and torch.equal(lib.mask[li], M)
        assert torch.allclose(lib.S[li], S, atol=1e-6)
        assert lib.n_valid(li).tolist() == [5, 9, 3, 9]
        assert lib.K[li].shape == (4, 9, 24)


def test_summary_is_unit_mean():
    skills = [skill_rho(32, DEPTHS, n=n, seed=i) for i, n in enumerate((6, 12, 3, 9))]
    lib = _lib(skills)
    li, rho = LAYERS8[0], DEPTHS[0]
    m = skills[2].K[rho].mean(0)
    assert torch.allclose(lib.S[li][2], m / m.norm(), atol=1e-5)


def test_subset_equals_rebuilt():
    skills = [skill_rho(32, DEPTHS, n=n, seed=i) for i, n in enumerate((6, 12, 3, 9))]
    lib = _lib(skills)
    for i in range(4):
        a, b = lib.subset([i]), _lib([skills[i]])
        assert a.n_chunks == 1 and a.layers == b.layers
        for li in a.layers:
            assert torch.equal(a.K[li], b.K[li]) and torch.equal(a.mask[li], b.mask[li])
            assert torch.allclose(a.S[li], b.S[li], atol=1e-6)
    ab = lib.subset([1, 3])
    ref = _lib([skills[1], skills[3]])
    for li in ab.layers:
        assert torch.equal(ab.K[li], ref.K[li]) and torch.allclose(ab.S[li], ref.S[li], atol=1e-6)
        Ko, Mo, So = O.subset(lib.K[li], lib.mask[li], [1, 3])
        assert torch.equal(ab.K[li], Ko) and torch.allclose(ab.S[li], So, atol=1e-6)
    with pytest.raises(ValueError):
        lib.subset([])


def test_centering():
    chunks = [skill_rho(24, DEPTHS, n=8, seed=s) for s in range(3)]
    base = _lib(chunks)
    zero = _lib(chunks, center={r: torch.zeros(24) for r in DEPTHS})
    for li in LAYERS8:
        assert torch.allclose(base.K[li], zero.K[li], atol=1e-6)
    mu = {r: torch.full((24,), 0.3) for r in DEPTHS}
    cen = _lib(chunks, center=mu)
    for li, rho in zip(LAYERS8, DEPTHS):
        M = cen.mask[li]
        norms = cen.K[li][M].norm(dim=-1)
        assert torch.allclose(norms, torch.ones_like(norms), atol=1e-4)
        assert not torch.allclose(cen.K[li], base.K[li])
        assert torch.equal(cen.K[li][~M], torch.zeros_like(cen.K[li][~M]))
        K, M2, S = O.library_tensors([c.K[rho] for c in chunks], center_mu=mu[rho])
        assert torch.allclose(cen.K[li], K, atol=1e-6) and torch.allclose(cen.S[li], S, atol=1e-6)


def test_library_guards_and_to():
    with pytest.raises(ValueError):
        Library([], LAYERS8, DEPTHS)
    with pytest.raises(ValueError):
        Library([skill_rho(8, DEPTHS)], LAYERS8[:3], DEPTHS)
    lib = _lib([skill_rho(8, DEPTHS, n=4, seed=1)])
    assert lib.to(dtype=torch.float64) is lib
    assert lib.K[2].dtype == torch.float64 and lib.S[2].dtype == torch.float64 and lib.mask[2].dtype == torch.bool


def test_untied_values():
    skills = [skill_rho(16, DEPTHS, n=n, seed=i) for i, n in enumerate((4, 7))]
    g = torch.Generator().manual_seed(9)
    for s in skills:
        s.V = {r: torch.randn(k.shape, generator=g) for r, k in s.K.items()}
    lib = _lib(skills)
    assert lib.V is not None
    assert torch.equal(lib.V[LAYERS8[1]][1, :7], skills[1].V[DEPTHS[1]])
    assert torch.equal(lib.V[LAYERS8[1]][0, 4:], torch.zeros(3, 16))
    sub = lib.subset([1])
    assert sub.V is not None and sub.V[LAYERS8[0]].shape == (1, 7, 16)


def test_from_doc_cache():
    g = torch.Generator().manual_seed(2)
    n_tok = [32, 32, 26]
    chunks, start = [], 0
    for n in n_tok:
        chunks.append({"K": {r: torch.randn(n, 24, generator=g) for r in DEPTHS}, "start": start, "n_tokens": n})
        start += n
    cache = {"depths": DEPTHS, "chunks": chunks, "doc_id": "dd", "encoder": "tiny-enc"}
    reader = TinyLM(d=40, n_layers=8)
    lib = Library.from_doc_cache(cache, reader)
    assert lib.n_chunks == 3 and lib.d_s == 24 and lib.layers == LAYERS8
    assert lib.mask[lib.layers[0]].sum(-1).tolist() == n_tok
    assert lib.K[lib.layers[0]].dtype == torch.float32
    assert [m["start"] for m in lib.chunk_meta] == [0, 32, 64]
    assert lib.chunk_meta[0]["doc_id"] == "dd"


def test_doc_cache_file_roundtrip(tmp_path):
    """save_doc_cache stores K (and V) as fp16 CPU tensors keyed by float depth; load_doc_cache
    reads it back with weights_only; a Library from the file equals one from the fp16 rows; the
    device pool build refuses a CPU device (no CPU path)."""
    from kv_skill_v2_amd.depth import load_doc_cache, save_doc_cache
    from kv_skill_v2_amd.ops import PagedLibrary

    g = torch.Generator().manual_seed(3)
    chunks = [{"K": {r: torch.randn(n, 16, generator=g) for r in DEPTHS},
               "V": {r: torch.randn(n, 16, generator=g) for r in DEPTHS}, "start": 0, "n_tokens": n}
              for n in (5, 9)]
    cache = {"depths": DEPTHS, "chunks": chunks, "doc_id": "x", "encoder": "e", "chunk_tokens": 512}
    path = tmp_path / "sub" / "c.pt"
    save_doc_cache(cache, str(path))
    assert sorted(p.name for p in path.parent.iterdir()) == ["c.pt"]   # no temporary left behind
    back = load_doc_cache(str(path))
    assert back["doc_id"] == "x" and back["chunk_tokens"] == 512 and len(back["chunks"]) == 2
    for c0, c1 in zip(chunks, back["chunks"]):
        for f in ("K", "V"):
            assert sorted(c1[f]) == sorted(float(r) for r in DEPTHS)
            for r in DEPTHS:
                t = c1[f][float(r)]
                assert t.dtype == torch.float16 and t.device.type == "cpu" and t.is_contiguous()
                assert torch.equal(t, c0[f][r].half())
    reader = TinyLM(d=40, n_layers=8)
    a = Library.from_doc_cache(back, reader)
    fp16 = {**cache, "chunks": [{**c, "K": {r: t.half() for r, t in c["K"].items()},
                                 "V": {r: t.half() for r, t in c["V"].items()}} for c in chunks]}
    b = Library.from_doc_cache(fp16, reader)
    for li in a.layers:
        assert torch.equal(a.K[li], b.K[li]) and torch.equal(a.V[li], b.V[li]) and torch.equal(a.S[li], b.S[li])
    with pytest.raises(RuntimeError, match="no CPU path"):
        PagedLibrary.from_doc_caches(back, 0.25, "cpu")
    from kv_skill_v2_amd.pool import LibraryPool
    with pytest.raises(RuntimeError, match="no CPU path"):
        LibraryPool(8, 64, 16, "cpu")
    from kv_skill_v2_amd.decode_reader import DecodeState
    with pytest.raises(RuntimeError, match="no CPU path"):
        DecodeState(4, 2, 2, 16, 8, 0, "cpu")


# ----------------------------------------------------------------------------- selector
D, CAND = 40, [3, 5, 7, 9, 11, 13, 15, 17]


def _sel(k=2, st=False, seed=0):
    torch.manual_seed(seed)
    return LayerSelector(D, CAND, k=k, alpha_init=0.02, straight_through=st)


def test_selector_weights_match_oracle():
    for st in (False, True):
        for k in (1, 2, 3):
            sel = _sel(k=k, st=st)
            h = torch.randn(3, 7, D)
            sel.compute(rms_norm(h))
            w = sel.weights()
            assert w.shape == (3, 7, 8)
            assert torch.allclose(w.sum(-1), torch.ones(3, 7), atol=1e-6)
            assert ((w != 0).sum(-1) == k).all() and (w >= 0).all()
            assert 0.0 <= float(sel.entropy()) <= math.log(k) + 1e-5
            z = sel.u(O.rms_norm(h))
            assert torch.allclose(w, O.selector_weights(z, k, st), atol=1e-6)


def test_selector_matched_norm_and_oracle():
    for st in (False, True):
        sel = _sel(st=st)
        alpha = float(sel.log_alpha.detach().exp())
        h = torch.randn(2, 5, D) * 3.0
        base = torch.randn(2, 5, D)
        for scale in (1.0, 100.0):
            sel.reset()
            sel.compute(rms_norm(h))
            w = sel.weights().detach().clone()
            for li in CAND:
                out = sel.apply(base * scale, h, li)
                ratio = out.norm(dim=-1) / h.norm(dim=-1)
                assert torch.allclose(ratio, w[..., sel.pos[li]] * alpha, atol=1e-5)
                ref = O.selector_apply(base * scale, h, w[..., sel.pos[li]], sel.log_alpha.detach())
                assert torch.allclose(out, ref, atol=1e-6)


def test_selector_gradients():
    sel = _sel()
    h = torch.randn(2, 4, D)
    delta = torch.randn(2, 4, D, requires_grad=True)
    sel.reset()
    sum(sel.apply(delta, h, li).sum() for li in CAND).backward()
    assert sel.u.weight.grad.abs().sum() > 0 and sel.u.bias.grad.abs().sum() > 0
    assert sel.log_alpha.grad.abs() > 0 and delta.grad is not None
    st = _sel(st=True)
    st.reset()
    sum((st.apply(torch.randn(2, 4, D), h, li) * (i + 1)).sum() for i, li in enumerate(CAND)).backward()
    assert st.u.bias.grad.abs().min() > 0


def test_selector_reset_decode_and_guards():
    sel = _sel()
    h = torch.randn(1, 6, D)
    for li in CAND:
        sel.apply(torch.randn(1, 6, D), h, li)
    assert sel.weights().shape == (1, 6, 8)
    sel.reset()
    assert sel.weights() is None and sel.entropy() is None
    prev = None
    for step in range(3):
        h1 = torch.randn(1, 1, D) * (step + 1)
        for li in CAND:
            out = sel.apply(torch.randn(1, 1, D), h1, li)
            assert out.shape == (1, 1, D) and torch.isfinite(out).all()
        w = sel.weights()
        assert torch.allclose(w, sel._weights_from_logits(sel.u(rms_norm(h1.float()))))
        if prev is not None:
            assert not torch.equal(w, prev)
        prev = w.detach().clone()
    sel.reset()
    hn0 = torch.randn(1, 1, D)
    sel.compute(hn0)
    w0 = sel.weights().clone()
    sel.apply(torch.randn(1, 1, D), torch.randn(1, 1, D), CAND[0])
    assert torch.equal(sel.weights(), w0)
    with pytest.raises(KeyError):
        sel.apply(torch.randn(1, 1, D), torch.randn(1, 1, D), 4)
    out = sel.apply(torch.randn(1, 3, D).bfloat16(), torch.randn(1, 3, D).bfloat16(), CAND[0])
    assert out.dtype == torch.bfloat16
    with pytest.raises(ValueError):
        LayerSelector(D, [3, 3])
    with pytest.raises(ValueError):
        LayerSelector(D, CAND, k=9)
    with pytest.raises(ValueError):
        LayerSelector(D, CAND, alpha_init=0.0)


def test_selected_rows_then_apply_reuse_weights():
    sel = _sel()
    h = torch.randn(2, 5, D)
    rows = sel.selected_rows(h, CAND[0])
    w = sel.weights().clone()
    assert torch.equal(rows, w[..., 0] != 0)
    sel.apply(torch.randn(2, 5, D), h, CAND[0])
    assert torch.equal(sel.weights(), w)
    assert torch.equal(sel.selected_rows(h, CAND[3]), w[..., 3] != 0)


# ----------------------------------------------------------------------------- interface
def test_make_interface_noop_and_shapes():
    itf = make_interface(40, 24, LAYERS8)
    assert isinstance(itf, ModelInterface) and itf.d_m == 40 and itf.d_s == 24
    assert itf.A.weight.shape == (24, 40) and itf.B.weight.shape == (40, 24)
    assert itf.B.weight.abs().sum() == 0 and itf.B.bias is None
    hn = rms_norm(torch.randn(2, 5, 40))
    assert itf.query(hn).shape == (2, 5, 24) and itf.gate(hn, 6).shape == (2, 5, 1)
    assert torch.equal(itf.write(torch.randn(2, 5, 24)), torch.zeros(2, 5, 40))
    assert float(itf.gain(4).detach()) == 1.0
    assert torch.allclose(itf.gate_b, torch.full((4,), -2.0)) and torch.equal(itf.log_gain, torch.zeros(4))
    assert itf._pos == {2: 0, 4: 1, 6: 2, 7: 3}
    with pytest.raises(ValueError):
        make_interface(40, 24, [2, 2, 4])
    low = make_interface(40, 24, LAYERS8, rank=8)
    assert sum(p.numel() for p in low.A.parameters()) == 40 * 8 + 8 * 24
    hn2 = rms_norm(torch.randn(3, 40))
    q = low.query(hn2)
    assert torch.allclose(q, O.query(hn2, low.A[1].weight @ low.A[0].weight), atol=1e-6)


def test_save_load_roundtrip(tmp_path):
    itf = make_interface(40, 24, LAYERS8)
    torch.manual_seed(0)
    with torch.no_grad():
        for p in itf.parameters():
            p.normal_()
    sel = LayerSelector(40, [1, 3, 5], k=2)
    path = str(tmp_path / "sub" / "itf.pt")
    save_interface(itf, path, selector=sel, extra={"step": 7})
    itf2, sel2, extra = load_interface(path, 40, 24, LAYERS8)
    for (k, a), (_, b) in zip(itf.state_dict().items(), itf2.state_dict().items()):
        assert torch.equal(a, b), k
    assert sel2 is not None and sel2.cand_layers == [1, 3, 5] and torch.equal(sel2.u.weight, sel.u.weight)
    assert extra == {"step": 7}
    with pytest.raises(ValueError):
        load_interface(path, 40, 32, LAYERS8)


def test_decode_reader_auto_chunk():
    """DecodeReader's split size (host logic): at most one workgroup per CU at capacity (or one
    split per (row, head) when even that is more), >= 512 keys, a multiple of 64, and splits
    that cover max_keys."""
    import math
    from kv_skill_v2_amd.decode_reader import DecodeReader
    assert DecodeReader.auto_chunk(32, 4, 16448) == 8256      # 2 splits: 256 workgroups
    assert DecodeReader.auto_chunk(8, 4, 16448) == 2112       # 8 splits: 256 workgroups
    assert DecodeReader.auto_chunk(4, 4, 16448) == 1088       # 16 splits: 256 workgroups
    assert DecodeReader.auto_chunk(1, 4, 16448) == 512        # 33 splits: 132 workgroups
    assert DecodeReader.auto_chunk(32, 4, 16448, cus=512) == 4160
    for cus in (80, 256, 304):
        for max_n, hkv, mk in [(32, 4, 16448), (1, 4, 16448), (8, 4, 2048), (4, 16, 512), (256, 8, 100000),
                               (1, 1, 1), (64, 8, 5000)]:
            c = DecodeReader.auto_chunk(max_n, hkv, mk, cus)
            S = math.ceil(mk / c)
            assert c >= 512 and c % 64 == 0 and S * c >= mk
            assert max_n * hkv * S <= max(cus, max_n * hkv), (cus, max_n, hkv, mk, c)
