"""Pins of the CPU oracle: each oracle function is checked against something it does not share
code with — pure-Python loops, closed forms, autograd/finite differences, or the invariants the
reference's own tests assert (cited per test)."""

from __future__ import annotations

import itertools
import math

import pytest
import torch

import oracle as O

torch.set_num_threads(2)


def _rows(n, d, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g, dtype=torch.float64)
    return x / x.norm(dim=-1, keepdim=True)


def _tiny_lib(ns=(4, 2, 3), d=6, seed=0):
    rows = [_rows(n, d, seed + i) for i, n in enumerate(ns)]
    return rows, O.library_tensors(rows, dtype=torch.float64)


def _q(B, T, d, seed=9):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, d, generator=g, dtype=torch.float64)
    return q / q.norm(dim=-1, keepdim=True)


# ---------------------------------------------------------------- R1: Library / summaries
def test_summaries_closed_form_pure_python():
    """S[c] = m/|m| with m the mean of the valid rows (tests/test_library.py:200-204)."""
    rows, (K, M, S) = _tiny_lib(ns=(5, 1, 3), d=7)
    for c, r in enumerate(rows):
        n, d = r.shape
        m = [sum(float(r[i, j]) for i in range(n)) / n for j in range(d)]
        nm = math.sqrt(sum(v * v for v in m))
        for j in range(d):
            assert abs(float(S[c, j]) - m[j] / (nm + 1e-6)) < 1e-12
    assert K.shape == (3, 5, 7) and M.sum(-1).tolist() == [5, 1, 3]
    assert float(K[1, 1:].abs().sum()) == 0.0, "padded slots are zero"


def test_centering_invariants():
    """mu = 0 is a no-op; nonzero mu gives unit-norm valid rows and zero masked rows
    (tests/test_library.py:241-261)."""
    rows = [_rows(8, 24, s).float() for s in range(3)]
    rows[1] = rows[1][:5]
    K0, M0, S0 = O.library_tensors(rows)
    Kz, _, _ = O.library_tensors(rows, center_mu=torch.zeros(24))
    assert torch.allclose(K0, Kz, atol=1e-6)
    Kc, Mc, _ = O.library_tensors(rows, center_mu=torch.full((24,), 0.3))
    norms = Kc[Mc].norm(dim=-1)
    assert torch.allclose(norms, torch.ones_like(norms), atol=1e-4)
    assert float(Kc[~Mc].abs().sum()) == 0.0
    assert not torch.allclose(Kc, K0)


def test_subset_equals_rebuild():
    """Library.subset equals a Library built from those chunks (tests/test_library.py:186-199)."""
    rows = [_rows(n, 8, i) for i, n in enumerate((6, 12, 3, 9))]
    K, M, S = O.library_tensors(rows, dtype=torch.float64)
    for sel in ([2], [1, 3], [0, 2]):
        Ks, Ms, Ss = O.subset(K, M, sel)
        Kr, Mr, Sr = O.library_tensors([rows[i] for i in sel], dtype=torch.float64)
        assert torch.equal(Ks, Kr) and torch.equal(Ms, Mr) and torch.allclose(Ss, Sr, atol=1e-12)


# ---------------------------------------------------------------- R4: route
def _route_brute(q, S, route_temp, k):
    """Pure Python: chunk c is kept iff fewer than k chunks rank before it (larger dot, or equal
    dot and lower index); w = exp(l - max) / sum over kept."""
    C = len(S)
    logit = [route_temp * sum(a * b for a, b in zip(q, s)) for s in S]
    dots = [sum(a * b for a, b in zip(q, s)) for s in S]
    if k and k < C:
        kept = [sum(1 for c2 in range(C) if dots[c2] > dots[c] or (dots[c2] == dots[c] and c2 < c)) < k
                for c in range(C)]
    else:
        kept = [True] * C
    mx = max(l for l, kp in zip(logit, kept) if kp)
    e = [math.exp(l - mx) if kp else 0.0 for l, kp in zip(logit, kept)]
    z = sum(e)
    return [v / z for v in e]


@pytest.mark.parametrize("k", [0, 1, 2, 3, 5, 7])
def test_route_matches_brute_force_with_ties(k):
    d, C = 5, 7
    S = _rows(C, d, 3)
    S[4] = S[1]            # exact tie between chunks 1 and 4
    S[6] = S[2]            # and between 2 and 6
    q = _q(2, 3, d)
    w = O.route(q, S, 10.0, k)
    for b, t in itertools.product(range(2), range(3)):
        ref = _route_brute(q[b, t].tolist(), S.tolist(), 10.0, k)
        assert max(abs(float(a) - r) for a, r in zip(w[b, t], ref)) < 1e-12
    # invariants of tests/test_library.py:140-142
    assert torch.allclose(w.sum(-1), torch.ones(2, 3, dtype=torch.float64), atol=1e-12)
    nz = (w > 0).sum(-1)
    assert bool((nz == (k if 0 < k < C else C)).all())


def test_route_tie_goes_to_lower_index():
    S = torch.tensor([[1.0, 0.0], [0.0, 1.0], [1.0, 0.0]], dtype=torch.float64)
    q = torch.tensor([[[1.0, 0.0]]], dtype=torch.float64)
    w = O.route(q, S, 10.0, 1)
    assert w[0, 0].tolist() == [1.0, 0.0, 0.0]
    assert O.topk_order(torch.tensor([0.5, 0.9, 0.9, 0.1]), 3).tolist() == [1, 2, 0]


# ---------------------------------------------------------------- R5: read
def _read_brute(q, K, M, w, temp, softmax=True):
    C, N, d = len(K), len(K[0]), len(K[0][0])
    r = [0.0] * d
    for c in range(C):
        valid = [n for n in range(N) if M[c][n]]
        s = {n: sum(a * b for a, b in zip(q, K[c][n])) for n in valid}
        if softmax:
            mx = max(temp * s[n] for n in valid)
            e = {n: math.exp(temp * s[n] - mx) for n in valid}
            z = sum(e.values())
            p = {n: e[n] / z for n in valid}
        else:
            p = {n: s[n] / math.sqrt(len(valid)) for n in valid}
        for n in valid:
            for j in range(d):
                r[j] += w[c] * p[n] * K[c][n][j]
    return r


@pytest.mark.parametrize("softmax", [True, False])
def test_read_matches_pure_python_loops(softmax):
    rows, (K, M, S) = _tiny_lib(ns=(4, 2, 3), d=6)
    q = _q(1, 2, 6)
    w = O.route(q, S, 10.0, 2)
    r, aw = O.read(q, K, M, w, 12.0, softmax)
    for t in range(2):
        ref = _read_brute(q[0, t].tolist(), K.tolist(), M.tolist(), w[0, t].tolist(), 12.0, softmax)
        assert max(abs(float(a) - b) for a, b in zip(r[0, t], ref)) < 1e-12
    assert float(aw[..., ~M].abs().sum()) == 0.0, "masked slots get no weight"


def test_one_chunk_read_closed_form():
    """1-chunk Library: r = softmax(read_temp q K^T) K (tests/test_library.py:91-123)."""
    K = _rows(11, 16, 4).unsqueeze(0)
    M = torch.ones(1, 11, dtype=torch.bool)
    q = _q(2, 5, 16)
    r, _ = O.read(q, K, M, torch.ones(2, 5, 1, dtype=torch.float64), 12.0)
    ref = torch.softmax(12.0 * q @ K[0].T, -1) @ K[0]
    assert torch.allclose(r, ref, atol=1e-12)


def test_linear_read_closed_form():
    """read_softmax=False: r = sum_c w_c sum_n <q,K[c,n]>/sqrt(n_c) K[c,n] (tests/test_integration.py:139-173)."""
    rows, (K, M, S) = _tiny_lib(ns=(4, 2, 3), d=6)
    q = _q(1, 1, 6)
    w = O.route(q, S, 10.0, 0)
    r, _ = O.read(q, K, M, w, 12.0, read_softmax=False)
    ref = sum(float(w[0, 0, c]) * (rows[c] @ q[0, 0]) @ rows[c] / math.sqrt(rows[c].shape[0]) for c in range(3))
    assert torch.allclose(r[0, 0], ref, atol=1e-12)


def test_force_attn_onehot_reads_that_slot():
    """A one-hot forced [C,N] distribution reads exactly K[1,1] (tests/test_d6_force_attn.py:49-63)."""
    rows, (K, M, S) = _tiny_lib()
    q = _q(2, 3, 6)
    fa = torch.zeros(M.shape, dtype=torch.float64)
    fa[1, 1] = 1.0
    r, _ = O.read(q, K, M, O.route(q, S), force_attn=fa)
    assert torch.allclose(r, K[1, 1].expand(2, 3, -1), atol=1e-12)
    with pytest.raises(ValueError):
        O.read(q, K, M, O.route(q, S), force_attn=torch.zeros(3, 9))


def test_untied_values_used_and_routing_from_k():
    """An untied V changes the read; V := K equals the tied read (tests/test_attn_harvest.py:129-149)."""
    rows, (K, M, S) = _tiny_lib()
    q = _q(1, 2, 6)
    w = O.route(q, S, 10.0, 2)
    rt, _ = O.read(q, K, M, w)
    rs, _ = O.read(q, K, M, w, V=K.clone())
    ru, _ = O.read(q, K, M, w, V=torch.roll(K, 1, dims=1))
    assert torch.allclose(rt, rs, atol=1e-14) and (ru - rt).abs().max() > 1e-3


@pytest.mark.parametrize("k", [0, 2])
def test_routed_only_read_equals_full_read(k):
    rows, (K, M, S) = _tiny_lib(ns=(4, 2, 3, 5), d=6)
    q = _q(1, 4, 6)
    w = O.route(q, S, 10.0, k)
    r_full, _ = O.read(q, K, M, w)
    kk = k if k else 4
    order = O.topk_order(w[0], kk)
    r_r = O.read_routed(q[0], K, M, order, w[0].gather(-1, order))
    assert torch.allclose(r_full[0], r_r, atol=1e-12)


def test_lse_split_merge_equals_chunk_softmax():
    """The split-K identity the decode kernel relies on: per split (m_j, l_j, acc_j) merged by
    log-sum-exp equals the chunk's softmax read."""
    K = _rows(37, 8, 5)
    q = _q(1, 1, 8)[0, 0]
    s = 12.0 * K @ q
    ref = torch.softmax(s, 0) @ K
    parts = [(0, 9), (9, 20), (20, 37)]
    ms = [float(s[a:b].max()) for a, b in parts]
    ls = [float(torch.exp(s[a:b] - m).sum()) for (a, b), m in zip(parts, ms)]
    accs = [torch.exp(s[a:b] - m) @ K[a:b] for (a, b), m in zip(parts, ms)]
    mg = max(ms)
    l = sum(l_ * math.exp(m - mg) for l_, m in zip(ls, ms))
    acc = sum(a * math.exp(m - mg) for a, m in zip(accs, ms))
    assert torch.allclose(acc / l, ref, atol=1e-13)


# ---------------------------------------------------------------- dQ (prefill backward)
@pytest.mark.parametrize("k", [0, 2])
def test_read_dq_matches_autograd_and_finite_differences(k):
    rows, (K, M, S) = _tiny_lib(ns=(4, 2, 3), d=6)
    q = _q(1, 3, 6).requires_grad_(True)
    g = torch.randn(1, 3, 6, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    dw_ext = torch.randn(1, 3, 3, generator=torch.Generator().manual_seed(8), dtype=torch.float64)

    def loss(qq):
        w = O.route(qq, S, 10.0, k)
        r, _ = O.read(qq, K, M, w, 12.0)
        return (r * g).sum() + (w * dw_ext).sum()

    (gq,) = torch.autograd.grad(loss(q), q)
    dq, _ = O.read_dq(q.detach(), K, M, S, g, 12.0, 10.0, k, dw_ext=dw_ext)
    assert torch.allclose(gq, dq, atol=1e-10), float((gq - dq).abs().max())
    # central finite difference on two coordinates (top-k set is stable at this q)
    for (t, j) in ((0, 1), (2, 4)):
        e = torch.zeros_like(q)
        e[0, t, j] = 1e-6
        fd = (loss(q.detach() + e) - loss(q.detach() - e)) / 2e-6
        assert abs(float(fd) - float(dq[0, t, j])) < 1e-6


# ---------------------------------------------------------------- R10: selector
@pytest.mark.parametrize("k", [1, 2, 3])
def test_selector_weights_invariants(k):
    """sum 1, exactly k nonzeros, entropy <= log k (tests/test_selector.py:25-38)."""
    z = torch.randn(3, 7, 8, generator=torch.Generator().manual_seed(k))
    for st in (False, True):
        w = O.selector_weights(z, k, st)
        assert torch.allclose(w.sum(-1), torch.ones(3, 7), atol=1e-6)
        assert bool(((w != 0).sum(-1) == k).all()) and bool((w >= 0).all())
        ent = -(w * torch.log(w.clamp_min(1e-12))).sum(-1).mean()
        assert 0.0 <= float(ent) <= math.log(k) + 1e-5


def test_selector_matched_norm_identity():
    """|apply(delta)| / |h| = w_l * alpha per token (tests/test_selector.py:41-55)."""
    h = torch.randn(2, 5, 40, generator=torch.Generator().manual_seed(1)) * 3.0
    base = torch.randn(2, 5, 40, generator=torch.Generator().manual_seed(2))
    w = O.selector_weights(torch.randn(2, 5, 8, generator=torch.Generator().manual_seed(3)), 2)
    la = math.log(0.02)
    for scale in (1.0, 100.0):
        out = O.selector_apply(base * scale, h, w[..., 3], la)
        ratio = out.norm(dim=-1) / h.norm(dim=-1)
        assert torch.allclose(ratio, w[..., 3] * 0.02, atol=1e-5)


# ---------------------------------------------------------------- R11: op B oracle
def _opb_case(N=3, hq=16, hkv=4, d=32, bs=4, nb_op=20, nb_own=10, seed=0):
    """Shapes and lengths of tests/test_d23_kernels.py:26-35."""
    g = torch.Generator().manual_seed(seed)
    op_k, op_v = torch.randn(nb_op, bs, hkv, d, generator=g), torch.randn(nb_op, bs, hkv, d, generator=g)
    own_k, own_v = torch.randn(nb_own, bs, hkv, d, generator=g), torch.randn(nb_own, bs, hkv, d, generator=g)
    q = torch.randn(N, hq, d, generator=g)
    op_len = torch.tensor([13, 1, 37][:N] + [5] * max(0, N - 3), dtype=torch.int32)
    own_len = torch.tensor([3, 9, 1][:N] + [2] * max(0, N - 3), dtype=torch.int32)
    op_bt = torch.stack([torch.randperm(nb_op, generator=g)[:10] for _ in range(N)]).int()
    own_bt = torch.stack([torch.randperm(nb_own, generator=g)[:3] for _ in range(N)]).int()
    return q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len


def test_decode_ref_equals_two_part_lse_merge():
    """tests/test_d23_kernels.py:38-48."""
    q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len = _opb_case()
    cu = torch.arange(q.shape[0] + 1, dtype=torch.int32)
    o1, l1 = O.ref_varlen(q, op_k, op_v, cu, op_len, 0.3, op_bt)
    o2, l2 = O.ref_varlen(q, own_k, own_v, cu, own_len, 0.3, own_bt, causal=True)
    ref = O.decode_read_ref(q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, 0.3)
    assert torch.allclose(O.lse_merge(o1, l1, o2, l2), ref, atol=1e-5)


def test_decode_ref_pure_python_loop():
    q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len = _opb_case(N=2, hq=4, hkv=2, d=3, bs=2,
                                                                            nb_op=6, nb_own=4, seed=3)
    op_len = torch.tensor([5, 2], dtype=torch.int32)
    own_len = torch.tensor([1, 3], dtype=torch.int32)
    out = O.decode_read_ref(q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, 0.7)
    BS, G = 2, 2
    for n in range(2):
        keys = []
        for pool_k, pool_v, bt, ln in ((op_k, op_v, op_bt, op_len), (own_k, own_v, own_bt, own_len)):
            for i in range(int(ln[n])):
                keys.append((pool_k[int(bt[n, i // BS]), i % BS], pool_v[int(bt[n, i // BS]), i % BS]))
        for h in range(4):
            kvh = h // G
            s = [0.7 * sum(float(q[n, h, j]) * float(k[kvh, j]) for j in range(3)) for k, _ in keys]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            z = sum(e)
            for j in range(3):
                ref = sum(ei / z * float(v[kvh, j]) for ei, (_, v) in zip(e, keys))
                assert abs(float(out[n, h, j]) - ref) < 1e-5


# ---------------------------------------------------------------- D8 slot top-k read ((f)4)
def test_select_scores_pure_python_loop():
    """select_scores against explicit loops over query heads and slots (GQA: head h reads kv
    head h // G), for max and mean pooling, with invalid slots at -inf."""
    g = torch.Generator().manual_seed(41)
    B, n_q, n_kv, hd, S = 2, 6, 3, 5, 9
    q = torch.randn(B, n_q, hd, generator=g, dtype=torch.float64)
    keys = torch.randn(S, n_kv, hd, generator=g, dtype=torch.float64)
    valid = torch.tensor([1, 1, 0, 1, 1, 1, 0, 1, 1], dtype=torch.bool)
    G = n_q // n_kv
    for pool in ("max", "mean"):
        s = O.select_scores(q, keys, valid, pool)
        for b in range(B):
            for i in range(S):
                per_head = [sum(q[b, h, e].item() * keys[i, h // G, e].item() for e in range(hd)) for h in range(n_q)]
                want = (max(per_head) if pool == "max" else sum(per_head) / n_q) if valid[i] else -math.inf
                assert (s[b, i].item() == want) if want == -math.inf else abs(s[b, i].item() - want) < 1e-12


def test_topk_read_pure_python_and_one_chunk_equivalence():
    """topk_read against explicit loops; and with every slot of a one-chunk library selected it
    equals the standard read of that chunk (the reference's own equivalence,
    tests/test_topk_read.py:150-170)."""
    g = torch.Generator().manual_seed(43)
    C, N, d, T, k = 3, 4, 5, 2, 4
    K = torch.randn(C, N, d, generator=g, dtype=torch.float64)
    q = torch.randn(1, T, d, generator=g, dtype=torch.float64)
    idx = torch.tensor([[7, 0, 11, 5]])
    r = O.topk_read(q, K, idx, 12.0)
    Kf = K.reshape(-1, d)
    for t in range(T):
        sc = [sum(q[0, t, e].item() * Kf[f, e].item() for e in range(d)) * 12.0 for f in idx[0].tolist()]
        m = max(sc)
        ex = [math.exp(x - m) for x in sc]
        z = sum(ex)
        for e in range(d):
            want = sum(ex[j] / z * Kf[f, e].item() for j, f in enumerate(idx[0].tolist()))
            assert abs(r[0, t, e].item() - want) < 1e-12
    rl = O.topk_read(q, K, idx, read_softmax=False)
    a = torch.einsum("td,kd->tk", q[0], Kf[idx[0]]) / 2.0
    assert torch.allclose(rl[0], a @ Kf[idx[0]], atol=1e-12)
    K1 = K[:1]
    M1 = torch.ones(1, N, dtype=torch.bool)
    ref, _ = O.read(q, K1, M1, torch.ones(1, T, 1, dtype=torch.float64), 12.0)
    assert torch.allclose(O.topk_read(q, K1, torch.arange(N).view(1, -1), 12.0), ref, atol=1e-12)
