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


def test_boundary_gap_closed_forms():
    """boundary_gap = (k-th largest dot) - ((k+1)-th largest dot), in fp64.  With S = I the dots
    are the query's own entries, so every gap is known in closed form: a planted tie at the k-th
    place gives exactly 0, planted gaps give themselves (entries out of order, so a missing sort
    or an off-by-one rank fails), and dense routing (k = 0 or k >= C) gives +inf."""
    S = torch.eye(4, dtype=torch.float64)
    q = torch.tensor([[[0.125, 0.625, 0.875, 0.5]], [[0.125, 0.625, 0.875, 0.625]]], dtype=torch.float64)
    assert O.boundary_gap(q, S, 1).tolist() == [[0.25], [0.25]]
    assert O.boundary_gap(q, S, 2).tolist() == [[0.125], [0.0]]        # row 1: a tie at the boundary
    assert O.boundary_gap(q, S, 3).tolist() == [[0.375], [0.5]]
    for k in (0, 4, 9):
        g = O.boundary_gap(q, S, k)
        assert g.shape == (2, 1) and bool(torch.isinf(g).all()) and g.dtype == torch.float64
    # fp32 inputs are compared in fp64: a gap below fp32's resolution near 1 is still seen
    q32 = torch.tensor([[1.0, 1.0 - 2.0 ** -23, 0.0]], dtype=torch.float32)
    assert O.boundary_gap(q32, torch.eye(3), 1).item() == 2.0 ** -23


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


# ---------------------------------------------------------------- R3 / R8: rms_norm, query, epilogue
# deltaskill (which holds rms_norm and ModelInterface) is absent, so the eps and the interface's
# initialisation stay documented parameters; what the mathematics fixes is pinned here.
def test_rms_norm_closed_forms():
    """Constant vector c*1 -> c / sqrt(c^2 + eps) in every entry (a sum in place of the mean would
    give c / sqrt(d c^2)); the output RMS is sqrt(ms / (ms + eps)); positive scaling leaves the
    output unchanged up to eps; a pure-Python loop on a ragged vector."""
    for c, d in ((3.0, 7), (-0.5, 16), (1e-2, 5)):
        y = O.rms_norm(torch.full((2, d), c, dtype=torch.float64))
        want = c / math.sqrt(c * c + 1e-6)
        assert torch.allclose(y, torch.full_like(y, want), rtol=0, atol=1e-15)
    x = torch.randn(4, 33, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    y = O.rms_norm(x)
    ms = x.pow(2).mean(-1)
    assert torch.allclose(y.pow(2).mean(-1).sqrt(), (ms / (ms + 1e-6)).sqrt(), rtol=0, atol=1e-14)
    # scaling by a moves the output by the relative amount eps (1 - 1/a^2) / (2 ms) at most
    assert torch.allclose(O.rms_norm(x * 250.0), y, rtol=2e-6, atol=0)
    assert not torch.allclose(O.rms_norm(x * 250.0), y, rtol=1e-9, atol=0)
    row = [0.25, -1.5, 2.0, 0.0, 3.75]
    ms_py = sum(v * v for v in row) / len(row)
    got = O.rms_norm(torch.tensor(row, dtype=torch.float64))
    for j, v in enumerate(row):
        assert abs(float(got[j]) - v / math.sqrt(ms_py + 1e-6)) < 1e-14


def test_query_closed_forms():
    """itf_query (xenc/injector.py:54-58): q = A hn / (|A hn| + 1e-6).  Identity A gives
    hn / (|hn| + 1e-6); the norm is |A hn| / (|A hn| + 1e-6) < 1; positive scaling of hn keeps
    the direction; a pure-Python matrix-vector product on a tiny case (a transposed A fails it)."""
    g = torch.Generator().manual_seed(7)
    hn = torch.randn(3, 4, 6, generator=g, dtype=torch.float64)
    q = O.query(hn, torch.eye(6, dtype=torch.float64))
    assert torch.allclose(q, hn / (hn.norm(dim=-1, keepdim=True) + 1e-6), rtol=0, atol=1e-15)
    A = torch.randn(5, 6, generator=g, dtype=torch.float64)
    q = O.query(hn, A)
    n = (hn @ A.T).norm(dim=-1)
    assert torch.allclose(q.norm(dim=-1), n / (n + 1e-6), rtol=0, atol=1e-14)
    assert bool((q.norm(dim=-1) < 1).all())
    q2 = O.query(hn * 40.0, A)
    cos = (q * q2).sum(-1) / (q.norm(dim=-1) * q2.norm(dim=-1))
    assert torch.allclose(cos, torch.ones_like(cos), rtol=0, atol=1e-14)
    A2 = [[1.0, 2.0, 0.0], [0.0, -1.0, 3.0]]
    h = [0.5, -2.0, 1.0]
    Ah = [sum(A2[i][j] * h[j] for j in range(3)) for i in range(2)]
    nrm = math.sqrt(sum(v * v for v in Ah))
    got = O.query(torch.tensor([h], dtype=torch.float64), torch.tensor(A2, dtype=torch.float64))[0]
    for i in range(2):
        assert abs(float(got[i]) - Ah[i] / (nrm + 1e-6)) < 1e-15
    bias = torch.tensor([1.0, -1.0], dtype=torch.float64)
    got_b = O.query(torch.tensor([h], dtype=torch.float64), torch.tensor(A2, dtype=torch.float64), bias)[0]
    Ahb = [Ah[0] + 1.0, Ah[1] - 1.0]
    nb = math.sqrt(sum(v * v for v in Ahb))
    assert abs(float(got_b[0]) - Ahb[0] / (nb + 1e-6)) < 1e-15


def test_epilogue_closed_forms():
    """delta = gain_scale * exp(log_gain[p]) * sigmoid(hn . gate_w + gate_b[p]) * B(r)
    (xenc/injector.py:61-77, 266-267):
      gate_w = 0, gate_b = 0, log_gain = 0, B = I       -> 0.5 r
      gate_b = log 3 (sigmoid = 3/4), log_gain = log 2  -> 1.5 B r (a sign flip in the gate gives 0.5)
      B = 0 (the interface's zero initialisation)       -> exactly 0 (the branch is a no-op at init)
    and a pure-Python loop over a tiny case with a bias and gain_scale."""
    g = torch.Generator().manual_seed(11)
    hn = torch.randn(2, 3, 8, generator=g, dtype=torch.float64)
    r = torch.randn(2, 3, 8, generator=g, dtype=torch.float64)
    z8, one = torch.zeros(8, dtype=torch.float64), torch.eye(8, dtype=torch.float64)
    zero = torch.tensor(0.0, dtype=torch.float64)
    d = O.epilogue(hn, r, one, None, z8, zero, zero)
    assert torch.allclose(d, 0.5 * r, rtol=0, atol=1e-15)
    Bw = torch.randn(5, 8, generator=g, dtype=torch.float64)
    d = O.epilogue(hn, r, Bw, None, z8, torch.tensor(math.log(3.0), dtype=torch.float64),
                   torch.tensor(math.log(2.0), dtype=torch.float64))
    assert torch.allclose(d, 1.5 * (r @ Bw.T), rtol=0, atol=1e-13)
    d = O.epilogue(hn, r, torch.zeros(5, 8, dtype=torch.float64), None, torch.randn(8, generator=g,
                   dtype=torch.float64), torch.tensor(-2.0, dtype=torch.float64), zero)
    assert float(d.abs().max()) == 0.0
    hn1, r1 = [0.5, -1.0, 2.0], [1.0, 0.25, -0.5]
    gw, gb, lg, gs = [0.3, 0.1, -0.2], -0.4, 0.7, 2.5
    Bm, bb = [[1.0, 0.0, 2.0], [-1.0, 3.0, 0.5]], [0.1, -0.2]
    gate = 1.0 / (1.0 + math.exp(-(sum(a * b for a, b in zip(hn1, gw)) + gb)))
    want = [gs * math.exp(lg) * gate * (sum(Bm[i][j] * r1[j] for j in range(3)) + bb[i]) for i in range(2)]
    t = lambda v: torch.tensor(v, dtype=torch.float64)  # noqa: E731
    got = O.epilogue(t([hn1]), t([r1]), t(Bm), t(bb), t(gw), t(gb), t(lg), gs)[0]
    for i in range(2):
        assert abs(float(got[i]) - want[i]) < 1e-14


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


# ----------------------------------------------------------------------------- D18 ((f)4)
def _d18_case(Ns=(5, 7, 4), T=3, P=2, Hkv=2, G=2, hd=4, seed=3):
    g = torch.Generator().manual_seed(seed)

    def r(*s):
        return torch.randn(*s, generator=g, dtype=torch.float64)
    D = len(Ns)
    docs = [(r(Hkv, n, hd), r(Hkv, n, hd)) for n in Ns]
    return r(D, Hkv, G, T, hd), r(Hkv, G, T, hd), docs, r(Hkv, P + T, hd), r(Hkv, P + T, hd), P


def test_d18_core_pure_python_loop():
    """d18_core against per-(head, row) loops: joint softmax over [doc keys (doc query) ; own keys
    (own query, causal)], LSE and max over the keys past `skip`, softmax over documents."""
    qd, qo, docs, Kown, Vown, P = _d18_case(Ns=(5, 7, 1))
    scale, skip, beta = 0.7, 2, 1.3
    out = O.d18_core(qd, qo, docs, Kown, Vown, P, scale, skip, beta)
    Hkv, G, T, hd = qo.shape
    dot = lambda a, b: sum(float(a[e]) * float(b[e]) for e in range(hd))
    for h, gg, t in itertools.product(range(Hkv), range(G), range(T)):
        od, rr, mx = [], [], []
        for d, (K, V) in enumerate(docs):
            sd = [scale * dot(qd[d, h, gg, t], K[h, j]) for j in range(K.shape[1])]
            so = [scale * dot(qo[h, gg, t], Kown[h, j]) for j in range(P + t + 1)]
            m = max(sd + so)
            ed, eo = [math.exp(x - m) for x in sd], [math.exp(x - m) for x in so]
            Z = sum(ed) + sum(eo)
            od.append([(sum(ed[j] * float(V[h, j, e]) for j in range(len(sd)))
                        + sum(eo[j] * float(Vown[h, j, e]) for j in range(len(so)))) / Z for e in range(hd)])
            content = sd[skip:] if len(sd) > skip else sd
            mc = max(content)
            rr.append(mc + math.log(sum(math.exp(x - mc) for x in content)))
            mx.append(mc)
        lm = max(beta * x for x in rr)
        ex = [math.exp(beta * x - lm) for x in rr]
        w = [x / sum(ex) for x in ex]
        assert torch.allclose(out["r"][h, gg, t], torch.tensor(rr, dtype=torch.float64), atol=1e-12)
        assert torch.allclose(out["rmax"][h, gg, t], torch.tensor(mx, dtype=torch.float64), atol=1e-12)
        assert torch.allclose(out["w"][h, gg, t], torch.tensor(w, dtype=torch.float64), atol=1e-12)
        want = [sum(w[d] * od[d][e] for d in range(len(docs))) for e in range(hd)]
        got = out["o"][t, (h * G + gg) * hd:(h * G + gg + 1) * hd]
        assert torch.allclose(got, torch.tensor(want, dtype=torch.float64), atol=1e-12)
    assert out["n"].tolist() == [3.0, 5.0, 1.0]          # N_d - skip, or N_d when N_d <= skip


def test_d18_core_routing_modes():
    """The routing modes the reference's tests exercise (tests/test_d18_library.py:73-93): w sums
    to 1; force = d is the one-document read of d; top_k = 1 is one-hot at the largest logit;
    wfix is used as given; a sharp beta picks the soft argmax; rmax <= r."""
    qd, qo, docs, Kown, Vown, P = _d18_case(Ns=(6, 9, 4, 8))
    soft = O.d18_core(qd, qo, docs, Kown, Vown, P, 0.5, skip=2)
    assert torch.allclose(soft["w"].sum(-1), torch.ones(soft["w"].shape[:-1], dtype=torch.float64))
    assert bool((soft["rmax"] <= soft["r"] + 1e-12).all())
    f1 = O.d18_core(qd, qo, docs, Kown, Vown, P, 0.5, skip=2, force=1)
    one = O.d18_core(qd[1:2], qo, docs[1:2], Kown, Vown, P, 0.5, skip=2)
    assert torch.allclose(f1["o"], one["o"], atol=1e-12) and torch.equal(one["w"], torch.ones_like(one["w"]))
    hard = O.d18_core(qd, qo, docs, Kown, Vown, P, 0.5, skip=2, top_k=1)
    assert torch.equal(hard["w"].argmax(-1), soft["r"].argmax(-1))
    assert torch.allclose(hard["w"].max(-1).values, torch.ones_like(hard["w"].max(-1).values))
    wf = torch.tensor([0.1, 0.2, 0.3, 0.4], dtype=torch.float64)
    fixed = O.d18_core(qd, qo, docs, Kown, Vown, P, 0.5, wfix=wf)
    assert torch.equal(fixed["w"][0, 0, 0], wf)
    sharp = O.d18_core(qd, qo, docs, Kown, Vown, P, 0.5, skip=2, beta=1e4)
    assert torch.equal(sharp["w"].argmax(-1), soft["w"].argmax(-1))


def test_d18_lib_read_one_document_is_the_joint_read():
    """With one document lib_read equals the D13 joint read (xenc/d18_library.py:14-15, RoPE is
    relative): q and the own keys rotated at the absolute positions N + P + t, one softmax over
    [operator ; own rows] (xenc/d13_read.py:192-245).  Also the incremental form: rows 0..3 then
    4..6 with the first call's past == all rows at once (tests/test_d18_library.py:60-70)."""
    pytest.importorskip("transformers")
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb
    import d18_tiny
    itf = d18_tiny.TinyItf()
    li = 5
    (K, V), = d18_tiny.operators(itf, [11])
    x = torch.randn(7, 64, generator=torch.Generator().manual_seed(3))
    got = O.d18_lib_read(itf, li, x, [(K, V)])
    att = itf.att[str(li)]
    hd = att.head_dim
    with torch.no_grad():
        xe = itf.map_x(li, x)
        T, N = xe.shape[0], K.shape[1]
        qh, gate = torch.chunk(att.q_proj(xe).view(T, -1, hd * 2), 2, dim=-1)
        q = att.q_norm(qh).transpose(0, 1)
        k = att.k_norm(att.k_proj(xe).view(T, -1, hd)).transpose(0, 1)
        v = att.v_proj(xe).view(T, -1, hd).transpose(0, 1)
        pos = torch.arange(N, N + T).view(1, 1, T).expand(3, 1, T)
        cos, sin = itf.rot(xe.unsqueeze(0), pos)
        qr, kr = apply_rotary_pos_emb(q.unsqueeze(0), k.unsqueeze(0), cos.float(), sin.float())
        Hkv = k.shape[0]
        G = q.shape[0] // Hkv
        Kall = torch.cat([K, kr[0]], 1).double()
        Vall = torch.cat([V, v], 1).double()
        s = torch.einsum("kgtd,kcd->kgtc", qr[0].double().view(Hkv, G, T, hd), Kall) * att.scaling
        col = torch.arange(N + T).view(1, -1)
        s = s.masked_fill((col > N + torch.arange(T).view(-1, 1)).view(1, 1, T, -1), float("-inf"))
        o = torch.einsum("kgtc,kcd->kgtd", torch.softmax(s, -1), Vall).reshape(-1, T, hd).transpose(0, 1).reshape(T, -1)
        y = itf.Bmap(li, att.o_proj((o * torch.sigmoid(gate.reshape(T, -1).double())).float()))
    assert torch.allclose(got["y"], y, atol=1e-5), float((got["y"] - y).abs().max())
    assert torch.equal(got["w"], torch.ones_like(got["w"]))
    a = O.d18_lib_read(itf, li, x[:4], [(K, V)])
    b = O.d18_lib_read(itf, li, x[4:], [(K, V)], past=a["past"])
    assert torch.allclose(torch.cat([a["y"], b["y"]]), got["y"], atol=1e-5)
