"""CPU restatement of xenc's Library read (test infrastructure; see oracle/__init__.py).

Every function follows the reference's operations in the reference's order; pass fp64 tensors
to evaluate the same math in double precision.  Citations are file:line in the reference.
"""

from __future__ import annotations

import math

import torch

EPS = 1e-6


# ----------------------------------------------------------------------------- Library (R1)
def l2(x: torch.Tensor) -> torch.Tensor:
    """xenc/library.py:21-22."""
    return x / (x.norm(dim=-1, keepdim=True) + EPS)


def summaries(K: torch.Tensor, M: torch.Tensor) -> torch.Tensor:
    """S = L2(masked mean of the valid rows) — xenc/library.py:69-74."""
    mean = (K * M.unsqueeze(-1).to(K.dtype)).sum(1) / M.sum(1, keepdim=True).clamp_min(1).to(K.dtype)
    return l2(mean)


def library_tensors(rows: list[torch.Tensor], dtype=torch.float32, center_mu: torch.Tensor | None = None):
    """Zero-padded K [C, N_max, d], valid-prefix mask [C, N_max], S [C, d] from per-chunk slot rows
    [n_c, d] — xenc/library.py:47-58 (padding, optional centering) and :67 (summaries)."""
    if not rows:
        raise ValueError("Library needs at least one chunk")
    n = [int(r.shape[0]) for r in rows]
    d = int(rows[0].shape[-1])
    K = torch.zeros(len(rows), max(n), d, dtype=dtype)
    M = torch.zeros(len(rows), max(n), dtype=torch.bool)
    for c, r in enumerate(rows):
        K[c, : n[c]] = r.to(dtype)
        M[c, : n[c]] = True
    if center_mu is not None:
        K = torch.where(M.unsqueeze(-1), l2(K - center_mu.to(dtype)), torch.zeros_like(K))
    return K, M, summaries(K, M)


def subset(K: torch.Tensor, M: torch.Tensor, idx) -> tuple:
    """Library.subset: keep chunks idx, re-trim N to their longest chunk — xenc/library.py:103-123."""
    it = torch.as_tensor(list(idx), dtype=torch.long)
    Ms = M.index_select(0, it)
    n = int(Ms.sum(-1).max())
    Ks = K.index_select(0, it)[:, :n].clone()
    Ms = Ms[:, :n].clone()
    return Ks, Ms, summaries(Ks, Ms)


# ----------------------------------------------------------------------------- route (R4)
def topk_mask(logit: torch.Tensor, k: int) -> torch.Tensor:
    """Boolean keep-mask of the k largest entries along the last dim; ties go to the lower index
    (torch.topk's tie order is unspecified; the build fixes this policy)."""
    order = torch.sort(logit, dim=-1, descending=True, stable=True).indices[..., :k]
    return torch.zeros_like(logit, dtype=torch.bool).scatter(-1, order, True)


def topk_order(logit: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the kept entries in rank order (descending logit, lower index first on ties)."""
    return torch.sort(logit, dim=-1, descending=True, stable=True).indices[..., :k]


def route(q: torch.Tensor, S: torch.Tensor, route_temp: float = 10.0, top_k: int = 0) -> torch.Tensor:
    """w [..., C] — LibraryInjector.route, xenc/injector.py:220-229."""
    logit = torch.einsum("...d,cd->...c", q, S) * route_temp
    C = logit.shape[-1]
    if top_k and top_k < C:
        logit = logit.masked_fill(~topk_mask(logit, top_k), float("-inf"))
    return torch.softmax(logit, -1)


def boundary_gap(q: torch.Tensor, S: torch.Tensor, top_k: int) -> torch.Tensor:
    """|dot_(k) - dot_(k+1)| per query in fp64: how close the top-k boundary is to a tie.
    Routed-index parity is exact wherever this gap exceeds the fp32 rounding of the dots."""
    dots = torch.einsum("...d,cd->...c", q.double(), S.double())
    C = dots.shape[-1]
    if not top_k or top_k >= C:
        return torch.full(dots.shape[:-1], float("inf"), dtype=torch.float64)
    s = torch.sort(dots, dim=-1, descending=True).values
    return s[..., top_k - 1] - s[..., top_k]


# ----------------------------------------------------------------------------- read (R5, R6)
def read(q: torch.Tensor, K: torch.Tensor, M: torch.Tensor, w: torch.Tensor, read_temp: float = 12.0,
         read_softmax: bool = True, V: torch.Tensor | None = None, force_attn=None,
         force_norm_match: bool = False):
    """(r [B,T,d], aw [B,T,C,N]) — the read of LibraryInjector._branch, xenc/injector.py:239-265.
    q [B,T,d]; K, V [C,N,d]; M [C,N] bool; w [B,T,C]."""
    a = torch.einsum("btd,cnd->btcn", q, K)
    if read_softmax:
        a = torch.softmax((a * read_temp).masked_fill(~M, float("-inf")), -1)
    else:
        n = M.sum(-1).to(a.dtype).clamp_min(1)
        a = a.masked_fill(~M, 0.0) / n.sqrt().view(1, 1, -1, 1)
    aw = a * w.unsqueeze(-1)
    if force_attn is not None:                                   # :246-258
        fa = force_attn.to(aw.dtype)
        if fa.shape != aw.shape[-2:]:
            raise ValueError(f"force_attn {tuple(fa.shape)} != library [C,N] {tuple(aw.shape[-2:])}")
        fa = fa.expand_as(aw)
        if force_norm_match:
            Kf = K.reshape(-1, K.shape[-1])
            r0 = aw.reshape(*aw.shape[:2], -1) @ Kf
            r1 = fa.reshape(*fa.shape[:2], -1) @ Kf
            fa = fa * (r0.norm(dim=-1, keepdim=True) / (r1.norm(dim=-1, keepdim=True) + EPS)).unsqueeze(-1)
        aw = fa
    B_, T_, C_, N_ = aw.shape
    Vt = K if V is None else V
    r = aw.reshape(B_, T_, C_ * N_) @ Vt.reshape(C_ * N_, -1)
    return r, aw


def branch_read(q, K, M, S, read_temp=12.0, route_temp=10.0, top_k=0, read_softmax=True, V=None):
    """(r, w): route then read, both over ALL chunks as the reference does (xenc/injector.py:236-265)."""
    w = route(q, S, route_temp, top_k)
    r, _ = read(q, K, M, w, read_temp, read_softmax, V)
    return r, w


def read_routed(q: torch.Tensor, K: torch.Tensor, M: torch.Tensor, order: torch.Tensor, wsel: torch.Tensor,
                read_temp: float = 12.0, read_softmax: bool = True) -> torch.Tensor:
    """r [Q, d] reading only the routed chunks order[Q, k] with weights wsel[Q, k] — equal to
    `read` in exact arithmetic (unrouted chunks carry w = 0 there).  q [Q, d]."""
    Kc = K[order]                                   # [Q, k, N, d]
    Mc = M[order]                                   # [Q, k, N]
    a = torch.einsum("qd,qknd->qkn", q, Kc)
    if read_softmax:
        a = torch.softmax((a * read_temp).masked_fill(~Mc, float("-inf")), -1)
    else:
        n = Mc.sum(-1).to(a.dtype).clamp_min(1)
        a = a.masked_fill(~Mc, 0.0) / n.sqrt().unsqueeze(-1)
    return torch.einsum("qkn,qknd->qd", a * wsel.unsqueeze(-1), Kc)


def read_dq(q, K, M, S, g, read_temp=12.0, route_temp=10.0, top_k=0, dw_ext=None):
    """Closed-form dL/dq of (route + softmax read) given g = dL/dr (and optionally dL/dw):
        u[c,n] = <g, K[c,n]>,  gamma_c = sum_n p u,  dq_read = read_temp sum w_c p (u - gamma_c) K
        dl_c = w_c (dw_c - sum w dw) with dw = gamma (+ dw_ext),  dq_route = route_temp sum dl_c S_c
    This is what autograd gives on the reference forward (scripts/register_doc.py:699)."""
    w = route(q, S, route_temp, top_k)
    a = torch.einsum("btd,cnd->btcn", q, K)
    p = torch.softmax((a * read_temp).masked_fill(~M, float("-inf")), -1)
    u = torch.einsum("btd,cnd->btcn", g, K)
    gamma = (p * u).sum(-1)                                     # [B,T,C]
    ds = w.unsqueeze(-1) * p * (u - gamma.unsqueeze(-1))
    dq = read_temp * torch.einsum("btcn,cnd->btd", ds, K)
    dw = gamma if dw_ext is None else gamma + dw_ext
    dl = w * (dw - (w * dw).sum(-1, keepdim=True))
    dq = dq + route_temp * torch.einsum("btc,cd->btd", dl, S)
    return dq, gamma


# ----------------------------------------------------------------------------- epilogue (R3, R8)
def rms_norm(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """deltaskill.derive.rms_norm is absent (parity unpinned); eps follows the local copies
    xenc/hyb_hm.py:37-38 and xenc/p5_copy.py:99-101."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def query(hn: torch.Tensor, A_w: torch.Tensor, A_b: torch.Tensor | None = None) -> torch.Tensor:
    """itf_query: q = A(hn); q / (|q| + 1e-6) — xenc/injector.py:54-58."""
    q = torch.nn.functional.linear(hn, A_w, A_b)
    return q / (q.norm(dim=-1, keepdim=True) + EPS)


def epilogue(hn, r, B_w, B_b, gate_w, gate_b_p, log_gain_p, gain_scale: float = 1.0):
    """delta = gain_scale * exp(log_gain[p]) * sigmoid(hn.gate_w + gate_b[p]) * B(r)
    — itf_gate/itf_gain/itf_write and _branch, xenc/injector.py:61-77, 266-267."""
    g = torch.sigmoid(hn @ gate_w + gate_b_p).unsqueeze(-1)
    return gain_scale * torch.exp(log_gain_p) * g * torch.nn.functional.linear(r, B_w, B_b)


# ----------------------------------------------------------------------------- selector (R10)
def selector_weights(z: torch.Tensor, k: int, straight_through: bool = False) -> torch.Tensor:
    """LayerSelector._weights_from_logits, xenc/selector.py:59-67 (ties to the lower index)."""
    order = topk_order(z, k)
    v = z.gather(-1, order)
    w_sparse = torch.zeros_like(z).scatter(-1, order, torch.softmax(v, dim=-1))
    if not straight_through:
        return w_sparse
    w_hard = torch.zeros_like(z).scatter(-1, order, torch.full_like(v, 1.0 / k))
    w_soft = torch.softmax(z, dim=-1)
    return w_hard + (w_soft - w_soft.detach())


def selector_apply(delta: torch.Tensor, h: torch.Tensor, w_l: torch.Tensor, log_alpha) -> torch.Tensor:
    """Matched-norm rescale then weight — LayerSelector.apply, xenc/selector.py:106-110."""
    d = delta.float()
    rel = d.norm(dim=-1, keepdim=True) / (h.float().norm(dim=-1, keepdim=True) + EPS)
    d = d / (rel + EPS) * torch.as_tensor(log_alpha, dtype=d.dtype).exp()
    return (w_l.unsqueeze(-1).to(d.dtype) * d).to(delta.dtype)


# ----------------------------------------------------------------------------- op B (R11)
def decode_read_ref(q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, scale):
    """Joint softmax over [operator pages ; own pages] per query head with GQA — the reference's
    pure-torch decode read, xenc/d23_read_kernels.py:31-47.  Returns fp32 [N, Hq, D]."""
    N, Hq, D = q.shape
    Hkv = op_k.shape[2]
    G = Hq // Hkv
    out = torch.zeros(N, Hq, D, dtype=torch.float32)
    for n in range(N):
        lo, lw = int(op_len[n]), int(own_len[n])
        K1 = op_k[op_bt[n].long()].reshape(-1, Hkv, D)[:lo]
        V1 = op_v[op_bt[n].long()].reshape(-1, Hkv, D)[:lo]
        K2 = own_k[own_bt[n].long()].reshape(-1, Hkv, D)[:lw]
        V2 = own_v[own_bt[n].long()].reshape(-1, Hkv, D)[:lw]
        Kc = torch.cat([K1, K2]).float().repeat_interleave(G, 1)
        Vc = torch.cat([V1, V2]).float().repeat_interleave(G, 1)
        s = torch.einsum("hd,lhd->hl", q[n].float(), Kc) * scale
        out[n] = torch.einsum("hl,lhd->hd", torch.softmax(s, -1), Vc)
    return out


def ref_varlen(q, k, v, cu_q, seqused_k, softmax_scale, block_table, causal=False):
    """Paged varlen attention with log-sum-exp output (fp32) — the reference's stand-in for
    flash_attn_varlen_func, xenc/d23_vllm_plugin.py:319-340.  Returns (out [n,Hq,D], lse [Hq,n])."""
    Hq, hd = q.shape[1], q.shape[2]
    Hkv = k.shape[2]
    G = Hq // Hkv
    out = torch.zeros(q.shape, dtype=torch.float32)
    lse = torch.zeros(Hq, q.shape[0])
    cu, used, bt = cu_q.tolist(), seqused_k.tolist(), block_table.long()
    for i in range(len(cu) - 1):
        a, b, n = cu[i], cu[i + 1], used[i]
        Kc = k[bt[i]].reshape(-1, Hkv, hd)[:n].float().repeat_interleave(G, 1)
        Vc = v[bt[i]].reshape(-1, Hkv, hd)[:n].float().repeat_interleave(G, 1)
        s_ = torch.einsum("thd,nhd->htn", q[a:b].float(), Kc) * softmax_scale
        if causal:
            T = b - a
            col = torch.arange(n).view(1, n)
            row = torch.arange(T).view(T, 1)
            s_ = s_.masked_fill((col > n - T + row).unsqueeze(0), float("-inf"))
        lse[:, a:b] = torch.logsumexp(s_, -1)
        out[a:b] = torch.einsum("htn,nhd->thd", torch.softmax(s_, -1), Vc)
    return out, lse


def lse_merge(o1, l1, o2, l2):
    """Merge two partial attentions by log-sum-exp — xenc/d23_vllm_plugin.py:393-397."""
    lse = torch.logaddexp(l1, l2)
    return o1.float() * torch.exp(l1 - lse).t().unsqueeze(-1) + o2.float() * torch.exp(l2 - lse).t().unsqueeze(-1)


# ----------------------------------------------------------------------------- batched decode (C2/C3)
def batched_decode(q: torch.Tensor, libs, route_temp=10.0, read_temp=12.0, top_k=0, routed_only=False):
    """One query row per sequence b, each reading its own Library (K_b, M_b, S_b): the reference has
    one Library per call, so this is a loop of calls (xenc/injector.py:236-265 per sequence).
    routed_only=True reads just the routed chunks (same value, fewer bytes).
    Returns (r [B, d], list of w_b [C_b])."""
    rs, ws = [], []
    for b, (K, M, S) in enumerate(libs):
        qb = q[b].view(1, 1, -1)
        w = route(qb, S, route_temp, top_k)
        if routed_only:
            C = S.shape[0]
            k = C if (not top_k or top_k >= C) else top_k
            order = topk_order(w.view(1, -1), k)
            r = read_routed(q[b:b + 1], K, M, order, w.view(1, -1).gather(-1, order), read_temp)
        else:
            r, _ = read(qb, K, M, w, read_temp)
        rs.append(r.reshape(-1))
        ws.append(w.reshape(-1))
    return torch.stack(rs), ws


# ----------------------------------------------------------------------------- D8 slot top-k read ((f)4)
def select_scores(q: torch.Tensor, keys: torch.Tensor, valid: torch.Tensor | None = None,
                  pool: str = "max") -> torch.Tensor:
    """Pooled selection scores [B, S] at one query position — TopKSelector.head_scores +
    pool_scores (query "last"), xenc/topk_read.py:205-226: per query head h,
    s_h[i] = q_h . K[i, h // G] (GQA, G = n_q / n_kv, no RoPE), then max (or mean) over the
    heads; invalid slots -inf.  q [B, n_q, hd], keys [S, n_kv, hd]."""
    B, n_q, hd = q.shape
    n_kv = keys.shape[1]
    G = n_q // n_kv
    qh = q.reshape(B, n_kv, G, hd)
    s = torch.einsum("bkgd,skd->bkgs", qh, keys.to(q.dtype)).reshape(B, n_q, -1)
    s = s.amax(1) if pool == "max" else s.mean(1)
    if valid is not None:
        s = s.masked_fill(~valid.bool().view(1, -1), float("-inf"))
    return s


def topk_read(q: torch.Tensor, K: torch.Tensor, idx: torch.Tensor, read_temp: float = 12.0,
              read_softmax: bool = True, V: torch.Tensor | None = None) -> torch.Tensor:
    """The D8 read over the selected slots — TopKLibraryInjector._branch, xenc/topk_read.py:390-410:
    Ks, Vs = K.flat[idx], V.flat[idx]; a = q . Ks; a = softmax(read_temp * a) (or a / sqrt(k));
    r = a . Vs.  q [B, T, d]; K, V [C, N, d]; idx [B, k] flat indices into [C * N] (a single row
    is shared by every batch row)."""
    Kf = K.reshape(-1, K.shape[-1])
    Vf = (K if V is None else V).reshape(-1, K.shape[-1])
    if idx.shape[0] != q.shape[0]:
        idx = idx[:1].expand(q.shape[0], -1)
    Ks, Vs = Kf[idx], Vf[idx]
    a = torch.einsum("btd,bkd->btk", q, Ks)
    a = torch.softmax(a * read_temp, -1) if read_softmax else a / (idx.shape[-1] ** 0.5)
    return torch.einsum("btk,bkd->btd", a, Vs)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("math", "torch", "annotations")]
