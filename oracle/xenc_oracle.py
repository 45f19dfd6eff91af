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


# ----------------------------------------------------------------------------- D18 multi-document read ((f)4)
def d18_core(qd: torch.Tensor, qo: torch.Tensor, docs: list, Kown: torch.Tensor, Vown: torch.Tensor, P: int,
             scale: float, skip: int = 0, beta: float = 1.0, top_k: int = 0, force: int | None = None,
             wfix: torch.Tensor | None = None) -> dict:
    """The attention core of lib_read, xenc/d18_library.py:63-90, given the rotated queries:
    qd [D, Hkv, G, T, hd] (rotated at N_d + P + t for document d), qo [Hkv, G, T, hd] (rotated at
    P + t), docs = [(K_d, V_d) [Hkv, N_d, hd]], Kown / Vown [Hkv, P + T, hd] (row t sees own
    columns <= P + t).  Per document: o_d = softmax([s_d ; s_own]) . [V_d ; V_own],
    r_d = logsumexp(s_d[skip:]) (all of s_d when N_d <= skip), rmax_d = max(s_d[skip:]);
    w = softmax_d(beta * r) (top_k kept, ties to the lower index; or force / wfix);
    o = sum_d w_d o_d.  -> {"o" [T, Hq*hd], "w", "r", "rmax" [Hkv, G, T, D], "n" [D]}."""
    Hkv, G, T, hd = qo.shape
    s_own = torch.einsum("kgtd,kcd->kgtc", qo, Kown) * scale
    col = torch.arange(P + T).view(1, -1)
    s_own = s_own.masked_fill((col > P + torch.arange(T).view(-1, 1)).view(1, 1, T, -1), float("-inf"))
    outs, routes, rmax, nlen = [], [], [], []
    for d, (K, V) in enumerate(docs):
        N = K.shape[1]
        s = torch.einsum("kgtd,kcd->kgtc", qd[d], K.to(qo.dtype)) * scale
        m = torch.maximum(s.amax(-1, keepdim=True), s_own.amax(-1, keepdim=True))
        e_d, e_o = (s - m).exp(), (s_own - m).exp()
        Z = e_d.sum(-1, keepdim=True) + e_o.sum(-1, keepdim=True)
        outs.append((torch.einsum("kgtc,kcd->kgtd", e_d, V.to(qo.dtype)) + torch.einsum("kgtc,kcd->kgtd", e_o, Vown)) / Z)
        sc = s[..., skip:] if N > skip else s
        routes.append(torch.logsumexp(sc, -1))
        rmax.append(sc.amax(-1))
        nlen.append(float(sc.shape[-1]))
    r = torch.stack(routes, -1)
    D = r.shape[-1]
    if force is not None:
        w = torch.zeros_like(r)
        w[..., int(force)] = 1.0
    elif wfix is not None:
        w = wfix.to(r).view(1, 1, 1, D).expand_as(r)
    else:
        logit = beta * r
        if top_k and top_k < D:
            logit = logit.masked_fill(~topk_mask(logit, top_k), float("-inf"))
        w = torch.softmax(logit, -1)
    O = torch.stack(outs, -2)
    o = (w.unsqueeze(-1) * O).sum(-2).reshape(Hkv * G, T, hd).transpose(0, 1).reshape(T, Hkv * G * hd)
    return {"o": o, "w": w, "r": r, "rmax": torch.stack(rmax, -1), "n": torch.tensor(nlen)}


def d18_lib_read(itf, li: int, x: torch.Tensor, ops: list, past=None, skip: int = 0, beta: float = 1.0,
                 top_k: int = 0, force: int | None = None, wfix: torch.Tensor | None = None,
                 dtype=torch.float64) -> dict:
    """lib_read, xenc/d18_library.py:34-96: the reader rows' query / gate / own key and value from
    the interface's projections (:41-49), the RoPE rotations at relative positions P + t and
    N_d + P + t (:50-55, :68-70), the core above, then o_proj(o * sigmoid(gate)) and B (:93-96).
    Evaluated in `dtype` (fp64 by default)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb
    att = itf.att[str(li)]
    hd = att.head_dim
    with torch.no_grad():
        xe = itf.map_x(li, x)
        T = xe.shape[0]
        qh, gate = torch.chunk(att.q_proj(xe).view(T, -1, hd * 2), 2, dim=-1)
        gate = gate.reshape(T, -1)
        q = att.q_norm(qh).transpose(0, 1)
        k = att.k_norm(att.k_proj(xe).view(T, -1, hd)).transpose(0, 1)
        v = att.v_proj(xe).view(T, -1, hd).transpose(0, 1)
        Hq, Hkv = q.shape[0], k.shape[0]
        G = Hq // Hkv
        P = 0 if past is None else past[0].shape[1]
        rel = torch.arange(P, P + T)

        def rope(pos):
            cos, sin = itf.rot(xe.unsqueeze(0), pos.view(1, 1, -1).expand(3, 1, -1))
            return cos.float(), sin.float()

        cos, sin = rope(rel)
        qo, ko = apply_rotary_pos_emb(q.unsqueeze(0), k.unsqueeze(0), cos, sin)
        qo, ko = qo[0], ko[0]
        Kown = ko if past is None else torch.cat([past[0], ko], 1)
        Vown = v if past is None else torch.cat([past[1], v], 1)
        qd = []
        for K, _ in ops:
            cos, sin = rope(rel + K.shape[1])
            qd.append(apply_rotary_pos_emb(q.unsqueeze(0), k.unsqueeze(0), cos, sin)[0][0])
        core = d18_core(torch.stack(qd).view(len(ops), Hkv, G, T, hd).to(dtype), qo.view(Hkv, G, T, hd).to(dtype),
                        [(K.to(dtype), V.to(dtype)) for K, V in ops], Kown.to(dtype), Vown.to(dtype), P,
                        att.scaling, skip, beta, top_k, force, wfix)
        o = att.o_proj((core["o"] * torch.sigmoid(gate.to(dtype))).float())
        return {"y": itf.Bmap(li, o), "o": o, "w": core["w"], "past": (Kown, Vown), "r": core["r"],
                "rmax": core["rmax"], "n": core["n"]}


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("math", "torch", "annotations")]
