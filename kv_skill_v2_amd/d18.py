"""D18: a library of D documents' operators read by the reader's own query in one pass
(xenc/d18_library.py).  The API is the reference's: lib_read, D18LibReader, route_stats,
question_route, ROUTE_AGGS.  The interface's projections, the RoPE rotations and o_proj / B stay
in torch as in the reference; the per-document read, the route logits and the routing softmax
(xenc/d18_library.py:63-90) run on HIP (ops.d18_read → xenc_d18_read), one launch pair for all
documents instead of a Python loop over them.  Forward only, as the reference evaluates D18 under
no_grad.  The BM25 retriever of the RAG baselines (xenc/d18_library.py:159-228) is not part of
the read path and is not provided here."""

from __future__ import annotations

import types

import torch

from . import ops as _ops
from .depth import decoder_layers


def lib_read(itf, li: int, x: torch.Tensor, ops, past=None, skip: int = 0, beta: float = 1.0,
             top_k: int = 0, force: int | None = None, wfix: torch.Tensor | None = None) -> dict:
    """x [T, d_r] fp32 reader rows; ops = [(K_d, V_d) [Hkv, N_d, hd] post-RoPE at 0..N_d-1] for
    this layer (or ops.d18_pack of them); past = (K_own, V_own) own earlier rows rotated at relative
    positions 0..P-1.  -> {"y" [T, d_r], "o" [T, d_e], "w" [Hkv, G, T, D], "past", "r", "rmax", "n"}.
    Same signature and results as xenc/d18_library.py:34-96."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb
    packed = _ops.d18_pack(ops)
    att = itf.att[str(li)]
    hd = att.head_dim
    xe = itf.map_x(li, x)
    T = xe.shape[0]
    qh, gate = torch.chunk(att.q_proj(xe).view(T, -1, hd * 2), 2, dim=-1)
    gate = gate.reshape(T, -1)
    q = att.q_norm(qh).transpose(0, 1)                                   # [Hq, T, hd] (unrotated)
    k = att.k_norm(att.k_proj(xe).view(T, -1, hd)).transpose(0, 1)       # [Hkv, T, hd]
    v = att.v_proj(xe).view(T, -1, hd).transpose(0, 1)
    P = 0 if past is None else past[0].shape[1]
    rel = torch.arange(P, P + T, device=xe.device)

    def rope(pos):
        cos, sin = itf.rot(xe.unsqueeze(0), pos.view(1, 1, -1).expand(3, 1, -1))
        return cos.float(), sin.float()

    cos, sin = rope(rel)
    qo, ko = apply_rotary_pos_emb(q.unsqueeze(0), k.unsqueeze(0), cos, sin)
    qo, ko = qo[0], ko[0]
    Kown = ko if past is None else torch.cat([past[0], ko], 1)
    Vown = v if past is None else torch.cat([past[1], v], 1)
    # One rotation per distinct document length (documents of equal length share it).
    by_len = {}
    for n in packed.lengths:
        if n not in by_len:
            c, s = rope(rel + n)
            by_len[n] = apply_rotary_pos_emb(q.unsqueeze(0), k.unsqueeze(0), c, s)[0][0]
    qd = torch.stack([by_len[n] for n in packed.lengths])                # [D, Hq, T, hd]
    core = _ops.d18_read(qd, qo, packed, Kown, Vown, att.scaling, skip, beta, top_k, force, wfix)
    o = att.o_proj(core["o"].to(gate.dtype) * torch.sigmoid(gate))
    return {"y": itf.Bmap(li, o), "o": o, "w": core["w"], "past": (Kown.detach(), Vown.detach()),
            "r": core["r"], "rmax": core["rmax"], "n": core["n"]}


class D18LibReader:
    """Patches the reader's attention at itf.layers (xenc/d18_library.py:99-157).  mode "off"
    (stock) | "lib" (the library read replaces the attention output, gated own + g * (read - own)).
    load(ops, skip) takes {enc_layer: [(K, V), ...]}; the operators of each layer are packed once
    there for the HIP read."""

    def __init__(self, model, itf):
        self.model, self.itf = model, itf
        L = decoder_layers(model)
        self.mods = {li: L[li].self_attn for li in itf.layers}
        self.mode = "off"
        self.ops: dict = {}
        self.skip, self.beta, self.top_k, self.force = 0, 1.0, 0, None
        self.wfix = None
        self.past: dict = {}
        self.route: dict = {}
        self.route_rows: dict = {}
        self.logit_rows: dict = {}
        self._packed: dict = {}
        self._orig = {}
        for li, m in self.mods.items():
            self._orig[li] = m.forward
            m.forward = types.MethodType(_lib_forward(self, li), m)

    def load(self, ops: dict, skip: int = 0):
        self.ops, self.skip, self.past, self.route, self.route_rows = ops, int(skip), {}, {}, {}
        self.logit_rows = {}
        self._packed = {en: _ops.d18_pack(lst) for en, lst in ops.items()}

    def reset(self):
        self.past, self.route, self.route_rows, self.logit_rows = {}, {}, {}, {}

    def detach(self):
        for li, f in self._orig.items():
            self.mods[li].forward = f
        self._orig.clear()


def _lib_forward(R: D18LibReader, li: int):
    def forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kwargs):
        out, w = type(self).forward(self, hidden_states, position_embeddings, attention_mask,
                                    past_key_values=past_key_values, **kwargs)
        if R.mode == "off":
            return out, w
        itf = R.itf
        en = itf.layer_map[li]
        res = lib_read(itf, li, hidden_states[0].float(), R._packed.get(en, R.ops[en]), past=R.past.get(li),
                       skip=R.skip, beta=R.beta, top_k=R.top_k, force=R.force, wfix=R.wfix)
        R.past[li] = res["past"]
        R.route[li] = res["w"][:, :, -1].detach()
        if res["w"].shape[2] > 1:
            R.route_rows[li] = res["w"].detach()
            R.logit_rows[li] = (res["r"], res["rmax"], res["n"])
        g = itf.gate(li)
        y = out[0].float() + g * (res["y"] - out[0].float())
        return y.to(out.dtype).unsqueeze(0), w

    return forward


def route_stats(route: dict, gold: int) -> dict:
    """{li: [Hkv, G, D]} -> mass on gold (mean over layers / heads), argmax of the mean route ==
    gold, per-layer mass (xenc/d18_library.py:160-169)."""
    if not route:
        return {}
    W = torch.stack([w.detach().float().reshape(-1, w.shape[-1]).mean(0) for w in route.values()])
    mean = W.mean(0)
    return {"gold_mass": float(mean[gold]), "top1": float(int(mean.argmax()) == gold),
            "layer_mass": {str(li): float(w.float().reshape(-1, w.shape[-1]).mean(0)[gold]) for li, w in route.items()},
            "chance": 1.0 / W.shape[-1]}


ROUTE_AGGS = ("lse_norm", "lse", "max")


def question_route(logit_rows: dict, rows: slice) -> dict:
    """Question-level routing from one prefill (xenc/d18_library.py:175-191): per aggregator the
    route score of every document averaged over the given reader rows, all heads and layers.
    lse_norm = logsumexp(s_d) - log N_d, lse = logsumexp(s_d), max = max_c s_d,c."""
    out = {k: [] for k in ROUTE_AGGS}
    for r, rm, n in logit_rows.values():
        rr, mm = r[:, :, rows].float(), rm[:, :, rows].float()
        out["lse"].append(rr.mean((0, 1, 2)))
        out["lse_norm"].append((rr - n.log()).mean((0, 1, 2)))
        out["max"].append(mm.mean((0, 1, 2)))
    return {k: torch.stack(v).mean(0) for k, v in out.items() if v}


__all__ = ["lib_read", "D18LibReader", "route_stats", "question_route", "ROUTE_AGGS"]
