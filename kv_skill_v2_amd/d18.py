"""D18: a library of D documents' operators read by the reader's own query in one pass
(the API of xenc/d18_library.py: lib_read, D18LibReader).

Per paired reader layer the reader rows are mapped into the encoder's space (itf.map_x), the
encoder's frozen attention gives their query, gate, key and value (`_project`), and the queries
are rotated once for the own rows (positions P + t) and once per distinct document length
(positions N_d + P + t).  The attention core — every document's keys joined with the own rows in
one softmax, the route logits r_d = logsumexp of a document's scores past `skip`, the routing
softmax over documents (top-k with ties to the lower index, a forced document or fixed weights)
and the route-weighted sum — runs on HIP (ops.d18_read -> xenc_d18_read), one launch pair for all
documents.  The gate, o_proj and B stay in torch.  Forward only: the reference evaluates D18
under no_grad.  The BM25 retriever of the reference's RAG baselines is not part of the read.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops as _ops
from .depth import decoder_layers


@dataclass
class _Rows:
    """The reader rows seen by one paired layer's frozen encoder attention (unrotated)."""
    xe: torch.Tensor      # [T, d_e] rows in the encoder's space
    q: torch.Tensor       # [Hq, T, hd] after q_norm
    k: torch.Tensor       # [Hkv, T, hd] after k_norm
    v: torch.Tensor       # [Hkv, T, hd]
    gate: torch.Tensor    # [T, Hq * hd]


def _project(itf, li: int, x: torch.Tensor) -> _Rows:
    att = itf.att[str(li)]
    hd = att.head_dim
    xe = itf.map_x(li, x)
    T = xe.shape[0]
    qg = att.q_proj(xe).view(T, -1, 2 * hd)                   # query and gate, interleaved per head
    q = att.q_norm(qg[..., :hd]).transpose(0, 1)
    k = att.k_norm(att.k_proj(xe).view(T, -1, hd)).transpose(0, 1)
    v = att.v_proj(xe).view(T, -1, hd).transpose(0, 1)
    return _Rows(xe, q, k, v, qg[..., hd:].reshape(T, -1))


def _rotated(itf, rows: _Rows, positions: torch.Tensor):
    """(q, k) rotated to the given absolute positions [T]."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb
    cos, sin = itf.rot(rows.xe[None], positions.view(1, 1, -1).expand(3, 1, -1))
    q, k = apply_rotary_pos_emb(rows.q[None], rows.k[None], cos.float(), sin.float())
    return q[0], k[0]


def lib_read(itf, li: int, x: torch.Tensor, ops, past=None, skip: int = 0, beta: float = 1.0,
             top_k: int = 0, force: int | None = None, wfix: torch.Tensor | None = None) -> dict:
    """x [T, d_r] fp32 reader rows; ops = [(K_d, V_d) [Hkv, N_d, hd] rotated at 0..N_d-1] for this
    layer (or ops.d18_pack of them); past = (K_own, V_own) earlier own rows rotated at 0..P-1.
    -> {"y" [T, d_r], "o" [T, d_e], "w" [Hkv, G, T, D], "past", "r", "rmax", "n"}, the results of
    xenc/d18_library.py:34-96."""
    packed = _ops.d18_pack(ops)
    att = itf.att[str(li)]
    rows = _project(itf, li, x)
    T = rows.xe.shape[0]
    P = 0 if past is None else past[0].shape[1]
    here = torch.arange(P, P + T, device=rows.xe.device)
    q_own, k_new = _rotated(itf, rows, here)
    K_own = k_new if past is None else torch.cat([past[0], k_new], 1)
    V_own = rows.v if past is None else torch.cat([past[1], rows.v], 1)
    per_length = {n: _rotated(itf, rows, here + n)[0] for n in sorted(set(packed.lengths))}
    q_docs = torch.stack([per_length[n] for n in packed.lengths])          # [D, Hq, T, hd]
    core = _ops.d18_read(q_docs, q_own, packed, K_own, V_own, att.scaling, skip, beta, top_k, force, wfix)
    o = att.o_proj(core["o"].to(rows.gate.dtype) * torch.sigmoid(rows.gate))
    return {"y": itf.Bmap(li, o), "o": o, "w": core["w"], "past": (K_own.detach(), V_own.detach()),
            "r": core["r"], "rmax": core["rmax"], "n": core["n"]}


class _LibraryAttention:
    """Replacement forward of one patched attention module: the stock attention, then (mode
    "lib") own + g * (read - own) with the library read of the same rows."""

    def __init__(self, reader: "D18LibReader", li: int, module):
        self.reader, self.li, self.module = reader, li, module

    def __call__(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kwargs):
        mod = self.module
        out, attn_w = type(mod).forward(mod, hidden_states, position_embeddings, attention_mask,
                                        past_key_values=past_key_values, **kwargs)
        R = self.reader
        if R.mode == "off":
            return out, attn_w
        li = self.li
        enc = R.itf.layer_map[li]
        res = lib_read(R.itf, li, hidden_states[0].float(), R._packed.get(enc, R.ops[enc]), past=R.past.get(li),
                       skip=R.skip, beta=R.beta, top_k=R.top_k, force=R.force, wfix=R.wfix)
        R.past[li] = res["past"]
        R.route[li] = res["w"][:, :, -1].detach()
        if res["w"].shape[2] > 1:
            R.route_rows[li] = res["w"].detach()
            R.logit_rows[li] = (res["r"], res["rmax"], res["n"])
        own = out[0].float()
        mixed = own + R.itf.gate(li) * (res["y"] - own)
        return mixed.to(out.dtype)[None], attn_w


class D18LibReader:
    """Patches the reader's attention at itf.layers.  mode "off" (stock) | "lib" (the library
    read replaces the attention output, gated own + g * (read - own)).  load(ops, skip) takes
    {encoder layer: [(K, V), ...]}; each layer's operators are packed once there."""

    def __init__(self, model, itf):
        self.model, self.itf = model, itf
        blocks = decoder_layers(model)
        self.mods = {li: blocks[li].self_attn for li in itf.layers}
        self.mode = "off"
        self.ops: dict = {}
        self.skip, self.beta, self.top_k, self.force = 0, 1.0, 0, None
        self.wfix = None
        self._packed: dict = {}
        self.reset()
        for li, m in self.mods.items():
            m.forward = _LibraryAttention(self, li, m)     # instance attribute over the class method

    def load(self, ops: dict, skip: int = 0):
        self.ops, self.skip = ops, int(skip)
        self._packed = {enc: _ops.d18_pack(lst) for enc, lst in ops.items()}
        self.reset()

    def reset(self):
        """Forget the own rows and the recorded routes (a new sequence)."""
        self.past, self.route, self.route_rows, self.logit_rows = {}, {}, {}, {}

    def detach(self):
        for m in self.mods.values():
            if isinstance(m.__dict__.get("forward"), _LibraryAttention):
                del m.forward
        self.mods = {}


__all__ = ["lib_read", "D18LibReader"]
