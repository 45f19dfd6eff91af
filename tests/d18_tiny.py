"""A small interface object with the attributes lib_read uses (xenc/d18_library.py:34-96;
D13Interface, xenc/d13_read.py:40-60, 162-182): per paired reader layer a frozen fp32 Qwen3.5
attention (gated q_proj, q/k RMSNorm, partial RoPE), the rotary embedding, map_x (A) and Bmap (B),
random-initialised from a seed.  Encoder operators are synthetic post-RoPE keys / values."""

from __future__ import annotations

import torch
from torch import nn

LAYERS = (1, 5)


class TinyItf(nn.Module):
    def __init__(self, d_r=64, d_e=48, heads=4, kv_heads=2, head_dim=32, seed=0):
        super().__init__()
        from transformers.models.qwen3_5 import modeling_qwen3_5 as M
        from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
        torch.manual_seed(seed)
        cfg = Qwen3_5TextConfig(hidden_size=d_e, num_attention_heads=heads, num_key_value_heads=kv_heads,
                                head_dim=head_dim, intermediate_size=64, num_hidden_layers=2, vocab_size=128)
        self.layers = list(LAYERS)
        self.layer_map = {li: li for li in LAYERS}
        self.att = nn.ModuleDict({str(li): M.Qwen3_5Attention(cfg, layer_idx=1).float().requires_grad_(False)
                                  for li in LAYERS})
        self.rot = M.Qwen3_5TextRotaryEmbedding(cfg).float()
        self.A = nn.ModuleDict({str(li): nn.Linear(d_r, d_e) for li in LAYERS})
        self.B = nn.ModuleDict({str(li): nn.Linear(d_e, d_r) for li in LAYERS})
        self.g = {li: 0.5 for li in LAYERS}
        for p in self.parameters():
            p.requires_grad_(False)

    def map_x(self, li, x):
        return self.A[str(li)](x)

    def Bmap(self, li, o):
        return self.B[str(li)](o)

    def gate(self, li):
        return self.g[li]


def operators(itf: TinyItf, lengths, seed=1, dtype=torch.float32):
    """One synthetic operator per length: [(K, V) [Hkv, N, hd]] (keys unit-scale like a post-norm,
    post-RoPE encoder key)."""
    att = itf.att[str(itf.layers[0])]
    hkv = att.k_proj.out_features // att.head_dim
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(hkv, n, att.head_dim, generator=g).to(dtype),
             torch.randn(hkv, n, att.head_dim, generator=g).to(dtype)) for n in lengths]
