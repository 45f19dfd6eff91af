"""DecodeReader: the serving-side joint decode read (op B) on the HIP kernel `joint_read_kernel`.

Same constructor and call signature as xenc/d23_read_kernels.py:134-160:

    dec = DecodeReader(max_n, hq, hkv, d, max_keys, device, chunk=1024, block_n=64)
    out = dec(q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, scale)   # fp32 [N, hq, d]

For each query row n and query head, one softmax over the operator's rows (paged pool op_k/op_v,
block table op_bt[n], op_len[n] rows) joined with the request's own rows (own_k/own_v, own_bt[n],
own_len[n]).  Pools are [num_blocks, block_size, hkv, d] in bf16 or fp16.

Like the reference, the reader owns a static workspace sized at construction and returns a view
of its own output buffer (callers clone it if they keep it across calls).  A call allocates
nothing, reads no device value on the host and synchronises nothing, so it can be captured in a
HIP graph and replayed with new lengths / block tables.  `block_n` is accepted for signature
compatibility (it sized the reference's key tile); the HIP kernel picks its own tiling.
"""

from __future__ import annotations

import math

import torch

from ._lib import check, lib, ptr, stream_handle

_DTYPES = {torch.float16: 0, torch.bfloat16: 1}


class DecodeReader:
    def __init__(self, max_n: int, hq: int, hkv: int, d: int, max_keys: int, device, chunk: int = 1024,
                 block_n: int = 64):
        if hq % hkv:
            raise ValueError(f"hq={hq} must be a multiple of hkv={hkv}")
        self.G, self.hq, self.hkv, self.d = hq // hkv, int(hq), int(hkv), int(d)
        if not 1 <= self.G <= 8 or d % 8 or d > 512 or self.G * d > 4096:
            raise ValueError(f"unsupported head layout: G={self.G} (1..8), d={d} (multiple of 8, <= 512)")
        self.max_n, self.chunk, self.block_n = int(max_n), int(chunk), int(block_n)
        self.S = max(1, math.ceil(max_keys / self.chunk))
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("DecodeReader runs only on a ROCm GPU (there is no CPU path)")
        L = lib()
        nbytes = L.xenc_joint_workspace_bytes(self.max_n, self.hkv, self.S, self.G, self.d)
        self.workspace = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        check(L.xenc_joint_workspace_init(ptr(self.workspace), self.workspace.numel(), self.max_n, self.hkv,
                                          stream_handle(device)), "xenc_joint_workspace_init")
        self.out = torch.empty(self.max_n, self.hq, self.d, dtype=torch.float32, device=device)
        self.device = device

    @staticmethod
    def _pool(k: torch.Tensor, v: torch.Tensor, name: str):
        if k.dim() != 4 or k.shape != v.shape or k.stride() != v.stride() or k.dtype != v.dtype:
            raise ValueError(f"{name} K and V pools must be [num_blocks, block_size, hkv, d] with equal "
                             "shapes, strides and dtypes")
        if k.stride(-1) != 1:
            raise ValueError(f"{name} pools need a contiguous last dim")
        return k.stride(0), k.stride(1), k.stride(2), k.shape[1]

    @staticmethod
    def _table(bt: torch.Tensor, ln: torch.Tensor, N: int, name: str):
        if bt.dtype != torch.int32 or bt.dim() != 2 or bt.shape[0] < N or bt.stride(1) != 1:
            raise ValueError(f"{name}_bt must be int32 [>= N, max_blocks] with contiguous rows")
        if ln.dtype != torch.int32 or ln.dim() != 1 or ln.shape[0] < N or ln.stride(0) != 1:
            raise ValueError(f"{name}_len must be a contiguous int32 [>= N] tensor")
        return bt.stride(0)

    def __call__(self, q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, scale):
        N = q.shape[0]
        if N > self.max_n or q.shape[1:] != (self.hq, self.d):
            raise ValueError(f"q must be [N <= {self.max_n}, {self.hq}, {self.d}], got {tuple(q.shape)}")
        for t, nm in ((q, "q"), (op_k, "op_k"), (own_k, "own_k"), (op_bt, "op_bt"), (own_bt, "own_bt")):
            if not t.is_cuda or t.device != self.device:
                raise RuntimeError(f"{nm} must be on {self.device} (there is no CPU path)")
        if op_k.dtype not in _DTYPES or own_k.dtype != op_k.dtype:
            raise ValueError("pools must both be fp16 or both bf16")
        if op_k.shape[2:] != (self.hkv, self.d) or own_k.shape[2:] != (self.hkv, self.d):
            raise ValueError(f"pools must be [num_blocks, block_size, {self.hkv}, {self.d}]")
        osb, oss, osh, obs = self._pool(op_k, op_v, "operator")
        wsb, wss, wsh, wbs = self._pool(own_k, own_v, "own")
        obt = self._table(op_bt, op_len, N, "op")
        wbt = self._table(own_bt, own_len, N, "own")
        if q.dtype != op_k.dtype:
            q = q.to(op_k.dtype)
        if q.stride(-1) != 1:
            q = q.contiguous()
        out = self.out[:N]
        if N == 0:
            return out
        rc = lib().xenc_paged_decode_joint(
            _DTYPES[op_k.dtype], N, self.hq, self.hkv, self.d, ptr(q), q.stride(0), q.stride(1),
            ptr(op_k), ptr(op_v), osb, oss, osh, obs, ptr(op_bt), obt, ptr(op_len),
            ptr(own_k), ptr(own_v), wsb, wss, wsh, wbs, ptr(own_bt), wbt, ptr(own_len),
            float(scale), self.S, self.chunk, ptr(out), out.stride(0), out.stride(1),
            ptr(self.workspace), self.workspace.numel(), self.max_n, stream_handle(self.device))
        check(rc, "xenc_paged_decode_joint")
        return out


__all__ = ["DecodeReader"]
