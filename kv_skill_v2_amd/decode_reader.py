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
compatibility (it sized the reference's key tile); the HIP kernel picks its own tiling.  `chunk`
(keys per split) keeps the reference's meaning and default (1024); chunk=None, an addition of this
build, chooses it from max_n, hkv and max_keys for about 1024 workgroups at full capacity (faster
at small batches: 37 against 48 us for one row over 16k keys).  The split only changes the order
of the LSE merge, not what is computed.
"""

from __future__ import annotations

import math

import torch

from . import torch_ops  # noqa: F401  (registers torch.ops.xenc.paged_decode_joint)
from ._lib import check, lib, ptr, stream_handle

_DTYPES = {torch.float16: 0, torch.bfloat16: 1}


class DecodeReaderError(ValueError, AssertionError):
    """A DecodeReader argument that does not fit the reader: a bad pool, table, shape or dtype.
    The reference checks its call preconditions with `assert` (xenc/d23_read_kernels.py:146-150),
    so callers written against it catch AssertionError; callers of this build catch ValueError.
    Both work."""


class DecodeReaderDeviceError(RuntimeError, AssertionError):
    """A DecodeReader tensor that is not on the reader's GPU (there is no CPU path).  The
    reference asserts `q.is_cuda` (xenc/d23_read_kernels.py:146), hence AssertionError too."""


class DecodeReader:
    def __init__(self, max_n: int, hq: int, hkv: int, d: int, max_keys: int, device, chunk: int | None = 1024,
                 block_n: int = 64):
        if hq % hkv:
            raise DecodeReaderError(f"hq={hq} must be a multiple of hkv={hkv}")
        self.G, self.hq, self.hkv, self.d = hq // hkv, int(hq), int(hkv), int(d)
        if not 1 <= self.G <= 8 or d % 8 or d > 512 or self.G * d > 4096:
            raise DecodeReaderError(f"unsupported head layout: G={self.G} (1..8), d={d} (multiple of 8, <= 512)")
        device = torch.device(device)
        if device.type != "cuda":
            raise DecodeReaderDeviceError("DecodeReader runs only on a ROCm GPU (there is no CPU path)")
        if chunk is None:
            cus = torch.cuda.get_device_properties(device).multi_processor_count
            chunk = self.auto_chunk(max_n, hkv, max_keys, cus)
        self.max_n, self.chunk, self.block_n = int(max_n), int(chunk), int(block_n)
        self.S = max(1, math.ceil(max_keys / self.chunk))
        L = lib()
        nbytes = L.xenc_joint_workspace_bytes(self.max_n, self.hkv, self.S, self.G, self.d)
        self.workspace = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        check(L.xenc_joint_workspace_init(ptr(self.workspace), self.workspace.numel(), self.max_n, self.hkv,
                                          stream_handle(device)), "xenc_joint_workspace_init")
        self.out = torch.empty(self.max_n, self.hq, self.d, dtype=torch.float32, device=device)
        self.device = device

    @staticmethod
    def auto_chunk(max_n: int, hkv: int, max_keys: int, cus: int = 256) -> int:
        """Keys per split: as many splits as keep a full-capacity launch (max_n rows x hkv heads x
        splits) at one workgroup per CU at most, with at least 512 keys per split, a multiple of 64
        (the MFMA read's 16-key tiles over 4 waves).  At hkv 4 and 16,448 keys on 256 CUs (hq 16,
        d 256, bf16; the wall clock of 50 calls, three runs each): 32 rows get 8,256 keys (256
        workgroups, 321 us against 326 us at 512 workgroups, 332 us at 1,024 and 362 us at 384),
        8 rows 2,112 (90 us against 94 us at 512 and 105 us at 928), 4 rows 1,088 (54 us against
        61 us at 464), one row 512 (132 workgroups, 35-36 us against 37 us at 172 and 39 us at
        208).  Workgroup counts that do not divide evenly over the CUs leave a ragged last round."""
        units = max(1, int(max_n) * int(hkv))
        splits = max(1, int(cus) // units)
        chunk = max(512, -(-int(max_keys) // splits))
        return -(-chunk // 64) * 64

    @staticmethod
    def _pool(k: torch.Tensor, v: torch.Tensor, name: str):
        if k.dim() != 4 or k.shape != v.shape or k.stride() != v.stride() or k.dtype != v.dtype:
            raise DecodeReaderError(f"{name} K and V pools must be [num_blocks, block_size, hkv, d] with equal "
                             "shapes, strides and dtypes")
        if k.stride(-1) != 1:
            raise DecodeReaderError(f"{name} pools need a contiguous last dim")
        return k.stride(0), k.stride(1), k.stride(2), k.shape[1]

    @staticmethod
    def _table(bt: torch.Tensor, ln: torch.Tensor, N: int, name: str):
        if bt.dtype != torch.int32 or bt.dim() != 2 or bt.shape[0] < N or bt.stride(1) != 1:
            raise DecodeReaderError(f"{name}_bt must be int32 [>= N, max_blocks] with contiguous rows")
        if ln.dtype != torch.int32 or ln.dim() != 1 or ln.shape[0] < N or ln.stride(0) != 1:
            raise DecodeReaderError(f"{name}_len must be a contiguous int32 [>= N] tensor")
        return bt.stride(0)

    def __call__(self, q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, scale):
        N = q.shape[0]
        if N > self.max_n or q.shape[1:] != (self.hq, self.d):
            raise DecodeReaderError(f"q must be [N <= {self.max_n}, {self.hq}, {self.d}], got {tuple(q.shape)}")
        for t, nm in ((q, "q"), (op_k, "op_k"), (own_k, "own_k"), (op_bt, "op_bt"), (own_bt, "own_bt")):
            if not t.is_cuda or t.device != self.device:
                raise DecodeReaderDeviceError(f"{nm} must be on {self.device} (there is no CPU path)")
        if op_k.dtype not in _DTYPES or own_k.dtype != op_k.dtype:
            raise DecodeReaderError("pools must both be fp16 or both bf16")
        if op_k.shape[2:] != (self.hkv, self.d) or own_k.shape[2:] != (self.hkv, self.d):
            raise DecodeReaderError(f"pools must be [num_blocks, block_size, {self.hkv}, {self.d}]")
        self._pool(op_k, op_v, "operator")
        self._pool(own_k, own_v, "own")
        self._table(op_bt, op_len, N, "op")
        self._table(own_bt, own_len, N, "own")
        if q.dtype != op_k.dtype:
            q = q.to(op_k.dtype)
        if q.stride(-1) != 1:
            q = q.contiguous()
        out = self.out[:N]
        if N == 0:
            return out
        torch.ops.xenc.paged_decode_joint(q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, float(scale),
                                          self.S, self.chunk, self.workspace, self.max_n, out)
        return out


class DecodeState:
    """Device-resident decode state of the op-B serving step: per request slot {operator start
    block, operator tokens, own rows so far} and per step row the slot it decodes.  `step()`
    (xenc_decode_step) advances every live row's own position and writes the block tables and
    lengths of the joint read into static buffers; `write_own()` (xenc_own_rows_write) puts the
    step's new K/V rows into the own pool.  The reference rebuilds the same tables on the host and
    copies them to the device each step (Static.fill and stage_step,
    xenc/d23_vllm_plugin.py:241-264, 433-457); here the host only writes when a request is admitted
    or released or the rows change, so a whole decode step (step, write_own, DecodeReader) can be
    captured once and replayed.

        st = DecodeState(max_n, n_slots, own_blocks, block, max_op_blocks, dummy_block, device)
        st.admit(slot, op_start_block, op_tokens); st.set_rows([slot, ...])
        st.step(); st.write_own(k_new, v_new, own_k, own_v)
        out = reader(q, op_k, op_v, st.op_bt, st.op_len, own_k, own_v, st.own_bt, st.own_len, scale)

    Slot s owns own-pool blocks [s * own_blocks, (s + 1) * own_blocks); the own pool needs at
    least n_slots * own_blocks blocks.  Padded rows (slot -1) read nothing and write nothing."""

    def __init__(self, max_n: int, n_slots: int, own_blocks: int, block_size: int, max_op_blocks: int,
                 dummy_block: int, device):
        device = torch.device(device)
        if device.type != "cuda":
            raise DecodeReaderDeviceError("DecodeState lives on a ROCm GPU (there is no CPU path)")
        if min(max_n, n_slots, own_blocks, block_size, max_op_blocks) < 1 or dummy_block < 0:
            raise ValueError("sizes must be >= 1 and dummy_block >= 0")
        self.max_n, self.n_slots, self.own_blocks = int(max_n), int(n_slots), int(own_blocks)
        self.block_size, self.max_op_blocks, self.dummy_block = int(block_size), int(max_op_blocks), int(dummy_block)
        self.device = device
        i32 = dict(dtype=torch.int32, device=device)
        self.slots = torch.zeros(self.n_slots, 4, **i32)
        self.row_slot = torch.full((self.max_n,), -1, **i32)
        self.op_bt = torch.full((self.max_n, self.max_op_blocks), self.dummy_block, **i32)
        self.op_len = torch.zeros(self.max_n, **i32)
        self.own_bt = torch.zeros(self.max_n, self.own_blocks, **i32)
        self.own_len = torch.zeros(self.max_n, **i32)
        self.write_pos = torch.full((self.max_n,), -1, dtype=torch.int64, device=device)
        self.n = 0

    def admit(self, slot: int, op_start: int, op_tokens: int, own_len: int = 0) -> None:
        """A request enters `slot`: its document operator is op_tokens rows in the operator pool's
        blocks op_start.. (contiguous, as the plugin's static pool lays documents out)."""
        if not 0 <= slot < self.n_slots:
            raise ValueError(f"slot {slot} outside [0, {self.n_slots})")
        if op_tokens < 0 or -(-op_tokens // self.block_size) > self.max_op_blocks:
            raise ValueError(f"op_tokens={op_tokens} needs more than max_op_blocks={self.max_op_blocks} blocks")
        if not 0 <= own_len <= self.own_blocks * self.block_size:
            raise ValueError("own_len outside the slot's own rows")
        self.slots[slot].copy_(torch.tensor([op_start, op_tokens, own_len, 0], dtype=torch.int32))

    def release(self, slot: int) -> None:
        self.slots[slot].zero_()

    def set_rows(self, slots) -> None:
        """Rows of the coming steps: row i decodes slot slots[i] (-1 = padded); each slot at most
        once."""
        slots = [int(x) for x in slots]
        if len(slots) > self.max_n:
            raise ValueError(f"{len(slots)} rows > max_n={self.max_n}")
        live = [x for x in slots if x >= 0]
        if len(set(live)) != len(live) or any(x >= self.n_slots for x in live):
            raise ValueError("each row's slot must be distinct and < n_slots")
        self.row_slot.fill_(-1)
        if slots:
            self.row_slot[:len(slots)].copy_(torch.tensor(slots, dtype=torch.int32))
        self.n = len(slots)

    def own_rows(self, slot: int) -> int:
        """Own rows written so far for `slot` (reads the device state: a synchronising call)."""
        return int(self.slots[slot, 2])

    def step(self, N: int | None = None) -> None:
        N = self.n if N is None else int(N)
        check(lib().xenc_decode_step(N, ptr(self.row_slot), ptr(self.slots), self.n_slots, self.own_blocks,
                                     self.block_size, self.max_op_blocks, self.dummy_block, ptr(self.op_bt),
                                     self.op_bt.stride(0), ptr(self.op_len), ptr(self.own_bt),
                                     self.own_bt.stride(0), ptr(self.own_len), ptr(self.write_pos),
                                     stream_handle(self.device)), "xenc_decode_step")

    def write_own(self, k_new: torch.Tensor, v_new: torch.Tensor, own_k: torch.Tensor, own_v: torch.Tensor,
                  N: int | None = None) -> None:
        """Write the step's new rows k_new / v_new [N, hkv, d] at the positions step() assigned."""
        N = self.n if N is None else int(N)
        if k_new.shape != v_new.shape or k_new.stride() != v_new.stride() or k_new.dim() != 3:
            raise ValueError("k_new and v_new must be [N, hkv, d] with equal strides")
        if k_new.shape[0] < N or k_new.stride(-1) != 1:
            raise ValueError("k_new must hold >= N rows with a contiguous last dim")
        sb, ss, sh, bs = DecodeReader._pool(own_k, own_v, "own")
        if bs != self.block_size or own_k.shape[0] < self.n_slots * self.own_blocks:
            raise ValueError(f"own pool must have block size {self.block_size} and >= "
                             f"{self.n_slots * self.own_blocks} blocks")
        if own_k.shape[2:] != k_new.shape[1:] or own_k.dtype != k_new.dtype or own_k.element_size() != 2:
            raise ValueError("new rows must match the own pool's [hkv, d] and 2-byte dtype")
        check(lib().xenc_own_rows_write(N, k_new.shape[1], k_new.shape[2], ptr(k_new), ptr(v_new),
                                        k_new.stride(0), k_new.stride(1), ptr(own_k), ptr(own_v), sb, ss, sh,
                                        bs, ptr(self.write_pos), stream_handle(self.device)),
              "xenc_own_rows_write")


__all__ = ["DecodeReader", "DecodeState"]
