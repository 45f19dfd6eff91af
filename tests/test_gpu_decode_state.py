"""GPU: the op-B serving step on the device (xenc_decode_step + xenc_own_rows_write + the joint
read), the counterpart of the plugin's per-step host fill and own-row writes
(xenc/d23_vllm_plugin.py:241-264, 433-457, 486-487).  Several requests decode step after step
from ONE captured graph: every step's tables equal the ones built on the host the plugin's way,
and every step's output matches the oracle decode_read_ref over the accumulated own rows
(relative error < 2e-3, the bar of tests/test_d23_kernels.py:51-82).  A request leaving and a
new one entering its slot mid-run, a padded row, and a slot running past its own-row capacity."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd.decode_reader import DecodeReader, DecodeState

pytestmark = pytest.mark.gpu

BS, HQ, HKV, D = 16, 16, 4, 128
NB_OP, DUMMY = 40, 39
DOCS = {"A": (0, 150), "B": (10, 230), "C": (25, 70)}     # (first block, tokens)


def say(*a):
    print("[case]", *a, flush=True)


class Mirror:
    """The host-side bookkeeping of the plugin (stage_step / Static.fill) and a CPU copy of the
    own pool, built independently of the device state."""

    def __init__(self, n_slots, own_blocks):
        self.own_blocks, self.cap = own_blocks, own_blocks * BS
        self.doc, self.pos = {}, {}
        self.own_k = torch.zeros(n_slots * own_blocks, BS, HKV, D)
        self.own_v = torch.zeros_like(self.own_k)

    def tables(self, rows, max_op_blocks, k_new, v_new):
        N = len(rows)
        op_bt = torch.full((N, max_op_blocks), DUMMY, dtype=torch.int32)
        own_bt = torch.zeros(N, self.own_blocks, dtype=torch.int32)
        op_len, own_len = torch.zeros(N, dtype=torch.int32), torch.zeros(N, dtype=torch.int32)
        wpos = torch.full((N,), -1, dtype=torch.int64)
        for i, s in enumerate(rows):
            if s < 0:
                continue
            start, tok = self.doc[s]
            nblk = -(-tok // BS)
            op_bt[i, :nblk] = torch.arange(start, start + nblk, dtype=torch.int32)
            op_len[i] = tok
            own_bt[i] = torch.arange(s * self.own_blocks, (s + 1) * self.own_blocks, dtype=torch.int32)
            p0 = self.pos[s]
            if p0 < self.cap:
                wpos[i] = s * self.cap + p0
                b, o = divmod(int(wpos[i]), BS)
                self.own_k[b, o] = k_new[i].float()
                self.own_v[b, o] = v_new[i].float()
                self.pos[s] = p0 + 1
            own_len[i] = self.pos[s]
        return op_bt, op_len, own_bt, own_len, wpos


def _run(dev, own_blocks, schedule, n_steps, seed, change=None):
    g = torch.Generator().manual_seed(seed)
    op_k = torch.randn(NB_OP, BS, HKV, D, generator=g).bfloat16()
    op_v = torch.randn(NB_OP, BS, HKV, D, generator=g).bfloat16()
    op_k[DUMMY] = 0
    op_v[DUMMY] = 0
    n_slots, max_n, max_op_blocks = 4, len(schedule), 16
    own_k = torch.zeros(n_slots * own_blocks, BS, HKV, D, dtype=torch.bfloat16, device=dev)
    own_v = torch.zeros_like(own_k)
    op_kd, op_vd = op_k.to(dev), op_v.to(dev)
    st = DecodeState(max_n, n_slots, own_blocks, BS, max_op_blocks, DUMMY, dev)
    mir = Mirror(n_slots, own_blocks)
    rows = list(schedule)
    for s in rows:
        if s >= 0:
            name = "ABC"[s % 3]
            st.admit(s, *DOCS[name])
            mir.doc[s], mir.pos[s] = DOCS[name], 0
    st.set_rows(rows)
    reader = DecodeReader(max_n, HQ, HKV, D, max_keys=max_op_blocks * BS + own_blocks * BS, device=dev, chunk=128)
    q = torch.zeros(max_n, HQ, D, dtype=torch.bfloat16, device=dev)
    k_new = torch.zeros(max_n, HKV, D, dtype=torch.bfloat16, device=dev)
    v_new = torch.zeros_like(k_new)
    scale = D ** -0.5

    def device_step():
        st.step()
        st.write_own(k_new, v_new, own_k, own_v)
        return reader(q, op_kd, op_vd, st.op_bt, st.op_len, own_k, own_v, st.own_bt, st.own_len, scale)

    gph, out = None, None
    for t in range(n_steps):
        if change is not None and t == change[0]:
            s, name = change[1], change[2]
            st.release(s)
            st.admit(s, *DOCS[name])
            mir.doc[s], mir.pos[s] = DOCS[name], 0
        qc = torch.randn(max_n, HQ, D, generator=g).bfloat16()
        kc = torch.randn(max_n, HKV, D, generator=g).bfloat16()
        vc = torch.randn(max_n, HKV, D, generator=g).bfloat16()
        q.copy_(qc)
        k_new.copy_(kc)
        v_new.copy_(vc)
        if t == 0:                            # eager first step (also the warm-up), then capture
            res = device_step().clone()
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                out = device_step()
        else:
            gph.replay()
            res = out.clone()
        torch.cuda.synchronize()
        op_bt, op_len, own_bt, own_len, wpos = mir.tables(rows, max_op_blocks, kc, vc)
        assert torch.equal(st.op_bt.cpu(), op_bt) and torch.equal(st.op_len.cpu(), op_len), t
        assert torch.equal(st.own_bt.cpu(), own_bt) and torch.equal(st.own_len.cpu(), own_len), t
        assert torch.equal(st.write_pos.cpu(), wpos), t
        ref = O.decode_read_ref(qc, op_k, op_v, op_bt, op_len, mir.own_k, mir.own_v, own_bt, own_len, scale)
        rel = float((res.double().cpu() - ref.double()).norm() / ref.double().norm().clamp_min(1e-30))
        assert rel < 2e-3, (t, rel)
        for i, s in enumerate(rows):
            if s < 0:
                assert float(res[i].abs().max()) == 0.0
    return st


def test_decode_steps_replay_from_one_graph(dev):
    say("op B serving steps", dict(rows=[0, 2, -1, 3], steps=12))
    _run(dev, own_blocks=4, schedule=[0, 2, -1, 3], n_steps=12, seed=1)


def test_slot_change_mid_run(dev):
    """Slot 2's request leaves after 5 steps and a request on document C takes the slot (own rows
    start over); the captured graph keeps serving."""
    say("op B slot change")
    _run(dev, own_blocks=4, schedule=[2, 0, 1], n_steps=10, seed=2, change=(5, 2, "C"))


def test_own_capacity_reached(dev):
    """One own block (16 rows) and 20 steps: past the capacity the step stops writing and the read
    keeps the 16 rows."""
    say("op B own capacity")
    st = _run(dev, own_blocks=1, schedule=[1, 3], n_steps=20, seed=3)
    assert st.own_rows(1) == 16 and st.own_rows(3) == 16


def test_decode_state_guards(dev):
    say("op B state guards")
    st = DecodeState(4, 2, 2, 16, 8, 0, dev)
    with pytest.raises(ValueError):
        st.admit(2, 0, 10)                     # slot out of range
    with pytest.raises(ValueError):
        st.admit(0, 0, 8 * 16 + 1)             # more operator blocks than max_op_blocks
    with pytest.raises(ValueError):
        st.set_rows([0, 0])                    # a slot twice
    with pytest.raises(ValueError):
        st.set_rows([0, 1, -1, -1, -1])        # more rows than max_n
    own = torch.zeros(2, 16, 4, 64, dtype=torch.bfloat16, device=dev)   # needs 4 blocks
    st.set_rows([0])
    with pytest.raises(ValueError):
        st.write_own(torch.zeros(1, 4, 64, dtype=torch.bfloat16, device=dev),
                     torch.zeros(1, 4, 64, dtype=torch.bfloat16, device=dev), own, own.clone())
