"""GPU: op B (DecodeReader, the joint operator + own-rows decode read) against the oracle's
decode_read_ref, as tests/test_d23_kernels.py:51-82 does for the reference kernel: bf16 pools,
hq=16 / hkv=4 / d=256 / block 16, three cases up to long operators crossing many splits and
pages, relative error < 2e-3, then graph capture and replay with halved operator lengths.  Plus
fp16, other GQA widths and head sizes, empty rows, and a reused workspace at varying N."""

from __future__ import annotations

import pytest
import torch

import oracle as O
from kv_skill_v2_amd.decode_reader import DecodeReader

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _case(N, hq, hkv, d, bs, nb_op, nb_own, seed, dtype, op_blocks=10, own_blocks=3, op_len=None,
          own_len=None):
    g = torch.Generator().manual_seed(seed)
    op_k, op_v = (torch.randn(nb_op, bs, hkv, d, generator=g).to(dtype) for _ in range(2))
    own_k, own_v = (torch.randn(nb_own, bs, hkv, d, generator=g).to(dtype) for _ in range(2))
    q = torch.randn(N, hq, d, generator=g).to(dtype)
    if op_len is None:
        op_len = ([13, 1, 37] + [5] * N)[:N]
    if own_len is None:
        own_len = ([3, 9, 1] + [2] * N)[:N]
    op_bt = torch.stack([torch.randperm(nb_op, generator=g)[:op_blocks] for _ in range(N)]).int()
    own_bt = torch.stack([torch.randperm(nb_own, generator=g)[:own_blocks] for _ in range(N)]).int()
    return [q, op_k, op_v, op_bt, torch.tensor(op_len, dtype=torch.int32), own_k, own_v, own_bt,
            torch.tensor(own_len, dtype=torch.int32)]


def _rel(out, ref):
    return float((out.double().cpu() - ref.double()).norm() / ref.double().norm().clamp_min(1e-30))


def _ref(args, scale):
    return O.decode_read_ref(*[a.cpu() for a in args], scale)


CASES = [(1, 40, 0), (3, 40, 1), (8, 300, 2)]


@pytest.mark.parametrize("N,nb_op,seed", CASES)
def test_decode_reader_matches_reference_and_replays(dev, N, nb_op, seed):
    say("op B", dict(N=N, nb_op=nb_op, seed=seed))
    kw = {}
    if N == 8:   # long operators crossing many splits / pages
        kw = dict(op_blocks=200, own_blocks=30, op_len=[3200, 1, 17, 2048, 1024, 1023, 15, 3199],
                  own_len=[1, 480, 33, 64, 2, 5, 300, 17])
    args = _case(N, 16, 4, 256, 16, nb_op, 40, seed, torch.bfloat16, **kw)
    dargs = [a.to(dev) for a in args]
    dec = DecodeReader(16, 16, 4, 256, max_keys=4096, device=dev, chunk=512)
    out = dec(*dargs, 0.0625).clone()
    ref = _ref(args, 0.0625)
    assert _rel(out, ref) < 2e-3, _rel(out, ref)
    # graph capture + replay with updated lengths
    gph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec(*dargs, 0.0625)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(gph):
        o_g = dec(*dargs, 0.0625)
    dargs[4].copy_(torch.clamp(dargs[4] // 2, min=1))
    for _ in range(3):
        gph.replay()
        torch.cuda.synchronize()
        args2 = list(args)
        args2[4] = dargs[4].cpu()
        assert _rel(o_g, _ref(args2, 0.0625)) < 2e-3


@pytest.mark.parametrize("hq,hkv,d,dtype", [(16, 16, 128, torch.float16), (8, 4, 64, torch.bfloat16),
                                            (32, 4, 128, torch.bfloat16), (12, 4, 80, torch.float16),
                                            (8, 1, 512, torch.float16), (16, 8, 256, torch.float16),
                                            (16, 2, 256, torch.bfloat16), (6, 2, 128, torch.bfloat16)])
def test_decode_reader_layouts(dev, hq, hkv, d, dtype):
    say("op B layout", dict(hq=hq, hkv=hkv, d=d, dtype=str(dtype)))
    args = _case(5, hq, hkv, d, 8, 64, 24, 7, dtype, op_blocks=40, own_blocks=10,
                 op_len=[300, 0, 64, 1, 257], own_len=[5, 40, 0, 1, 80])
    dec = DecodeReader(8, hq, hkv, d, max_keys=512, device=dev, chunk=128)
    out = dec(*[a.to(dev) for a in args], 1.0 / d ** 0.5)
    ref = _ref(args, 1.0 / d ** 0.5)
    assert _rel(out, ref) < 2e-3, _rel(out, ref)


def _rel_rows(out, ref):
    """Largest relative error over the (row, query head) vectors with a nonzero reference; rows
    with no keys must read exactly 0."""
    out, ref = out.double().cpu(), ref.double()
    nrm = ref.norm(dim=-1)
    live = nrm > 0
    if bool((~live).any()):
        assert float(out[~live].abs().max()) == 0.0
    return float(((out - ref).norm(dim=-1)[live] / nrm[live]).max())


@pytest.mark.parametrize("op_bs,own_bs", [(12, 16), (16, 12), (12, 12), (16, 8)])
@pytest.mark.parametrize("hq,hkv,d,dtype", [(8, 2, 64, torch.bfloat16), (16, 4, 128, torch.float16),
                                            (16, 4, 256, torch.bfloat16)])
def test_decode_reader_block_sizes_per_row(dev, op_bs, own_bs, hq, hkv, d, dtype):
    """Operator and own pools with different block sizes, including ones that are not powers of
    two (the division path of the key lookup), on the VALU form (d = 64) and the MFMA form
    (d = 128, 256); every (row, head) output within rel 2e-3 of the oracle on its own."""
    say("op B block sizes", dict(op_bs=op_bs, own_bs=own_bs, hq=hq, hkv=hkv, d=d, dtype=str(dtype)))
    g = torch.Generator().manual_seed(op_bs * 100 + own_bs + d)
    N = 6
    op_len, own_len = [300, 0, 12, 1, 257, 131], [5, 40, 0, 1, 80, 13]
    nb_op, nb_own = 64, 40
    op_k, op_v = (torch.randn(nb_op, op_bs, hkv, d, generator=g).to(dtype) for _ in range(2))
    own_k, own_v = (torch.randn(nb_own, own_bs, hkv, d, generator=g).to(dtype) for _ in range(2))
    q = torch.randn(N, hq, d, generator=g).to(dtype)
    op_bt = torch.stack([torch.randperm(nb_op, generator=g)[:-(-max(op_len) // op_bs)] for _ in range(N)]).int()
    own_bt = torch.stack([torch.randperm(nb_own, generator=g)[:-(-max(own_len) // own_bs)] for _ in range(N)]).int()
    args = [q, op_k, op_v, op_bt, torch.tensor(op_len, dtype=torch.int32), own_k, own_v, own_bt,
            torch.tensor(own_len, dtype=torch.int32)]
    for chunk in (64, 1024):
        dec = DecodeReader(8, hq, hkv, d, max_keys=max(a + b for a, b in zip(op_len, own_len)), device=dev,
                           chunk=chunk)
        out = dec(*[a.to(dev) for a in args], 1.0 / d ** 0.5)
        ref = _ref(args, 1.0 / d ** 0.5)
        err = _rel_rows(out, ref)
        assert err < 2e-3, (chunk, err)


def test_decode_reader_empty_rows_and_reuse(dev):
    """A row with no keys reads 0; one workspace serves calls of different N in any order; keys
    past nsplit * chunk are still read (the last split takes them)."""
    say("op B empty rows / reuse")
    dec = DecodeReader(6, 8, 2, 64, max_keys=256, device=dev, chunk=64)
    for N, seed in ((6, 1), (2, 2), (5, 3), (6, 4)):
        args = _case(N, 8, 2, 64, 16, 40, 20, seed, torch.bfloat16, op_blocks=30, own_blocks=5,
                     op_len=([0, 400, 3, 0, 256, 64] * 2)[:N], own_len=([0, 7, 0, 1, 60, 64] * 2)[:N])
        out = dec(*[a.to(dev) for a in args], 0.125)
        ref = _ref(args, 0.125)
        if N >= 1:
            assert float(out[0].abs().max()) == 0.0      # op_len = own_len = 0
        assert _rel(out, ref) < 2e-3, (N, _rel(out, ref))


def test_decode_reader_is_deterministic(dev):
    say("op B determinism")
    args = [a.to(dev) for a in _case(4, 16, 4, 128, 16, 200, 20, 9, torch.bfloat16, op_blocks=150,
                                     own_blocks=6, op_len=[2300, 700, 5, 1999], own_len=[3, 90, 1, 40])]
    dec = DecodeReader(4, 16, 4, 128, max_keys=2400, device=dev, chunk=256)
    a = dec(*args, 0.09).clone()
    for _ in range(3):
        assert torch.equal(dec(*args, 0.09), a)


def test_decode_reader_rejects_bad_inputs(dev):
    """Bad shapes, tables, dtypes and devices raise errors that are both this build's types
    (ValueError / RuntimeError) and the reference's (AssertionError: its __call__ asserts its
    preconditions, xenc/d23_read_kernels.py:146-150)."""
    say("op B guards")
    with pytest.raises(ValueError):
        DecodeReader(4, 36, 4, 64, 128, dev)          # G = 9
    with pytest.raises(AssertionError):
        DecodeReader(4, 16, 4, 60, 128, dev)          # d % 8
    dec = DecodeReader(2, 8, 2, 64, 128, dev)
    args = [a.to(dev) for a in _case(3, 8, 2, 64, 16, 10, 10, 0, torch.bfloat16, op_blocks=4, own_blocks=4)]
    for exc in (ValueError, AssertionError):
        with pytest.raises(exc):
            dec(*args, 0.1)                            # N above max_n
    args = [a.to(dev) for a in _case(2, 8, 2, 64, 16, 10, 10, 0, torch.bfloat16, op_blocks=4, own_blocks=4)]
    bad = list(args)
    bad[4] = bad[4].long()
    for exc in (ValueError, AssertionError):
        with pytest.raises(exc):
            dec(*bad, 0.1)
    bad = list(args)
    bad[2] = bad[2].half()
    for exc in (ValueError, AssertionError):
        with pytest.raises(exc):
            dec(*bad, 0.1)
    bad = list(args)
    bad[5] = bad[5][:, :8]                             # own K and V pools of different shapes
    with pytest.raises(AssertionError):
        dec(*bad, 0.1)
    bad = list(args)
    bad[0] = bad[0].cpu()                              # q on the host
    for exc in (RuntimeError, AssertionError):
        with pytest.raises(exc):
            dec(*bad, 0.1)


def test_decode_reader_zero_rows(dev):
    say("op B zero rows")
    dec = DecodeReader(4, 8, 2, 64, max_keys=128, device=dev)
    args = [a.to(dev) for a in _case(1, 8, 2, 64, 16, 10, 10, 0, torch.bfloat16, op_blocks=4, own_blocks=4)]
    args[0] = args[0][:0]
    out = dec(*args, 0.1)
    assert out.shape == (0, 8, 64)
