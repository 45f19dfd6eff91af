"""The C-ABI library loads on a GPU-less host and exports every entry point include/*.h declares
(no compute calls here)."""

from __future__ import annotations

import re

from conftest import ROOT


def _declared() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(xenc_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert {"xenc_route_topk", "xenc_library_read_decode", "xenc_strerror"} <= names, names


def test_library_exports_every_declared_symbol():
    from kv_skill_v2_amd import _lib
    L = _lib.lib()
    for name in sorted(_declared()):
        assert hasattr(L, name), f"{name} declared in include/ but not exported by {_lib.LIB_PATH}"
    assert L.xenc_abi_version() == _lib.ABI_VERSION


def test_binding_covers_header():
    from kv_skill_v2_amd import _lib
    assert _declared() == set(_lib.SIGNATURES), "ctypes signatures and include/*.h disagree"


def test_error_codes_and_size_queries():
    from kv_skill_v2_amd import _lib
    L = _lib.lib()
    assert L.xenc_strerror(0) == b"ok"
    assert b"aligned" in L.xenc_strerror(-3)
    units = 64 * 8 * 4
    assert L.xenc_decode_workspace_bytes(64, 8, 4, 2048) >= units * 2048 * 4 + units * 8
    assert L.xenc_decode_workspace_bytes(0, 8, 4, 2048) == 0


def test_host_side_validation_rejects_bad_sizes():
    """Argument checks run on the host before any launch: safe without a GPU."""
    from kv_skill_v2_amd import _lib
    L = _lib.lib()
    # d not a multiple of 8
    assert L.xenc_route_topk(None, 12, 1, 12, None, None, None, 1, 2, 10.0, None, 4, None, None, 2, None) == -1
    # NULL pointers with valid sizes
    assert L.xenc_route_topk(None, 16, 1, 16, None, None, None, 1, 2, 10.0, None, 4, None, None, 2, None) == -2
    assert L.xenc_library_read_decode(None, 16, 1, 16, None, 4, 64, None, None, None, None, 1, None, None, 2,
                                      12.0, 1, 1, None, 16, None, 0, 1, None) == -2
    # nsplit out of range
    assert L.xenc_library_read_decode(None, 16, 1, 16, None, 4, 64, None, None, None, None, 1, None, None, 2,
                                      12.0, 1, 65, None, 16, None, 0, 1, None) == -1
    # more rows than the workspace capacity
    assert L.xenc_library_read_decode(None, 16, 2, 16, None, 4, 64, None, None, None, None, 1, None, None, 2,
                                      12.0, 1, 1, None, 16, None, 0, 1, None) == -4
    # op B: G = hq / hkv above 8, d not a multiple of 8, NULL pointers, N above the capacity
    args = dict(dtype=1, N=1, hq=16, hkv=4, d=64)

    def joint(**kw):
        a = {**args, **kw}
        return L.xenc_paged_decode_joint(a["dtype"], a["N"], a["hq"], a["hkv"], a["d"], None, 16 * 64, 64,
                                         None, None, a.get("op_sb", 64 * 4 * 16), 64 * 4, 64, 16, None, 8, None,
                                         None, None, 64 * 4 * 16, 64 * 4, 64, 16, None, 8, None,
                                         0.125, 2, 512, None, 16 * 64, 64, None, 0, a.get("max_n", 4), None)
    assert joint(hq=36, hkv=4) == -1
    assert joint(op_sb=1 << 31) == -1        # a pool block of 2^31 elements or more
    assert joint(d=60) == -1
    assert joint(dtype=2) == -1
    assert joint() == -2
    assert joint(N=5) == -4
    assert L.xenc_joint_workspace_bytes(4, 4, 2, 4, 64) >= 4 * 4 * 2 * 4 * 64 * 4
    # the prefill backward's readout with the routing term: d not a multiple of 64, NULL pointers,
    # a dl row shorter than the chunk count, dl rows too long for 32-bit tile offsets, no tiles

    def routed(**kw):
        a = dict(G=1, n_tiles=1, d=64, cmax=2, ldl=2)
        a.update(kw)
        return L.xenc_prefill_readout_routed(None, 4, None, None, a["G"], a["n_tiles"], None, 64, a["d"], 64 * 64,
                                             None, None, None, 2, None, 2, None, 0, None, a["cmax"], 10.0, None,
                                             a["ldl"], None, 64, None)
    assert routed(d=60) == -1
    assert routed() == -2
    assert routed(ldl=1) == -1
    assert routed(ldl=1 << 25) == -1
    assert routed(n_tiles=0) == 0
    # the fp32 -> fp16 row cast: d not a multiple of 8, a row stride below d or not a multiple
    # of 4, no rows, NULL pointers, and (fake, never dereferenced) pointers off 16-byte alignment
    cast = L.xenc_cast_rows_f16
    assert cast(None, 16, 4, 12, None, None) == -1
    assert cast(None, 8, 4, 16, None, None) == -1
    assert cast(None, 18, 4, 16, None, None) == -1
    assert cast(None, 16, -1, 16, None, None) == -1
    assert cast(None, 16, 0, 16, None, None) == 0
    assert cast(None, 16, 4, 16, None, None) == -2
    assert cast(0x1004, 16, 4, 16, 0x2000, None) == -3
    assert cast(0x1000, 16, 4, 16, 0x2008, None) == -3


def test_cpp_operators_registered():
    """libxenc_torch.so loads on a GPU-less host and defines the per-token operators in torch's
    dispatcher with a device (HIP) kernel, plus the fake kernels registered from Python."""
    import torch

    from kv_skill_v2_amd import torch_ops
    assert torch_ops.TORCH_OPS_PATH.exists()
    for name in ("route_topk", "library_read", "route_read", "paged_decode_joint"):
        op = getattr(torch.ops.xenc, name).default
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA"), name
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Meta"), name
    schema = str(torch.ops.xenc.route_read.default._schema)
    assert "Tensor(a!) workspace" in schema and schema.endswith("-> (Tensor, Tensor, Tensor, Tensor)")


def test_python_operators_registered():
    """The many-row operators (torch.library.custom_op in kv_skill_v2_amd.torch_ops) are in the
    dispatcher with fake kernels, and the differentiable ones carry registered autograd."""
    import torch

    from kv_skill_v2_amd import torch_ops  # noqa: F401
    names = ("route_rows", "route_backward_", "library_prefill_fwd", "library_prefill_lse", "library_prefill_bwd_dq",
             "library_prefill_bwd_routed", "library_read_routed")
    for name in names:
        op = getattr(torch.ops.xenc, name).default
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Meta"), name
    for name in ("route_rows", "library_prefill_fwd", "library_read_routed"):
        op = getattr(torch.ops.xenc, name).default
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Autograd"), name
    schema = str(torch.ops.xenc.library_read_routed.default._schema)
    assert schema.endswith("-> (Tensor, Tensor, Tensor, Tensor, Tensor)"), schema
