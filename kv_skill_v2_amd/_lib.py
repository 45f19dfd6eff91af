"""ctypes binding of libxenc_hip.so (the C ABI declared in include/xenc_hip.h).

The library is loaded after torch so that it binds to the HIP runtime torch already loaded
(both carry the SONAME libamdhip64.so.7).  There is no fallback: if the library is missing or
was built for another ABI version, every call raises.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int, c_longlong, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must be loaded first: shares its HIP runtime with the library)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libxenc_hip.so"
ABI_VERSION = 18

_lock = threading.Lock()
_lib = None

# name -> (restype, argtypes)
SIGNATURES = {
    "xenc_strerror": (ctypes.c_char_p, [c_int]),
    "xenc_last_hip_error": (c_int, []),
    "xenc_abi_version": (c_int, []),
    "xenc_route_topk": (c_int, [
        c_void_p, c_longlong, c_int, c_int,          # q, ldq, M, d
        c_void_p, c_void_p, c_void_p, c_int,         # S, chunk_ptr, q_group, G
        c_int, c_float,                              # top_k, route_temp
        c_void_p, c_longlong, c_void_p, c_void_p, c_int,  # w_dense, ldw, idx, w_sel, kk
        c_void_p]),                                  # stream
    "xenc_route_topk_rows": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_void_p,  # q, ldq, M, d, S
        c_void_p, c_void_p, c_void_p, c_int, c_int,  # chunk_ptr, row_ptr, tile_ptr, G, n_tiles
        c_int, c_float, c_void_p, c_longlong,        # top_k, route_temp, w_dense, ldw
        c_void_p, c_void_p, c_int, c_void_p, c_void_p]),       # idx, w_sel, kk, stream
    "xenc_decode_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "xenc_decode_workspace_init": (c_int, [c_void_p, c_size_t, c_int, c_void_p]),
    "xenc_library_read_decode": (c_int, [
        c_void_p, c_longlong, c_int, c_int,          # q, ldq, M, d
        c_void_p, c_int, c_longlong,                 # pages, slots_per_page, page_stride
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,  # chunk_page, chunk_nvalid, chunk_ptr, q_group, G
        c_void_p, c_void_p, c_int,                   # idx, w_sel, kk
        c_float, c_int, c_int,                       # read_temp, softmax, nsplit
        c_void_p, c_longlong,                        # r, ldr
        c_void_p, c_size_t, c_int, c_void_p]),       # workspace, bytes, max_rows, stream
    "xenc_route_read_decode": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_void_p,  # q, ldq, M, d, S
        c_void_p, c_int, c_longlong,                 # pages, slots_per_page, page_stride
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,  # chunk_page, chunk_nvalid, chunk_ptr, q_group, G
        c_int, c_float, c_void_p, c_longlong,        # top_k, route_temp, w_dense, ldw
        c_void_p, c_void_p, c_int,                   # idx, w_sel, kk
        c_float, c_int, c_int,                       # read_temp, softmax, nsplit
        c_void_p, c_longlong,                        # r, ldr
        c_void_p, c_size_t, c_int, c_void_p]),       # workspace, bytes, max_rows, stream
    "xenc_library_read_decode_noalloc": (c_int, [
        c_void_p, c_longlong, c_int, c_int,          # q, ldq, M, d
        c_void_p, c_int, c_longlong,                 # pages, slots_per_page, page_stride
        c_void_p, c_void_p, c_void_p, c_void_p, c_int,  # chunk_page, chunk_nvalid, chunk_ptr, q_group, G
        c_void_p, c_void_p, c_int,                   # idx, w_sel, kk
        c_float, c_int, c_int,                       # read_temp, softmax, nsplit
        c_void_p, c_longlong, c_void_p]),            # r, ldr, stream
    "xenc_calibrate_mfma": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "xenc_calibrate_stream": (c_int, [c_void_p, c_longlong, c_int, c_void_p, c_void_p]),
    "xenc_cast_rows_f16": (c_int, [c_void_p, c_longlong, c_int, c_int, c_void_p, c_void_p]),
    "xenc_fragment_pages": (c_int, [c_void_p, c_longlong, c_int, c_int, c_int, c_void_p, c_void_p]),
    "xenc_build_pages": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_void_p,
                                 c_longlong, c_void_p, c_longlong, c_void_p, c_void_p]),
    "xenc_write_back": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_void_p, c_int,  # r, ldr, M, d, row_group, G
        c_void_p, c_longlong, c_longlong, c_int,     # W, w_group_stride, ldw, d_out
        c_void_p, c_longlong, c_void_p,              # bias, bias_group_stride, row_scale
        c_void_p, c_longlong, c_void_p]),            # out, ldo, stream
    "xenc_prefill_scores": (c_int, [
        c_int, c_void_p, c_int, c_void_p, c_void_p,  # mode, x, d, row_ptr, tile_ptr
        c_int, c_int, c_void_p, c_int, c_longlong,   # G, n_tiles, pages_a, slots_per_page, page_stride
        c_void_p, c_void_p, c_void_p, c_float,       # chunk_ptr, chunk_page, chunk_nvalid, temp
        c_void_p, c_longlong, c_void_p, c_longlong,  # w, ldw, p, p_rows
        c_void_p, c_void_p, c_longlong, c_void_p]),  # ds, gamma, ldg, stream
    "xenc_prefill_readout": (c_int, [
        c_void_p, c_longlong, c_void_p, c_void_p,    # a, a_rows, row_ptr, tile_ptr
        c_int, c_int, c_void_p, c_int, c_int,        # G, n_tiles, pages_b, slots_per_page, d
        c_longlong, c_void_p, c_void_p,              # page_stride, chunk_ptr, chunk_page
        c_void_p, c_longlong, c_void_p, c_longlong, c_void_p]),  # w, ldw, out, ldo, stream
    "xenc_joint_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "xenc_joint_workspace_init": (c_int, [c_void_p, c_size_t, c_int, c_int, c_void_p]),
    "xenc_paged_decode_joint": (c_int, [
        c_int, c_int, c_int, c_int, c_int,           # dtype, N, hq, hkv, d
        c_void_p, c_longlong, c_longlong,            # q, s_qn, s_qh
        c_void_p, c_void_p, c_longlong, c_longlong, c_longlong, c_int,  # op_k, op_v, strides, bs
        c_void_p, c_longlong, c_void_p,              # op_bt, op_bt_stride, op_len
        c_void_p, c_void_p, c_longlong, c_longlong, c_longlong, c_int,  # own_k, own_v, strides, bs
        c_void_p, c_longlong, c_void_p,              # own_bt, own_bt_stride, own_len
        c_float, c_int, c_int,                       # scale, nsplit, chunk
        c_void_p, c_longlong, c_longlong,            # out, s_on, s_oh
        c_void_p, c_size_t, c_int, c_void_p]),       # workspace, bytes, max_n, stream
    "xenc_selector_weights": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_int,   # z, ldz, B, n, k
        c_void_p, c_longlong, c_void_p, c_void_p, c_longlong, c_void_p]),  # w, ldw, idx, w_sel, ld, stream
    "xenc_selector_apply": (c_int, [
        c_int, c_int, c_int, c_void_p, c_longlong,   # B, k, d, delta, ldd
        c_void_p, c_longlong, c_void_p, c_void_p,    # h, ldh, w_row, log_alpha (device scalar)
        c_void_p, c_longlong, c_void_p]),            # out, ldo, stream
    "xenc_gate_scale": (c_int, [
        c_int, c_int, c_void_p, c_longlong, c_void_p, c_void_p, c_int,  # M, d, hn, ldh, row_token, row_pos, n_pos
        c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p]),    # gate_w, gate_b, log_gain, gain_scale, scale, stream
    "xenc_multi_depth_prepare": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_int,   # z, ldz, B, n, k
        c_void_p, c_longlong, c_longlong, c_int,     # q_all, q_depth_stride, q_token_stride, d
        c_void_p, c_longlong, c_int,                 # hn, ldh, d_r
        c_void_p, c_void_p, c_void_p, c_float,       # gate_w, gate_b, log_gain, gain_scale
        c_void_p, c_longlong, c_void_p, c_void_p, c_longlong,  # w, ldw, idx, w_sel, ld_sel
        c_void_p, c_longlong, c_void_p, c_void_p]),  # q_rows, ldr, scale, stream
    "xenc_multi_depth_prepare_route": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_int,   # z, ldz, B, n, k
        c_void_p, c_longlong, c_longlong, c_int,     # q_all, q_depth_stride, q_token_stride, d
        c_void_p, c_longlong, c_int,                 # hn, ldh, d_r
        c_void_p, c_void_p, c_void_p, c_float,       # gate_w, gate_b, log_gain, gain_scale
        c_void_p, c_longlong, c_void_p, c_void_p, c_longlong,  # w, ldw, idx, w_sel, ld_sel
        c_void_p, c_longlong, c_void_p,              # q_rows, ldr, scale
        c_void_p, c_void_p, c_int, c_int, c_float,   # S, chunk_ptr, G, top_k, route_temp
        c_void_p, c_longlong, c_void_p, c_void_p, c_int,  # w_dense, ldwd, ridx, rw_sel, kk
        c_void_p]),                                  # stream
    "xenc_select_scores": (c_int, [
        c_void_p, c_int, c_int, c_int, c_int,        # q, B, n_q, n_kv, hd
        c_void_p, c_int, c_void_p, c_int,            # keys, S, valid, pool_mean
        c_void_p, c_longlong, c_void_p]),            # scores, ld_s, stream
    "xenc_topk_rows": (c_int, [
        c_void_p, c_longlong, c_int, c_int, c_int,   # scores, ld_s, B, S, k
        c_void_p, c_void_p, c_longlong, c_void_p]),  # idx, vals, ld_o, stream
    "xenc_d18_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "xenc_d18_read": (c_int, [
        c_int, c_int, c_int, c_int, c_int, c_int,    # dtype, T, hq, hkv, hd, n_docs
        c_void_p, c_void_p,                          # qd, qo
        c_void_p, c_void_p, c_longlong, c_longlong, c_void_p,  # k_docs, v_docs, s_dh, s_dn, doc_ptr
        c_void_p, c_void_p, c_longlong, c_longlong, c_int,     # k_own, v_own, s_oh, s_on, P
        c_float, c_int, c_float, c_int, c_int, c_void_p, c_int,  # scale, skip, beta, top_k, force, wfix, nsplit
        c_void_p, c_void_p, c_void_p, c_void_p,      # out, w, r, rmax
        c_void_p, c_size_t, c_void_p]),              # workspace, workspace_bytes, stream
    "xenc_gather_pages": (c_int, [
        c_void_p, c_int, c_longlong, c_int,          # pages, slots_per_page, page_stride, d
        c_void_p, c_int, c_int, c_void_p, c_longlong,  # chunk_page, n_chunks, n_flat, idx, ld_idx
        c_int, c_int, c_int, c_void_p, c_void_p]),   # G, k, kpad, out, stream
    "xenc_decode_step": (c_int, [
        c_int, c_void_p, c_void_p, c_int, c_int,     # N, row_slot, slots, n_slots, own_blocks
        c_int, c_int, c_int, c_void_p, c_longlong,   # block_size, max_op_blocks, dummy_block, op_bt, ld
        c_void_p, c_void_p, c_longlong, c_void_p,    # op_len, own_bt, ld, own_len
        c_void_p, c_void_p]),                        # write_pos, stream
    "xenc_own_rows_write": (c_int, [
        c_int, c_int, c_int, c_void_p, c_void_p,     # N, hkv, d, k_new, v_new
        c_longlong, c_longlong, c_void_p, c_void_p,  # s_n, s_h, own_k, own_v
        c_longlong, c_longlong, c_longlong, c_int,   # sb, ss, sh, block_size
        c_void_p, c_void_p]),                        # write_pos, stream
    "xenc_route_backward": (c_int, [
        c_void_p, c_longlong, c_void_p, c_longlong,  # w, ldw, dw_read, ldr
        c_void_p, c_longlong, c_void_p, c_void_p,    # dw_ext, lde, row_ptr, tile_ptr
        c_int, c_int, c_int, c_void_p, c_void_p,     # G, n_tiles, cmax, S, chunk_ptr
        c_int, c_float, c_void_p, c_longlong, c_void_p]),  # d, route_temp, dq, ldq, stream
    "xenc_prefill_readout_routed": (c_int, [
        c_void_p, c_longlong, c_void_p, c_void_p,    # ds, a_rows, row_ptr, tile_ptr
        c_int, c_int, c_void_p, c_int, c_int,        # G, n_tiles, pages_b, slots_per_page, d
        c_longlong, c_void_p, c_void_p,              # page_stride, chunk_ptr, chunk_page
        c_void_p, c_longlong, c_void_p, c_longlong,  # w, ldw, dw_read, ldr
        c_void_p, c_longlong, c_void_p, c_int,       # dw_ext, lde, S, cmax
        c_float, c_void_p, c_longlong,               # route_temp, dl, ldl
        c_void_p, c_longlong, c_void_p]),            # dq, ldq, stream
}


class XencError(RuntimeError):
    pass


def lib():
    """The loaded library (loads on first use; raises if it is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise XencError(f"{LIB_PATH} is not built: run kv_skill_v2_amd._build.build() "
                                "(the Library read has no CPU path)")
            handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
            got = handle.xenc_abi_version()
            if got != ABI_VERSION:
                raise XencError(f"{LIB_PATH} has ABI version {got}, expected {ABI_VERSION}: rebuild it")
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    L = lib()
    msg = L.xenc_strerror(rc).decode()
    if rc == -5:
        msg += f" (hipError {L.xenc_last_hip_error()})"
    if rc in (-1, -2, -3, -4, -6):
        raise ValueError(f"{what}: {msg}")
    raise XencError(f"{what}: {msg}")


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on `device` (0 = the null stream)."""
    return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())


def _raw_stream_api(index: int) -> int:
    return torch.cuda.current_stream(index).cuda_stream


# torch's own accessor of the raw current stream (what its Triton launcher uses) skips building a
# Stream object per call; the public API is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or _raw_stream_api


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
