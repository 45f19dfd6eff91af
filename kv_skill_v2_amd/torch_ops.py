"""The Library-read boundary as operators in torch's dispatcher (namespace `xenc`).

Each operator is a thin call through the C ABI of libxenc_hip.so (include/xenc_hip.h) on torch's
current stream; every tensor argument is a plain device tensor and every size an int, so the
dispatcher, FakeTensor tracing and torch.compile see ordinary operators:

    xenc::route_topk             routing of few rows: q . S, top-k (ties to the lower chunk),
                                 softmax -> (w [M, cmax], idx [M, kk] int32, w_sel [M, kk])
                                 (LibraryInjector.route, xenc/injector.py:220-229)
    xenc::library_read           paged split-K read of the routed pages -> r [M, d]; writes its
                                 workspace (the read of LibraryInjector._branch,
                                 xenc/injector.py:236-265)
    xenc::route_read             both of the above in one call (the top-k inside the read kernel
                                 when every library has at most 64 chunks)
    xenc::route_rows             routing of many rows grouped by library (fp32 MFMA tiles), also
                                 emitting the rows as fp16; differentiable in q
    xenc::library_prefill_lse    per (row, chunk) log-sum-exp of the read's scores (the join of the
                                 sub-pages of pages longer than 512 slots)
    xenc::library_prefill_fwd    the MFMA read of many rows -> (r [M, d], p); differentiable in q
                                 and w (its backward is the next operator plus the route term)
    xenc::library_prefill_bwd_dq (dq through the read, gamma = dL/dw) from the upstream gradient
    xenc::route_backward_        dq += the routing term, in place
    xenc::library_prefill_bwd_routed  dq through the read and the routing in one pass over dq
    xenc::library_read_routed    route_rows + library_prefill_fwd as one autograd node (its
                                 backward is library_prefill_bwd_routed)
    xenc::paged_decode_joint     DecodeReader's joint read (xenc/d23_read_kernels.py:145-160) into
                                 a caller-owned output; writes its workspace

The fake (meta) implementations give the output shapes from the arguments alone (chunk counts
and tile counts are ints, never read from device tensors), so tracing needs no device values.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor
from torch.library import custom_op

from ._lib import LIB_PATH, XencError, check, lib, ptr, stream_handle

# The per-token operators (route_topk, library_read, route_read, paged_decode_joint) are defined
# and implemented in C++ (csrc/torch_ops.cpp -> libxenc_torch.so): one dispatcher hop into the C
# ABI per call.  Their fake kernels are registered below.
TORCH_OPS_PATH = LIB_PATH.with_name("libxenc_torch.so")


def _load_cpp_ops() -> None:
    lib()  # libxenc_hip.so first: its C ABI is version-checked, and libxenc_torch.so links to it
    if not TORCH_OPS_PATH.exists():
        raise XencError(f"{TORCH_OPS_PATH} is not built: run kv_skill_v2_amd._build.build() "
                        "(the Library read has no CPU path)")
    torch.ops.load_library(str(TORCH_OPS_PATH))


_load_cpp_ops()


def _st(t: Tensor) -> int:
    return stream_handle(t.device)


def kept_width(top_k: int, cmax: int) -> int:
    """Columns of the routed-index arrays for a pool whose largest library has cmax chunks."""
    return cmax if (top_k <= 0 or top_k >= cmax) else top_k


# ----------------------------------------------------------------------------- decode routing
@torch.library.register_fake("xenc::route_topk")
def _(q, S, chunk_ptr, q_group, top_k, route_temp, cmax, kk):
    M = q.shape[0]
    return (q.new_empty(M, cmax), q.new_empty(M, kk, dtype=torch.int32), q.new_empty(M, kk))


# ----------------------------------------------------------------------------- decode read
@torch.library.register_fake("xenc::library_read")
def _(q, pages, chunk_page, chunk_nvalid, chunk_ptr, q_group, idx, w_sel, read_temp, softmax, nsplit,
      workspace, max_rows):
    return q.new_empty(q.shape[0], pages.shape[-1])


# ----------------------------------------------------------------------------- decode routing + read
@torch.library.register_fake("xenc::route_read")
def _(q, S, pages, chunk_page, chunk_nvalid, chunk_ptr, q_group, top_k, route_temp, cmax, kk, read_temp, softmax,
      nsplit, workspace, max_rows):
    M = q.shape[0]
    return (q.new_empty(M, cmax), q.new_empty(M, kk, dtype=torch.int32), q.new_empty(M, kk),
            q.new_empty(M, pages.shape[-1]))


# ----------------------------------------------------------------------------- many-row routing
@custom_op("xenc::route_rows", mutates_args=())
def route_rows(q: Tensor, S: Tensor, chunk_ptr: Tensor, row_ptr: Tensor, logit_tiles: Tensor,
               route_tiles: Tensor, n_logit: int, n_route: int, top_k: int, route_temp: float, cmax: int,
               kk: int, emit_f16: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(w [M, cmax], idx [M, kk], w_sel [M, kk], q as fp16 [M, d] when emit_f16 else [0, d])."""
    M, d = q.shape
    w = torch.empty(M, cmax, dtype=torch.float32, device=q.device)
    idx = torch.empty(M, kk, dtype=torch.int32, device=q.device)
    wsel = torch.empty(M, kk, dtype=torch.float32, device=q.device)
    qh = torch.empty(M if emit_f16 else 0, d, dtype=torch.float16, device=q.device)
    if M:
        check(lib().xenc_route_topk_rows(ptr(q), q.stride(0), M, d, ptr(S), ptr(chunk_ptr), ptr(row_ptr),
                                         ptr(logit_tiles), chunk_ptr.numel() - 1, n_logit, top_k, route_temp,
                                         ptr(w), w.stride(0), ptr(idx), ptr(wsel), kk,
                                         ptr(qh) if emit_f16 else None, _st(q)), "xenc_route_topk_rows")
    return w, idx, wsel, qh


@route_rows.register_fake
def _(q, S, chunk_ptr, row_ptr, logit_tiles, route_tiles, n_logit, n_route, top_k, route_temp, cmax, kk,
      emit_f16):
    M, d = q.shape
    return (q.new_empty(M, cmax), q.new_empty(M, kk, dtype=torch.int32), q.new_empty(M, kk),
            q.new_empty(M if emit_f16 else 0, d, dtype=torch.float16))


@custom_op("xenc::route_backward_", mutates_args=("dq",))
def route_backward_(dq: Tensor, w: Tensor, dw: Tensor, dw_ext: Optional[Tensor], S: Tensor, chunk_ptr: Tensor,
                    row_ptr: Tensor, route_tiles: Tensor, n_route: int, route_temp: float) -> None:
    """dq[t] += route_temp * sum_c w (dw + dw_ext - sum_c' w (dw + dw_ext)) S_c."""
    check(lib().xenc_route_backward(ptr(w), w.stride(0), ptr(dw), dw.stride(0), ptr(dw_ext),
                                    dw_ext.stride(0) if dw_ext is not None else 0, ptr(row_ptr), ptr(route_tiles),
                                    chunk_ptr.numel() - 1, n_route, w.shape[1], ptr(S), ptr(chunk_ptr),
                                    dq.shape[1], route_temp, ptr(dq), dq.stride(0), _st(dq)), "xenc_route_backward")


@route_backward_.register_fake
def _(dq, w, dw, dw_ext, S, chunk_ptr, row_ptr, route_tiles, n_route, route_temp):
    return None


def _route_rows_setup(ctx, inputs, output):
    q, S, chunk_ptr, row_ptr, logit_tiles, route_tiles, n_logit, n_route = inputs[:8]
    route_temp = inputs[9]
    w = output[0]
    ctx.save_for_backward(w, S, chunk_ptr, row_ptr, route_tiles)
    ctx.n_route, ctx.route_temp, ctx.d = n_route, route_temp, q.shape[1]
    ctx.mark_non_differentiable(output[1], output[2], output[3])


def _route_rows_backward(ctx, dw, _didx, _dwsel, _dqh):
    w, S, chunk_ptr, row_ptr, route_tiles = ctx.saved_tensors
    dq = torch.zeros(w.shape[0], ctx.d, dtype=torch.float32, device=w.device)
    if dw is not None:
        torch.ops.xenc.route_backward_(dq, w, dw.contiguous(), None, S, chunk_ptr, row_ptr, route_tiles,
                                       ctx.n_route, ctx.route_temp)
    return (dq,) + (None,) * 12


route_rows.register_autograd(_route_rows_backward, setup_context=_route_rows_setup)


# ----------------------------------------------------------------------------- MFMA prefill read
@custom_op("xenc::library_prefill_bwd_dq", mutates_args=())
def library_prefill_bwd_dq(g: Tensor, w: Tensor, p: Tensor, frag_v_scores: Tensor, frag_k_readout: Tensor,
                           chunk_ptr: Tensor, chunk_page: Tensor, chunk_nvalid: Tensor, row_ptr: Tensor,
                           score_tiles: Tensor, readout_tiles: Tensor, n_score: int, n_readout: int,
                           slots: int, read_temp: float, softmax: bool) -> tuple[Tensor, Tensor]:
    """(dq [M, d] through the read, gamma [M, cmax] = dL/dw) for the upstream gradient g [M, d]."""
    M, d = g.shape
    ds, gamma = _bwd_scores(g, w, p, frag_v_scores, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles,
                            n_score, slots, read_temp, softmax)
    dq = torch.empty(M, d, dtype=torch.float32, device=g.device)
    check(lib().xenc_prefill_readout(ptr(ds), M, ptr(row_ptr), ptr(readout_tiles), chunk_ptr.numel() - 1,
                                     n_readout, ptr(frag_k_readout), slots, d, frag_k_readout.stride(0),
                                     ptr(chunk_ptr), ptr(chunk_page), None, 0, ptr(dq), dq.stride(0), _st(g)),
          "xenc_prefill_readout")
    return dq, gamma


def _bwd_scores(g, w, p, frag_v_scores, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles, n_score, slots,
                read_temp, softmax):
    """The backward's scores pass: (dS octet-major like p, gamma [M, cmax] = dL/dw through the read)."""
    M, d = g.shape
    L, st = lib(), _st(g)
    gh = torch.empty(M, d, dtype=torch.float16, device=g.device)
    check(L.xenc_cast_rows_f16(ptr(g), g.stride(0), M, d, ptr(gh), st), "xenc_cast_rows_f16")
    ds = torch.empty_like(p)
    gamma = torch.zeros(M, w.shape[1], dtype=torch.float32, device=g.device)
    check(L.xenc_prefill_scores(1 if softmax else 3, ptr(gh), d, ptr(row_ptr), ptr(score_tiles),
                                chunk_ptr.numel() - 1, n_score, ptr(frag_v_scores), slots, frag_v_scores.stride(0),
                                ptr(chunk_ptr), ptr(chunk_page), ptr(chunk_nvalid), read_temp, ptr(w), w.stride(0),
                                ptr(p), M, ptr(ds), ptr(gamma), gamma.stride(0), st), "xenc_prefill_scores")
    return ds, gamma


@custom_op("xenc::library_prefill_bwd_routed", mutates_args=())
def library_prefill_bwd_routed(g: Tensor, w: Tensor, p: Tensor, dw_ext: Optional[Tensor], S: Tensor,
                               frag_v_scores: Tensor, frag_k_readout: Tensor, chunk_ptr: Tensor, chunk_page: Tensor,
                               chunk_nvalid: Tensor, row_ptr: Tensor, score_tiles: Tensor, readout_tiles: Tensor,
                               n_score: int, n_readout: int, slots: int, read_temp: float, softmax: bool,
                               route_temp: float) -> Tensor:
    """dq [M, d] through the read AND the routing, for the upstream gradient g = dL/dr and the
    gradient dw_ext that reaches w from elsewhere (None: none): the scores pass gives gamma =
    dL/dw through the read, then route_coef_kernel + readout_kernel write
    dq = dS . K + route_temp * sum_c w (dw - sum w dw) S_c with dw = gamma + dw_ext, the routing
    term folded into the readout (its accumulators start from it)."""
    M, d = g.shape
    cmax = w.shape[1]
    ds, gamma = _bwd_scores(g, w, p, frag_v_scores, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles,
                            n_score, slots, read_temp, softmax)
    dl = torch.empty(M, cmax, dtype=torch.float32, device=g.device)
    dq = torch.empty(M, d, dtype=torch.float32, device=g.device)
    check(lib().xenc_prefill_readout_routed(
        ptr(ds), M, ptr(row_ptr), ptr(readout_tiles), chunk_ptr.numel() - 1, n_readout, ptr(frag_k_readout), slots,
        d, frag_k_readout.stride(0), ptr(chunk_ptr), ptr(chunk_page), ptr(w), w.stride(0), ptr(gamma),
        gamma.stride(0), ptr(dw_ext), dw_ext.stride(0) if dw_ext is not None else 0, ptr(S), cmax, route_temp,
        ptr(dl), dl.stride(0), ptr(dq), dq.stride(0), _st(g)), "xenc_prefill_readout_routed")
    return dq


@library_prefill_bwd_routed.register_fake
def _(g, w, p, dw_ext, S, frag_v_scores, frag_k_readout, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles,
      readout_tiles, n_score, n_readout, slots, read_temp, softmax, route_temp):
    return g.new_empty(g.shape)


@library_prefill_bwd_dq.register_fake
def _(g, w, p, frag_v_scores, frag_k_readout, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles,
      readout_tiles, n_score, n_readout, slots, read_temp, softmax):
    M, d = g.shape
    return g.new_empty(M, d), g.new_empty(M, w.shape[1])


@custom_op("xenc::library_prefill_fwd", mutates_args=())
def library_prefill_fwd(q: Tensor, qh: Optional[Tensor], w: Tensor, frag_k_scores: Tensor,
                        frag_v_readout: Tensor, frag_v_scores: Tensor, frag_k_readout: Tensor, chunk_ptr: Tensor,
                        chunk_page: Tensor, chunk_nvalid: Tensor, row_ptr: Tensor, score_tiles: Tensor,
                        readout_tiles: Tensor, n_score: int, n_readout: int, slots: int, read_temp: float,
                        softmax: bool, ragged: bool) -> tuple[Tensor, Tensor]:
    """(r [M, d], p fp16 octet-major [cmax * slots / 8, M, 8]).  qh: q as fp16 rows when the
    routing pass already wrote them (else cast here).  The value-side fragment copies
    (frag_v_scores, frag_k_readout) are only read by the backward.  ragged: the libraries have
    different chunk counts, so p is zeroed first (the kernel writes a row's own chunks only)."""
    M, d = q.shape
    G = chunk_ptr.numel() - 1
    L, st = lib(), _st(q)
    if qh is None or qh.numel() == 0:
        qh = torch.empty(M, d, dtype=torch.float16, device=q.device)
        check(L.xenc_cast_rows_f16(ptr(q), q.stride(0), M, d, ptr(qh), st), "xenc_cast_rows_f16")
    p = (torch.zeros if ragged else torch.empty)(w.shape[1] * slots // 8, M, 8, dtype=torch.float16,
                                                  device=q.device)
    check(L.xenc_prefill_scores(0 if softmax else 2, ptr(qh), d, ptr(row_ptr), ptr(score_tiles), G, n_score,
                                ptr(frag_k_scores), slots, frag_k_scores.stride(0), ptr(chunk_ptr), ptr(chunk_page),
                                ptr(chunk_nvalid), read_temp, None, 0, ptr(p), M, None, None, 0, st),
          "xenc_prefill_scores")
    r = torch.empty(M, d, dtype=torch.float32, device=q.device)
    check(L.xenc_prefill_readout(ptr(p), M, ptr(row_ptr), ptr(readout_tiles), G, n_readout, ptr(frag_v_readout),
                                 slots, d, frag_v_readout.stride(0), ptr(chunk_ptr), ptr(chunk_page), ptr(w),
                                 w.stride(0), ptr(r), r.stride(0), st), "xenc_prefill_readout")
    return r, p


@library_prefill_fwd.register_fake
def _(q, qh, w, frag_k_scores, frag_v_readout, frag_v_scores, frag_k_readout, chunk_ptr, chunk_page,
      chunk_nvalid, row_ptr, score_tiles, readout_tiles, n_score, n_readout, slots, read_temp, softmax, ragged):
    M, d = q.shape
    return q.new_empty(M, d), q.new_empty(w.shape[1] * slots // 8, M, 8, dtype=torch.float16)


@custom_op("xenc::library_prefill_lse", mutates_args=())
def library_prefill_lse(q: Tensor, qh: Optional[Tensor], frag_k_scores: Tensor, chunk_ptr: Tensor,
                        chunk_page: Tensor, chunk_nvalid: Tensor, row_ptr: Tensor, score_tiles: Tensor,
                        n_score: int, slots: int, read_temp: float, cmax: int) -> Tensor:
    """lse [M, cmax] fp32: logsumexp_n(read_temp * q . K[c, n]) over the valid slots of each of the
    row's chunks (the forward scores pass; -inf for chunks a row's library does not have)."""
    M, d = q.shape
    G = chunk_ptr.numel() - 1
    L, st = lib(), _st(q)
    if qh is None or qh.numel() == 0:
        qh = torch.empty(M, d, dtype=torch.float16, device=q.device)
        check(L.xenc_cast_rows_f16(ptr(q), q.stride(0), M, d, ptr(qh), st), "xenc_cast_rows_f16")
    p = torch.empty(cmax * slots // 8, M, 8, dtype=torch.float16, device=q.device)
    lse = torch.full((M, cmax), float("-inf"), dtype=torch.float32, device=q.device)
    check(L.xenc_prefill_scores(0, ptr(qh), d, ptr(row_ptr), ptr(score_tiles), G, n_score, ptr(frag_k_scores),
                                slots, frag_k_scores.stride(0), ptr(chunk_ptr), ptr(chunk_page), ptr(chunk_nvalid),
                                read_temp, None, 0, ptr(p), M, None, ptr(lse), lse.stride(0), st),
          "xenc_prefill_scores")
    return lse


@library_prefill_lse.register_fake
def _(q, qh, frag_k_scores, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles, n_score, slots, read_temp,
      cmax):
    return q.new_empty(q.shape[0], cmax)


_PREFILL_TENSORS = ("frag_v_scores", "frag_k_readout", "chunk_ptr", "chunk_page", "chunk_nvalid", "row_ptr",
                    "score_tiles", "readout_tiles")


def _prefill_setup(ctx, inputs, output):
    (q, qh, w, _fks, _fvr, fvs, fkr, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles, readout_tiles,
     n_score, n_readout, slots, read_temp, softmax, _ragged) = inputs
    ctx.save_for_backward(w, output[1], fvs, fkr, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles,
                          readout_tiles)
    ctx.sizes = (n_score, n_readout, slots, read_temp, softmax)
    ctx.mark_non_differentiable(output[1])


def _prefill_backward(ctx, dr, _dp):
    w, p, *rest = ctx.saved_tensors
    dq, gamma = torch.ops.xenc.library_prefill_bwd_dq(dr.contiguous(), w, p, *rest, *ctx.sizes)
    return (dq, None, gamma) + (None,) * 16


library_prefill_fwd.register_autograd(_prefill_backward, setup_context=_prefill_setup)


# ----------------------------------------------------------------------------- routing + MFMA read, one node
@custom_op("xenc::library_read_routed", mutates_args=())
def library_read_routed(q: Tensor, S: Tensor, chunk_ptr: Tensor, row_ptr: Tensor, logit_tiles: Tensor,
                        route_tiles: Tensor, n_logit: int, n_route: int, top_k: int, route_temp: float, cmax: int,
                        kk: int, frag_k_scores: Tensor, frag_v_readout: Tensor, frag_v_scores: Tensor,
                        frag_k_readout: Tensor, chunk_page: Tensor, chunk_nvalid: Tensor, score_tiles: Tensor,
                        readout_tiles: Tensor, n_score: int, n_readout: int, slots: int, read_temp: float,
                        softmax: bool, ragged: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(r [M, d], w [M, cmax], idx, w_sel, p): xenc::route_rows (which also writes q as fp16) then
    xenc::library_prefill_fwd, as ONE autograd node.  Its backward (library_prefill_bwd_routed)
    writes dq once, the routing term with dL/dw = gamma + the gradient that reaches w from
    elsewhere (the injector's route_terms) folded into the readout, so no zeroed gradient
    buffer, no second pass over dq and no gradient sum are needed."""
    w, idx, wsel, qh = torch.ops.xenc.route_rows(q, S, chunk_ptr, row_ptr, logit_tiles, route_tiles, n_logit,
                                                  n_route, top_k, route_temp, cmax, kk, True)
    r, p = torch.ops.xenc.library_prefill_fwd(q, qh, w, frag_k_scores, frag_v_readout, frag_v_scores,
                                              frag_k_readout, chunk_ptr, chunk_page, chunk_nvalid, row_ptr,
                                              score_tiles, readout_tiles, n_score, n_readout, slots, read_temp,
                                              softmax, ragged)
    return r, w, idx, wsel, p


@library_read_routed.register_fake
def _(q, S, chunk_ptr, row_ptr, logit_tiles, route_tiles, n_logit, n_route, top_k, route_temp, cmax, kk,
      frag_k_scores, frag_v_readout, frag_v_scores, frag_k_readout, chunk_page, chunk_nvalid, score_tiles,
      readout_tiles, n_score, n_readout, slots, read_temp, softmax, ragged):
    M, d = q.shape
    return (q.new_empty(M, d), q.new_empty(M, cmax), q.new_empty(M, kk, dtype=torch.int32), q.new_empty(M, kk),
            q.new_empty(cmax * slots // 8, M, 8, dtype=torch.float16))


def _routed_setup(ctx, inputs, output):
    (q, S, chunk_ptr, row_ptr, _lt, route_tiles, _nl, n_route, _tk, route_temp, _cmax, _kk, _fks, _fvr, fvs, fkr,
     chunk_page, chunk_nvalid, score_tiles, readout_tiles, n_score, n_readout, slots, read_temp, softmax,
     _ragged) = inputs
    _, w, _, _, p = output
    ctx.save_for_backward(w, p, fvs, fkr, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles, readout_tiles,
                          S, route_tiles)
    ctx.sizes = (n_score, n_readout, slots, read_temp, softmax)
    ctx.route = (n_route, route_temp)
    ctx.d = q.shape[1]
    ctx.mark_non_differentiable(output[2], output[3], output[4])


def _routed_backward(ctx, dr, dw, _didx, _dwsel, _dp):
    w, p, fvs, fkr, chunk_ptr, chunk_page, chunk_nvalid, row_ptr, score_tiles, readout_tiles, S, route_tiles = \
        ctx.saved_tensors
    dw = None if dw is None else dw.contiguous()
    if dr is None:  # only w reaches the loss: the routing term alone
        dq = torch.zeros(w.shape[0], ctx.d, dtype=torch.float32, device=w.device)
        torch.ops.xenc.route_backward_(dq, w, torch.zeros_like(w), dw, S, chunk_ptr, row_ptr, route_tiles,
                                       *ctx.route)
    else:
        n_score, n_readout, slots, read_temp, softmax = ctx.sizes
        dq = torch.ops.xenc.library_prefill_bwd_routed(dr.contiguous(), w, p, dw, S, fvs, fkr, chunk_ptr, chunk_page,
                                                        chunk_nvalid, row_ptr, score_tiles, readout_tiles, n_score,
                                                        n_readout, slots, read_temp, softmax, ctx.route[1])
    return (dq,) + (None,) * 25


library_read_routed.register_autograd(_routed_backward, setup_context=_routed_setup)


# ----------------------------------------------------------------------------- op B
_JOINT_DTYPES = {torch.float16: 0, torch.bfloat16: 1}


@torch.library.register_fake("xenc::paged_decode_joint")
def _(q, op_k, op_v, op_bt, op_len, own_k, own_v, own_bt, own_len, scale, nsplit, chunk, workspace, max_n, out):
    return None


__all__ = ["route_rows", "route_backward_", "library_prefill_lse", "library_prefill_fwd",
           "library_prefill_bwd_dq", "library_prefill_bwd_routed", "library_read_routed", "kept_width", "TORCH_OPS_PATH"]
