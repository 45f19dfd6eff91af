"""One decode step of a reader whose Library read is spread over candidate depths by a LayerSelector.

The reference (xenc/injector.py:231-273 with xenc/selector.py:95-110) runs the whole branch at
every candidate layer and multiplies the update of every unselected layer by zero.  Here the
selector's top-k runs first, and only the (token, selected depth) rows are routed, read and
written back:

    1. per token, in one launch (xenc_multi_depth_prepare_route): the selector's top-k of the
       logits z [B, L] with a softmax over the kept ones (ties go to the lower depth), the query
       row of each kept depth gathered from q_all [L, B, d], gate * gain of each (token, depth)
       row, and beside them, in the same launch, the q . S dots of every row over the chunks of
       its depth library; then the top-k of every row;
    2. the paged split-K read of the routed pages (xenc_library_read_decode: the ranking of the
       routed (row, page) entries by page, the read with the rows that routed the same page side
       by side, the merge of the partials);
    3. the depth's B streamed once with the row scale folded in (xenc_write_back);
    4. the matched-norm rescale times the selector weight, summed over a token's kept depths
       (xenc_selector_apply).

The depth libraries are one pool (`PagedLibrary` with one library per depth); the row's library
index is its depth.  In a model each depth's update is added at its own layer; the step returns
their sum per token, which is what the model's residual stream receives in total.  Every kernel
is asynchronous and allocation sizes depend only on the shapes, so a HIP graph can capture a
step and replay it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops


@dataclass
class MultiDepthDecode:
    """Static state of the step: the depth pool, each depth's write map and the epilogue scalars.

    lib       PagedLibrary holding L libraries (library l = depth l)
    B_w       fp32 [L, d_r, d]: depth l's write map (B of its interface, out-major rows)
    gate_w    fp32 [d_r]; gate_b, log_gain fp32 [L] (one position per depth)
    log_alpha the selector's log alpha (a device scalar tensor or a float)
    """

    lib: ops.PagedLibrary
    B_w: torch.Tensor
    gate_w: torch.Tensor
    gate_b: torch.Tensor
    log_gain: torch.Tensor
    log_alpha: torch.Tensor | float
    k_sel: int = 2
    top_k: int = 8
    route_temp: float = 10.0
    read_temp: float = 12.0
    gain_scale: float = 1.0
    nsplit: int | None = None   # slot splits per routed page of the read (None: the read's default)

    def __post_init__(self):
        L = self.lib.n_libraries
        if self.B_w.dim() != 3 or self.B_w.shape[0] != L or self.B_w.shape[2] != self.lib.d:
            raise ValueError(f"B_w must be [{L}, d_r, {self.lib.d}]")
        if not 1 <= self.k_sel <= L:
            raise ValueError(f"k_sel={self.k_sel} must lie in [1, {L}]")

    def __call__(self, z: torch.Tensor, q_all: torch.Tensor, h: torch.Tensor, hn: torch.Tensor):
        """z fp32 [B, L] selector logits, q_all fp32 [L, B, d] each depth's query rows, h fp32
        [B, d_r] the residual and hn its RMS norm.  Returns (out [B, d_r], idx [B*k_sel, kk]
        routed chunks, depth [B*k_sel] int32): row b*k_sel + j is token b's j-th kept depth."""
        k = self.k_sel
        with torch.no_grad():
            if self.lib.n_libraries <= 64:
                _, top, wtop, qr, scale, _, idx, wsel = ops.multi_depth_prepare_route(
                    z, k, q_all, hn, self.gate_w, self.gate_b, self.log_gain, self.lib, top_k=self.top_k,
                    route_temp=self.route_temp, gain_scale=self.gain_scale)
                depth = top.reshape(-1)
                r = ops.library_read_decode(qr, self.lib, idx, wsel, q_group=depth, read_temp=self.read_temp,
                                            nsplit=self.nsplit)
            else:
                _, top, wtop, qr, scale = ops.multi_depth_prepare(z, k, q_all, hn, self.gate_w, self.gate_b,
                                                                  self.log_gain, self.gain_scale)
                depth = top.reshape(-1)
                _, idx, wsel, r = ops.route_read_decode(qr, self.lib, depth, top_k=self.top_k,
                                                        route_temp=self.route_temp, read_temp=self.read_temp,
                                                        nsplit=self.nsplit)
            upd = ops.write_back(r, self.B_w, depth, None, scale)
            out = ops.selector_apply(upd, h, wtop.reshape(-1), self.log_alpha, k=k)
        return out, idx, depth


__all__ = ["MultiDepthDecode"]
