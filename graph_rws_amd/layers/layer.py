"""BCSR graph convolution with autograd (layers/layer.py:28-191 of the reference).

Same classes, signatures and arithmetic as the reference:
  forward   H = A (X W)                         (layer.py:38-59)
  backward  G_agg = A^T dH, dX = G_agg W^T, dW = X^T G_agg   (layer.py:61-92)
  conv      out = trim(A (X W_neigh)) + X_target W_self      (layer.py:118-191)
The SpMM runs on the gfx950 kernel (H1); A^T dH runs the same kernel over the
cached device-built transpose of A instead of the reference's atomic scatter.
A (X W) may be associated as (A X) W when that gathers fewer columns.
BCSRGraphConv runs as one autograd node (_GraphConvFunction): the self
product is added by a beta=1 GEMM, and a target that is a prefix of X gets
its gradient added into dX in place.  BCSRSPMMFunction keeps the reference's
A (X W) node for callers that use it directly.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.autograd import Function

from ..core import ops as _ops
from ..helper.timer import record_spmm_time


# Add the self path's product inside the SpMM's epilogue (one GEMM makes
# both X W_n and X W_s) when the targets are (nearly) all of X's rows;
# False restores the separate beta=1 GEMM.
FUSED_SELF = True

# Aggregate-first layers whose input the graph gathers through a zero-padded,
# line-aligned copy (112 features on a 128-element pitch) run both GEMMs on
# that padded width: the padding columns and zero weight rows add exact zeros,
# and the library GEMM is faster at K=128 than at K=112 (c4: 0.45 against
# 0.62 ms, and 0.58 against 0.71 ms for the accumulating one).  False keeps
# the unpadded width.
PAD_AGGREGATE = True


def _spmm_timed(graph, x: torch.Tensor, residual: torch.Tensor = None):
    """graph.spmm with the reference's (output, ms) convention (bind.cpp:124-130)."""
    if not _ops.TIMING:
        return graph.spmm(x, residual=residual), 0.0
    s = torch.cuda.current_stream(x.device)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(s)
    y = graph.spmm(x, residual=residual)
    e1.record(s)
    e1.synchronize()
    return y, float(e0.elapsed_time(e1))


def _autocast_operand(x: torch.Tensor) -> torch.Tensor:
    """x in the dtype autocast would multiply it in (x itself otherwise)."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        if x.dtype != dt and x.is_floating_point():
            return x.to(dt)
    return x


def _weight_grad(x: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """x^T @ g: the split-K gfx950 kernel for tall f16/bf16 operands (the
    library GEMM leaves most of the chip idle on this shape), torch
    otherwise.  float32 result from the kernel."""
    if x.shape[0] >= 4096 and _ops.gemm_tn_supported(x, g):
        return _ops.gemm_tn(x, g, out_dtype=torch.float32)
    return torch.matmul(x.t(), g)


def _aggregate_first(in_w: int, out_w: int, x_needs_grad: bool) -> bool:
    """Whether A (X W) is cheaper evaluated as (A X) W.  The SpMM's cost is
    its gathered width: X-first aggregates out_w columns forward and again
    backward (A^T G feeds the weight gradient); aggregate-first gathers in_w
    columns forward, and backward only when X itself needs a gradient
    (dW = (A X)^T G is a plain GEMM)."""
    if x_needs_grad:
        return in_w < out_w
    return in_w < 2 * out_w


class BCSRSPMMFunction(Function):
    """output = A @ (X @ W) with A a BCSRGraph (layer.py:28-92).  The product
    is associated as A (X W), as the reference does, or as (A X) W when that
    gathers fewer columns (a layer widening its input, or any layer whose
    input needs no gradient); the result is the same product, rounded in the
    other order.  Under torch.autocast the backward runs in the forward's
    autocast state, so a float16/bfloat16 forward has a float16/bfloat16
    backward SpMM; saved operands are kept in the autocast dtype for the
    weight gradient."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, graph, features, weight, warps_per_block):
        xh = _autocast_operand(features)
        ctx.graph = graph
        ctx.warps_per_block = warps_per_block
        ctx.num_input_nodes = features.shape[0]
        ctx.agg_first = _aggregate_first(weight.shape[0], weight.shape[1], features.requires_grad)
        if ctx.agg_first:
            agg, timing = _spmm_timed(graph, xh)
            output = torch.matmul(agg, weight)
            ctx.save_for_backward(agg, weight)
        else:
            x_mult_w = torch.matmul(xh, weight)
            output, timing = _spmm_timed(graph, x_mult_w)
            ctx.save_for_backward(xh, weight)
        record_spmm_time(timing)
        return output

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad_output):
        saved, weight = ctx.saved_tensors
        graph = ctx.graph
        grad_features = None
        grad_weight = None
        g = grad_output.contiguous()
        if ctx.agg_first:
            # H = (A X) W:  dW = (A X)^T dH,  dX = A^T (dH W^T)
            if ctx.needs_input_grad[2]:
                grad_weight = _weight_grad(saved, g)
            if ctx.needs_input_grad[1]:
                grad_features = graph.spmm_transpose(torch.matmul(g, weight.t()).contiguous(),
                                                     ctx.num_input_nodes)
            return None, grad_features, grad_weight, None
        grad_input_aggr = graph.spmm_transpose(g, ctx.num_input_nodes)
        if ctx.needs_input_grad[1]:
            grad_features = torch.matmul(grad_input_aggr, weight.t())
        if ctx.needs_input_grad[2]:
            grad_weight = _weight_grad(saved, grad_input_aggr)
        return None, grad_features, grad_weight, None


def _is_prefix_view(t: torch.Tensor, base: torch.Tensor) -> bool:
    """Whether t is base[:t.shape[0]] (same storage, offset and strides)."""
    return (t.dim() == 2 and base.dim() == 2 and t.shape[1] == base.shape[1] and t.shape[0] <= base.shape[0]
            and t.untyped_storage().data_ptr() == base.untyped_storage().data_ptr()
            and t.storage_offset() == base.storage_offset() and t.stride() == base.stride())


class _GraphConvFunction(Function):
    """out[T] = A (X W_n) [:T] + X_tgt W_s (layer.py:118-191) as one autograd
    node.  The self product is added into the SpMM output by a beta=1 GEMM
    instead of a separate add; when X_tgt is a prefix of X (the full-graph
    and node-wise block cases) its gradient is added into dX in place, and
    the backward SpMM reads the T gradient rows directly (rows of A beyond T
    contribute nothing), so no padded gradient is materialised.  The product
    is associated as A (X W_n) or (A X) W_n by _aggregate_first."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, graph, x, x_tgt, w_n, w_s, prefix_rows):
        xh = _autocast_operand(x)
        if x_tgt is None:
            xt = xh[:prefix_rows]
        else:
            xt = _autocast_operand(x_tgt)
        T = xt.shape[0]
        ctx.graph = graph
        ctx.num_input_nodes = x.shape[0]
        ctx.prefix = x_tgt is None
        ctx.agg_first = _aggregate_first(w_n.shape[0], w_n.shape[1], x.requires_grad)

        def rows_T(y):
            if y.shape[0] >= T:
                return y[:T]
            return F.pad(y, (0, 0, 0, T - y.shape[0]))

        # the beta=1 GEMMs accumulate in place into a tensor this function
        # made (no copy of it into a new output); in-place ops are not
        # autocast, so the weights take the operands' dtype explicitly
        ctx.kpad = 0
        padded = getattr(graph, "padded_input", None)
        xp = (padded(xh) if (PAD_AGGREGATE and padded is not None and ctx.agg_first and x_tgt is None
                             and xh.is_cuda) else None)
        if xp is not None:
            # (A Xp) Wn_p + Xp[:T] Ws_p over the zero-padded width
            k, kp = xh.shape[1], xp.shape[1]
            y, ms = _spmm_timed(graph, xp)
            yt = rows_T(y)
            xtp = xp[:T]
            out = torch.matmul(xtp, F.pad(w_s, (0, 0, 0, kp - k)).to(xtp.dtype))
            out.addmm_(yt, F.pad(w_n, (0, 0, 0, kp - k)).to(out.dtype))
            ctx.save_for_backward(yt, xtp, w_n, w_s)
            ctx.kpad = k
        elif ctx.agg_first:
            y, ms = _spmm_timed(graph, xh)
            yt = rows_T(y)
            out = torch.matmul(xt, w_s)
            out.addmm_(yt, w_n.to(out.dtype))
            ctx.save_for_backward(yt, xt, w_n, w_s)
        elif (FUSED_SELF and x_tgt is None and T <= 16 * graph.num_windows and 10 * T >= 9 * xh.shape[0]
              and xh.is_cuda and _ops.fuse_self_pays(xh.shape[0], w_n.shape[1], xh.element_size())):
            # out = A (X W_n)[:T] + X[:T] W_s: both products from one GEMM,
            # the self term added by the SpMM before it rounds Y
            t_n, t_s = _ops.mm_pair_line_pitched(xh, w_n, w_s)
            y, ms = _spmm_timed(graph, t_n, residual=t_s[:T])
            out = y[:T]
            ctx.save_for_backward(xh, xt, w_n, w_s)
        else:
            y, ms = _spmm_timed(graph, _ops.mm_line_pitched(xh, w_n))
            yt = rows_T(y)
            out = yt.addmm_(xt, w_s.to(yt.dtype))
            ctx.save_for_backward(xh, xt, w_n, w_s)
        record_spmm_time(ms)
        return out

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, grad):
        saved, xt, w_n, w_s = ctx.saved_tensors
        graph = ctx.graph
        # row-strided gradients (a line-pitched loss gradient) are used as
        # they are: every consumer below takes a row stride
        row_strided = grad.dim() == 2 and grad.stride(1) == 1 and grad.stride(0) >= grad.shape[1]
        g = grad if row_strided else grad.contiguous()
        need_x, need_xt, need_wn, need_ws = (ctx.needs_input_grad[1], ctx.needs_input_grad[2],
                                             ctx.needs_input_grad[3], ctx.needs_input_grad[4])
        dx = dxt = dwn = dws = None
        if need_ws:
            dws = _weight_grad(xt, g)
            if ctx.kpad:
                dws = dws[: ctx.kpad]  # the padded width's extra rows are zero
        if ctx.agg_first:
            # out = (A X)[:T] W_n + X_tgt W_s
            if need_wn:
                dwn = _weight_grad(saved, g)
                if ctx.kpad:
                    dwn = dwn[: ctx.kpad]
            if need_x:
                dx = graph.spmm_transpose(torch.matmul(g, w_n.t()).contiguous(), ctx.num_input_nodes)
        else:
            g_agg = graph.spmm_transpose(g, ctx.num_input_nodes)
            if need_wn:
                dwn = _weight_grad(saved, g_agg)
            if need_x:
                dx = torch.matmul(g_agg, w_n.t())
        if ctx.prefix:
            if need_x:
                if not dx.is_contiguous():
                    dx = dx.contiguous()
                dx[: g.shape[0]].addmm_(g, w_s.t().to(g.dtype))
        elif need_xt:
            dxt = torch.matmul(g, w_s.t())
        return None, dx, dxt, dwn, dws, None


class BCSRGraphConv(nn.Module):
    """GraphSAGE-style convolution: neighbour aggregation plus self transform
    (layer.py:95-191).  `warps_per_block` is kept for API compatibility; the
    gfx950 kernel chooses its own launch shape."""

    def __init__(self, in_feats: int, out_feats: int, dropout: float = 0.5,
                 warps_per_block: int = 8):
        super().__init__()
        self.in_feats = in_feats
        self.out_feats = out_feats
        self.warps_per_block = warps_per_block
        self.weight_neigh = nn.Parameter(torch.empty(in_feats, out_feats))
        self.weight_self = nn.Parameter(torch.empty(in_feats, out_feats))
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.xavier_uniform_(self.weight_neigh)
        nn.init.xavier_uniform_(self.weight_self)

    def needs_transpose(self, x_needs_grad: bool) -> bool:
        """Whether this layer's backward runs A^T (an SpMM over the graph's
        transpose) when its input does (not) need a gradient."""
        return x_needs_grad or not _aggregate_first(self.in_feats, self.out_feats, False)

    def forward(self, graph, features: torch.Tensor,
                features_target: torch.Tensor = None) -> torch.Tensor:
        """A (X W_neigh) + X_target W_self, trimmed or zero-padded to the
        target rows (layer.py:118-191): features_target, or the graph's 16W
        rows (features sliced or zero-padded to them) when it is None."""
        target_rows = 16 * graph.num_windows
        if features_target is None:
            if features.shape[0] >= target_rows:
                features_target = features[:target_rows]
            else:
                features_target = F.pad(features, (0, 0, 0, target_rows - features.shape[0]))
        if _is_prefix_view(features_target, features):
            return _GraphConvFunction.apply(graph, features, None, self.weight_neigh, self.weight_self,
                                            features_target.shape[0])
        return _GraphConvFunction.apply(graph, features, features_target, self.weight_neigh, self.weight_self, 0)
