"""Autograd wrappers of the fused per-row epilogues (csrc/fused.hip).

``act_norm_dropout`` is the hidden-layer tail of the reference model
(models/model.py:259-264): ``dropout(LayerNorm(act(h)))`` in one pass each
way instead of torch's separate cast, activation, LayerNorm, dropout and cast
kernels.  Under autocast the output is written in the autocast dtype: the
unfused path produces fp32 there (LayerNorm runs in fp32) and the next
layer's product casts it to that dtype, so the next layer sees the same
values.  The dropout mask comes from Philox keyed by a seed drawn from
torch's CPU generator (reproducible under torch.manual_seed; not the same
mask torch's dropout would draw).  While the stream is being captured into
a graph the seed is drawn on the device instead (torch's CUDA generator,
whose draws advance on every replay) and the kernels read it from there, so
each replay of a captured training step draws a new mask.

``cross_entropy_rows`` is ``F.cross_entropy(logits[rows], labels)`` plus the
argmax hit count of helper/engine.py:22-41, in one kernel each way.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch.autograd import Function

from ..core import ops as _ops


def _seed() -> int:
    return int(torch.randint(0, 2 ** 62, (1,)).item())


class _ActNormDropout(Function):
    @staticmethod
    def forward(ctx, z, weight, bias, eps, p, act, out_dtype):
        seed, seed_dev = 0, None
        if p > 0:
            if torch.cuda.is_current_stream_capturing():
                seed_dev = torch.randint(0, 2 ** 62, (1,), dtype=torch.int64, device=z.device)
            else:
                seed = _seed()
        need = any(ctx.needs_input_grad[:3])
        out, mean, rstd = _ops.act_norm_dropout_fwd(z, weight, bias, eps, p, act, seed, out_dtype, need, seed_dev)
        if need:
            ctx.save_for_backward(z, weight, mean, rstd)
        ctx.p, ctx.act, ctx.seed, ctx.seed_dev = p, act, seed, seed_dev
        return out

    @staticmethod
    def backward(ctx, dout):
        z, weight, mean, rstd = ctx.saved_tensors
        dz, dg, db = _ops.act_norm_dropout_bwd(dout, z, mean, rstd, weight, ctx.p, ctx.act, ctx.seed, ctx.seed_dev)
        return (dz if ctx.needs_input_grad[0] else None, dg.to(weight.dtype) if ctx.needs_input_grad[1] else None,
                db if ctx.needs_input_grad[2] else None, None, None, None, None)


def act_norm_dropout(z: torch.Tensor, norm: torch.nn.LayerNorm, p: float, relu: bool) -> torch.Tensor:
    """dropout_p(norm(relu(z) if relu else z)) on the fused kernel; the
    output dtype is the autocast dtype when autocast is on, fp32 otherwise."""
    if torch.is_autocast_enabled("cuda"):
        out_dtype = torch.get_autocast_dtype("cuda")
    else:
        out_dtype = torch.float32 if z.dtype == torch.float32 else z.dtype
    with torch.autocast("cuda", enabled=False):
        return _ActNormDropout.apply(z, norm.weight, norm.bias, float(norm.eps), float(p), 1 if relu else 0,
                                     out_dtype)


def fusable_norm(norm, z: torch.Tensor) -> bool:
    """Whether act_norm_dropout can replace norm's LayerNorm on z."""
    return (isinstance(norm, torch.nn.LayerNorm) and norm.elementwise_affine and norm.weight is not None
            and norm.bias is not None and tuple(norm.normalized_shape) == (z.shape[-1],)
            and _ops.act_norm_dropout_supported(z))


class _CrossEntropyRows(Function):
    @staticmethod
    def forward(ctx, logits, rows, labels):
        loss, counts, lse = _ops.cross_entropy_fwd(logits, rows, labels)
        ctx.save_for_backward(logits, rows if rows is not None else torch.empty(0), labels, lse, counts)
        ctx.has_rows = rows is not None
        ctx.mark_non_differentiable(counts)
        return loss, counts

    @staticmethod
    def backward(ctx, dloss, _dcounts):
        logits, rows, labels, lse, counts = ctx.saved_tensors
        grad = _ops.cross_entropy_bwd(logits, rows if ctx.has_rows else None, labels, lse, dloss, counts)
        return grad, None, None


def cross_entropy_rows(logits: torch.Tensor, rows: Optional[torch.Tensor], labels: torch.Tensor):
    """(loss, correct) = (F.cross_entropy(logits[rows].float(), labels),
    (logits[rows].argmax(1) == labels).sum()); rows must be distinct
    (None = the first labels.numel() rows)."""
    return _CrossEntropyRows.apply(logits, rows, labels)


def rows_distinct(rows: torch.Tensor) -> bool:
    """Whether rows is strictly ascending (so distinct), cached per tensor
    version (one small device reduction and one sync the first time)."""
    key = (rows.data_ptr(), rows._version, rows.numel())
    hit = getattr(rows, "_grws_ascending", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    ok = rows.numel() < 2 or bool((rows[1:] > rows[:-1]).all().item())
    rows._grws_ascending = (key, ok)
    return ok


def cross_entropy_supported(logits: torch.Tensor, labels: torch.Tensor) -> bool:
    return (logits.is_cuda and logits.dim() == 2 and logits.stride(1) == 1 and labels.dim() == 1
            and labels.dtype == torch.int64 and labels.is_cuda
            and logits.dtype in (torch.float32, torch.float16, torch.bfloat16))
