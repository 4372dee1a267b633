"""Memory layout helpers for dense operands of the SpMM.

The SpMM gathers X row segments of up to 128 columns.  When a row's byte
pitch is a multiple of the 128-byte cache line, every segment starts on a
line boundary and costs exactly ceil(bytes/128) lines; an unaligned pitch
(e.g. 608 fp16 columns = 1216 B) makes about one segment in two straddle an
extra line.  `aligned_rows` stores the same matrix with a padded pitch; the
padding columns are never read.
"""
from __future__ import annotations

import torch


def aligned_rows(x: torch.Tensor, align_bytes: int = 128) -> torch.Tensor:
    """A view of the 2-D tensor `x` whose row stride is padded to a multiple
    of `align_bytes` (the values and shape are unchanged)."""
    if x.dim() != 2:
        raise ValueError("aligned_rows expects a 2-D tensor")
    esz = x.element_size()
    if align_bytes % esz:
        raise ValueError("align_bytes must be a multiple of the element size")
    per = align_bytes // esz
    pitch = (x.shape[1] + per - 1) // per * per
    if x.stride(1) == 1 and x.stride(0) == pitch:
        return x
    buf = torch.zeros((x.shape[0], pitch), dtype=x.dtype, device=x.device)
    buf[:, : x.shape[1]] = x
    return buf[:, : x.shape[1]]
