"""Checks of full-size SpMM results against the float64 oracle, for graphs
too large to multiply whole on the host in float64 (c3: 1.2G column slots).

Two checks, both against the oracle's products on the stored element types
(oracle.bcsr_spmm_windows / bcsr_spmv / bcsr_spmv_t / bcsr_spmm_t_rows,
pinned to scipy.sparse in tests/test_oracle.py):

* elementwise on a fixed window set: the first and last windows, the 64
  heaviest, every window the plan splits, and a seeded 1% sample;
  |Y - Y_ref| <= rtol * (|A| |X|) (the north_star bound);
* a projection over every output row: Y r against A (X r) in float64 for a
  seeded random r, bounded by rtol * |A| (|X| |r|), which the elementwise
  bound implies row by row.

The transposed product A^T G is checked the same way on its output rows
(windows of the transpose) and by A^T (G r).
"""
from __future__ import annotations

import numpy as np
import torch

import oracle

DT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def raw(t: torch.Tensor) -> np.ndarray:
    """Host copy of t in its stored element type (bf16 as uint16 bits)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


class HostGraph:
    """Host copies of a BCSRGraph's arrays (values in their stored type)."""

    def __init__(self, G):
        self.win = G.window_offset.cpu().numpy()
        self.cols = G.original_col_indices.cpu().numpy()
        self.vals = raw(G.values_condensed)
        self.vdt = DT[G.values_condensed.dtype]
        self.tc = G.tile_cols
        self.W = G.num_windows
        self.num_cols = G.num_cols


def select_windows(win: np.ndarray, plan=None, seed: int = 0, heavy: int = 64, frac: float = 0.01):
    """First, last, the `heavy` windows with most tiles, every split window
    of `plan`, and a seeded `frac` sample."""
    W = len(win) - 1
    tiles = np.diff(win)
    sel = [0, W - 1]
    sel += list(np.argsort(-tiles, kind="stable")[:heavy])
    if plan is not None and plan.num_split > 0:
        sp = plan.split[: 3 * plan.num_split].view(-1, 3)[:, 0].cpu().numpy()
        sel += list(sp)
    rng = np.random.default_rng(seed)
    sel += list(rng.choice(W, size=max(1, int(W * frac)), replace=False))
    return np.unique(np.asarray(sel, np.int64))


def _rows_dot(M: np.ndarray, r: np.ndarray, chunk: int = 1 << 16):
    """(M r, |M| |r|) in float64, over row chunks (M may be 16-bit)."""
    out = np.empty(M.shape[0]), np.empty(M.shape[0])
    ra = np.abs(r)
    for i in range(0, M.shape[0], chunk):
        m = M[i:i + chunk].astype(np.float64)
        out[0][i:i + chunk] = m @ r
        out[1][i:i + chunk] = np.abs(m) @ ra
    return out


def _as_float(a: np.ndarray, dt: str) -> np.ndarray:
    if dt == "bf16":
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).float().numpy()
    return a


def _assert_within(err, bound, what):
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} out of tolerance; worst excess "
                           f"{float((err - bound).max()):.3e}")


def check_forward(hg: HostGraph, X: torch.Tensor, Y: torch.Tensor, rtol: float, plan=None,
                  seed: int = 0) -> dict:
    """Y = A X (Y [16W, N] on the device) against the oracle; returns stats."""
    N = Y.shape[1]
    xdt = DT[X.dtype]
    Xh = raw(X[:, :N])
    Yh = Y.float().cpu().numpy() if Y.dtype == torch.bfloat16 else Y.cpu().numpy()
    sel = select_windows(hg.win, plan, seed)
    Yr, Ya = oracle.bcsr_spmm_windows(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, Xh, xdt, sel)
    rows = (sel[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    err = np.abs(Yh[rows].astype(np.float64) - Yr)
    _assert_within(err, rtol * Ya, f"windows ({sel.size})")
    rng = np.random.default_rng(seed + 1)
    r = rng.standard_normal(N)
    v, va = _rows_dot(_as_float(Xh, xdt), r)
    z, za = oracle.bcsr_spmv(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, v, va, X.shape[0])
    yr, _ = _rows_dot(Yh, r)
    _assert_within(np.abs(yr - z), rtol * za, "projection")
    rel = float(np.linalg.norm(Yh[rows] - Yr) / max(np.linalg.norm(Yr), 1e-300))
    return {"windows": int(sel.size), "rel_fro_windows": rel}


def check_transpose(hg: HostGraph, hgT: HostGraph, Gout: torch.Tensor, out: torch.Tensor, rtol: float,
                    planT=None, seed: int = 0) -> dict:
    """out = A^T Gout (out [num_cols, D]) against the oracle, on A (not on
    the device-built transpose): output rows are picked as windows of the
    transpose (first, last, heaviest, split, 1%)."""
    D = out.shape[1]
    gdt = DT[Gout.dtype]
    Gh = raw(Gout)
    Oh = out.float().cpu().numpy() if out.dtype == torch.bfloat16 else out.cpu().numpy()
    n = out.shape[0]
    wsel = select_windows(hgT.win, planT, seed)
    rows = (wsel[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    rows = rows[rows < n]
    Or, Oa = oracle.bcsr_spmm_t_rows(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, Gh, gdt, n, rows)
    _assert_within(np.abs(Oh[rows].astype(np.float64) - Or), rtol * Oa, f"transpose rows ({rows.size})")
    rng = np.random.default_rng(seed + 1)
    r = rng.standard_normal(D)
    u, ua = _rows_dot(_as_float(Gh, gdt), r)
    z, za = oracle.bcsr_spmv_t(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, u, ua, n)
    o, _ = _rows_dot(Oh, r)
    _assert_within(np.abs(o - z), rtol * za, "transpose projection")
    return {"rows": int(rows.size)}
