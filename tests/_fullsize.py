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

Each check runs two tiers.  The contract tier is the north_star's 1e-2
bound above.  The tight tier is the error the arithmetic itself allows, so
that a kernel that drops or repeats a term fails even where the contract
bound has room for it (one nonzero of a c3 window dropped moves its row
by ~|a| |x| ~ 2e-3 |x|: about 40x the tight bound, 1/4 of the contract's):

  |Y - Y_ref|_ij <= u_out |Y_ref|_ij + C k_i 2^-24 (|A||X|)_ij
                    + k_i 2^-126 + s_out

* the products of two 16-bit values are exact in fp32 (11 + 11 or 8 + 8
  significand bits), so the fp32 accumulation of row i's k_i non-zero
  terms, in any order or grouping (MFMA blocks, slabs, split partials),
  makes at most k_i - 1 roundings, each at most 2^-24 (round to nearest;
  2^-23 if an adder truncated) of a partial sum bounded by (|A||X|)_ij;
  C = 2 covers truncating adders and the second-order terms; adding an
  exact zero (an empty slot) rounds nothing;
* k_i 2^-126: an fp32 adder that flushes subnormal results loses at most
  the smallest normal per addition;
* one rounding to the output type: u_out = 2^-11 (f16), 2^-8 (bf16),
  2^-24 (f32), plus s_out, half the output type's smallest subnormal;
* fp32 inputs: each product rounds once more, C = 3.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle

DT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}

# tight tier constants (module docstring)
U32 = 2.0 ** -24
U_OUT = {"f32": 2.0 ** -24, "f16": 2.0 ** -11, "bf16": 2.0 ** -8}
S_OUT = {"f32": 2.0 ** -150, "f16": 2.0 ** -25, "bf16": 2.0 ** -134}
FTZ = 2.0 ** -126


C_SUM_16 = 2.0


def c_sum(vdt: str, xdt: str) -> float:
    """C of the tight tier: 2 when every product is exact in fp32 (both
    operands 16-bit), 3 when products round (an fp32 operand)."""
    return C_SUM_16 if vdt in ("f16", "bf16") and xdt in ("f16", "bf16") else C_SUM_16 + 1.0


def tight_bound(y_ref, ya, k, vdt: str, xdt: str, ydt: str):
    """The tight tier's bound elementwise (k broadcasts over columns)."""
    k = np.asarray(k, np.float64)
    return U_OUT[ydt] * np.abs(y_ref) + c_sum(vdt, xdt) * U32 * k * ya + k * FTZ + S_OUT[ydt]


def _nonzero(vals: np.ndarray, dt: str) -> np.ndarray:
    """Stored values that are not +-0 (16-bit types as raw bits)."""
    if dt in ("f16", "bf16"):
        return (vals.view(np.uint16) & 0x7FFF) != 0
    return vals != 0


def window_row_nnz(hg: "HostGraph", sel) -> np.ndarray:
    """Non-zero values of each output row of the windows in sel, [16 sel]."""
    out = np.zeros((len(sel), 16), np.int64)
    tc = hg.tc
    for k, w in enumerate(sel):
        a, b = int(hg.win[w]), int(hg.win[w + 1])
        t = hg.vals[a * 16 * tc:b * 16 * tc].reshape(-1, 16, tc)
        out[k] = _nonzero(t, hg.vdt).sum(axis=(0, 2))
    return out.reshape(-1)


def _slot_counts(hg: "HostGraph", axis: int, step: int = 1 << 18) -> np.ndarray:
    """Per tile, non-zero counts summed over `axis` of [tile][row][col]."""
    T = hg.cols.size // hg.tc
    n = 16 if axis == 2 else hg.tc
    cnt = np.empty((T, n), np.int32)
    for i in range(0, T, step):
        t = hg.vals[i * 16 * hg.tc:(i + step) * 16 * hg.tc].reshape(-1, 16, hg.tc)
        cnt[i:i + step] = _nonzero(t, hg.vdt).sum(axis=axis)
    return cnt


def all_row_nnz(hg: "HostGraph") -> np.ndarray:
    """Non-zero values of every output row, [16W]."""
    cnt = _slot_counts(hg, axis=2)
    cs = np.zeros((cnt.shape[0] + 1, 16), np.int64)
    np.cumsum(cnt, axis=0, out=cs[1:])
    return (cs[hg.win[1:]] - cs[hg.win[:-1]]).reshape(-1)


def col_nnz(hg: "HostGraph", n: int) -> np.ndarray:
    """Non-zero values of each column of A (the rows of A^T), [n]."""
    cnt = _slot_counts(hg, axis=1).reshape(-1)
    valid = (hg.cols >= 0) & (hg.cols < n)
    return np.bincount(hg.cols[valid], weights=cnt[valid], minlength=n)[:n]


def rows_nnz_of(win: np.ndarray, vals: np.ndarray, tc: int, dt: str = "f32") -> np.ndarray:
    """Non-zero values of every output row of a BCSR (window offsets and
    values of any stored type), [16W]."""
    class _H:
        pass
    h = _H()
    h.win, h.vals, h.tc, h.vdt = win, vals, tc, dt
    h.cols = np.zeros(vals.size // 16, np.int32)
    return all_row_nnz(h)


def assert_tight(Yd, Yr, Ya, k, vdt: str, xdt: str, ydt: str, what: str = "tight tier") -> float:
    """The tight tier over a whole small product: Yd (device, as float64),
    Yr / Ya the float64 oracle's A X and |A||X| (residual terms included),
    k the non-zero terms of each row [rows]."""
    err = np.abs(np.asarray(Yd, np.float64) - Yr)
    return _assert_within(err, tight_bound(Yr, Ya, np.asarray(k)[:, None], vdt, xdt, ydt), what)


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
    return float((err / np.maximum(bound, 1e-300)).max()) if err.size else 0.0


def flagged(err, bound) -> int:
    """Elements over the bound (for the checker's own sensitivity test)."""
    return int((err > bound).sum())


def check_forward(hg: HostGraph, X: torch.Tensor, Y: torch.Tensor, rtol: float, plan=None,
                  seed: int = 0) -> dict:
    """Y = A X (Y [16W, N] on the device) against the oracle; returns stats."""
    N = Y.shape[1]
    xdt = DT[X.dtype]
    ydt = DT[Y.dtype]
    Xh = raw(X[:, :N])
    Yh = Y.float().cpu().numpy() if Y.dtype == torch.bfloat16 else Y.cpu().numpy()
    sel = select_windows(hg.win, plan, seed)
    Yr, Ya = oracle.bcsr_spmm_windows(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, Xh, xdt, sel)
    rows = (sel[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    err = np.abs(Yh[rows].astype(np.float64) - Yr)
    q_contract = _assert_within(err, rtol * Ya, f"windows ({sel.size})")
    k = window_row_nnz(hg, sel)[:, None]
    q_tight = _assert_within(err, tight_bound(Yr, Ya, k, hg.vdt, xdt, ydt), f"windows, tight tier ({sel.size})")
    rng = np.random.default_rng(seed + 1)
    r = rng.standard_normal(N)
    v, va = _rows_dot(_as_float(Xh, xdt), r)
    z, za = oracle.bcsr_spmv(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, v, va, X.shape[0])
    yr, ya_r = _rows_dot(Yh, r)
    perr = np.abs(yr - z)
    _assert_within(perr, rtol * za, "projection")
    kall = all_row_nnz(hg)
    _assert_within(perr, _proj_tight(ya_r, za, kall, np.abs(r).sum(), hg.vdt, xdt, ydt),
                   "projection, tight tier")
    rel = float(np.linalg.norm(Yh[rows] - Yr) / max(np.linalg.norm(Yr), 1e-300))
    return {"windows": int(sel.size), "rel_fro_windows": rel, "worst_of_contract": q_contract,
            "worst_of_tight": q_tight}


def _proj_tight(y_abs_r, za, k, r_abs_sum, vdt, xdt, ydt):
    """Tight tier on a projection: sum_j |err_ij| |r_j| with the elementwise
    bound, |Y_ref| taken as |Y| (1 + 2 u_out) (the rounding above), plus
    float64 slack for the projections themselves (1e-12 relative)."""
    k = np.asarray(k, np.float64)
    return (U_OUT[ydt] * (1 + 2 * U_OUT[ydt]) * y_abs_r + (c_sum(vdt, xdt) + 1e-6) * U32 * k * za * (1 + 1e-3)
            + (k * FTZ + S_OUT[ydt]) * r_abs_sum + 1e-12 * (za + y_abs_r))


def check_transpose(hg: HostGraph, hgT: HostGraph, Gout: torch.Tensor, out: torch.Tensor, rtol: float,
                    planT=None, seed: int = 0) -> dict:
    """out = A^T Gout (out [num_cols, D]) against the oracle, on A (not on
    the device-built transpose): output rows are picked as windows of the
    transpose (first, last, heaviest, split, 1%)."""
    D = out.shape[1]
    gdt = DT[Gout.dtype]
    odt = DT[out.dtype]
    Gh = raw(Gout)
    Oh = out.float().cpu().numpy() if out.dtype == torch.bfloat16 else out.cpu().numpy()
    n = out.shape[0]
    wsel = select_windows(hgT.win, planT, seed)
    rows = (wsel[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    rows = rows[rows < n]
    Or, Oa = oracle.bcsr_spmm_t_rows(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, Gh, gdt, n, rows)
    err = np.abs(Oh[rows].astype(np.float64) - Or)
    q_contract = _assert_within(err, rtol * Oa, f"transpose rows ({rows.size})")
    kc = col_nnz(hg, n)
    q_tight = _assert_within(err, tight_bound(Or, Oa, kc[rows][:, None], hg.vdt, gdt, odt),
                             f"transpose rows, tight tier ({rows.size})")
    rng = np.random.default_rng(seed + 1)
    r = rng.standard_normal(D)
    u, ua = _rows_dot(_as_float(Gh, gdt), r)
    z, za = oracle.bcsr_spmv_t(hg.win, hg.cols, hg.vals, hg.vdt, hg.tc, u, ua, n)
    o, oa_r = _rows_dot(Oh, r)
    perr = np.abs(o - z)
    _assert_within(perr, rtol * za, "transpose projection")
    _assert_within(perr, _proj_tight(oa_r, za, kc, np.abs(r).sum(), hg.vdt, gdt, odt),
                   "transpose projection, tight tier")
    return {"rows": int(rows.size), "worst_of_contract": q_contract, "worst_of_tight": q_tight}
