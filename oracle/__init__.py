"""CPU oracle for the Graph_RWS hot path -- TEST INFRASTRUCTURE ONLY.

This package is the parity checker for the HIP library in ``graph_rws_amd``.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or as the timed CPU
baseline).  The product path never imports, links or calls anything here.

The arithmetic lives in ``grws_oracle.c`` (plain C, built into
``liboracle.so`` by ``oracle/Makefile``); this module is a thin numpy/ctypes
front end.  Each function names the reference file:line it restates.

Pinning (how each function is checked against something other than itself):
  * csr_to_bcsr        -- against the reference's own converter compiled from
                          /root/reference (oracle/_ref, see build_ref.py), and
                          against BCSR->dense == CSR->dense.
  * bcsr_spmm          -- against scipy.sparse CSR @ X (an independent
                          library routine) on the CSR the BCSR came from, and
                          closed forms (identity, linearity).
  * bcsr_spmm_t        -- against scipy.sparse (A^T) @ G.
  * bcsr_spmm_windows, bcsr_spmv, bcsr_spmv_t, bcsr_spmm_t_rows
                       -- the same products on the stored 16-bit types, for
                          full-size checks: against scipy.sparse on the CSR
                          the BCSR came from, with values and features
                          quantised by numpy/torch (tests/test_oracle.py).
  * reindex_prune      -- hand-built cases with known answers (C truncation of
                          negative columns included).
  * philox4x32_10      -- against vectors produced by ATen's independent
                          PhiloxRNGEngine.h (tests/golden/philox_aten.npz,
                          generator script alongside).
  * sample_hop/relabel -- invariants (distinct, min(deg,k) per node, sorted,
                          in range, bijective relabel, frontier prefix) and a
                          brute-force Floyd restatement in pure Python.
  * repack_subgraph    -- a hand-built known answer, and edge-set equality
                          against the dense matrix of the original graph
                          restricted to the kept rows and columns.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
from typing import Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# GRWS_ORACLE_LIB: another build of grws_oracle.c (the sanitizer build of
# tests/sanitize/ runs the oracle tests against it)
_LIB_PATH = os.environ.get("GRWS_ORACLE_LIB", os.path.join(HERE, "liboracle.so"))
_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_f64p = ctypes.POINTER(ctypes.c_double)
_f32p = ctypes.POINTER(ctypes.c_float)


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_csr_to_bcsr_count.restype = ctypes.c_int64
        L.orc_csr_to_bcsr_count.argtypes = [ctypes.c_int64, _i64p, _i32p, ctypes.c_int64,
                                            ctypes.c_int64, _i64p]
        L.orc_csr_to_bcsr_fill.restype = None
        L.orc_csr_to_bcsr_fill.argtypes = [ctypes.c_int64, _i64p, _i32p, _f64p, ctypes.c_int64,
                                           ctypes.c_int64, _i64p, _i32p, _f64p]
        L.orc_bcsr_spmm_f64.restype = None
        L.orc_bcsr_spmm_f64.argtypes = [ctypes.c_int64, _i64p, _i32p, _f64p, ctypes.c_int64,
                                        ctypes.c_int64, _f64p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, _f64p, _f64p]
        L.orc_bcsr_spmm_f32.restype = None
        L.orc_bcsr_spmm_f32.argtypes = [ctypes.c_int64, ctypes.c_int64, _i64p, _i32p, _f32p,
                                        ctypes.c_int64, ctypes.c_int64, _f32p, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int64, _f32p]
        L.orc_bcsr_spmm_t_f64.restype = None
        L.orc_bcsr_spmm_t_f64.argtypes = [ctypes.c_int64, _i64p, _i32p, _f64p, ctypes.c_int64,
                                          ctypes.c_int64, _f64p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_int64, _f64p, _f64p]
        L.orc_bcsr_spmm_windows_f64.restype = None
        L.orc_bcsr_spmm_windows_f64.argtypes = [ctypes.c_int64, _i64p, _i64p, _i32p, ctypes.c_void_p,
                                                ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                                ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                                ctypes.c_int64, ctypes.c_int64, _f64p, _f64p]
        L.orc_bcsr_spmv_f64.restype = None
        L.orc_bcsr_spmv_f64.argtypes = [ctypes.c_int64, _i64p, _i32p, ctypes.c_void_p, ctypes.c_int32,
                                        ctypes.c_int64, ctypes.c_int64, _f64p, _f64p, ctypes.c_int64,
                                        _f64p, _f64p]
        L.orc_bcsr_spmv_t_f64.restype = None
        L.orc_bcsr_spmv_t_f64.argtypes = [ctypes.c_int64, _i64p, _i32p, ctypes.c_void_p, ctypes.c_int32,
                                          ctypes.c_int64, ctypes.c_int64, _f64p, _f64p, ctypes.c_int64,
                                          _f64p, _f64p]
        L.orc_bcsr_spmm_t_rows_f64.restype = None
        L.orc_bcsr_spmm_t_rows_f64.argtypes = [ctypes.c_int64, _i64p, _i32p, ctypes.c_void_p,
                                               ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                               ctypes.c_int64, ctypes.c_int64, _i32p, ctypes.c_int64,
                                               _f64p, _f64p]
        L.orc_reindex_prune.restype = None
        L.orc_reindex_prune.argtypes = [_i32p, ctypes.c_int64, _f32p, _i32p, ctypes.c_int64,
                                        ctypes.c_int32, ctypes.c_int32, _i32p]
        L.orc_philox4x32_10.restype = None
        L.orc_philox4x32_10.argtypes = [_u32p, _u32p, _u32p]
        L.orc_philox_draws.restype = None
        L.orc_philox_draws.argtypes = [ctypes.c_uint64, _i64p, _u32p, ctypes.c_int64, _u32p]
        L.orc_sample_hop.restype = ctypes.c_int64
        L.orc_sample_hop.argtypes = [_i64p, _i32p, ctypes.c_uint64, _i64p, ctypes.c_int64,
                                     ctypes.c_int, _i32p, _i64p]
        L.orc_relabel.restype = ctypes.c_int64
        L.orc_relabel.argtypes = [_i64p, ctypes.c_int64, _i64p, ctypes.c_int64, _i32p, _i64p]
        L.orc_num_threads.restype = ctypes.c_int
        L.orc_set_num_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


# ----------------------------------------------------------------------------
# CSR -> BCSR  (convert_wrapper.cpp:27-180)
# ----------------------------------------------------------------------------
def csr_to_bcsr(num_rows: int, row_ptr, col_idx, values, tile_rows: int = 16,
                tile_cols: int = 8) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Restates csr_to_bcsr_cpu (convert_wrapper.cpp:27-180).  Values are
    carried in float64 (exact for any f16/bf16/f32 input)."""
    rp = _c(row_ptr, np.int64)
    ci = _c(col_idx, np.int32)
    va = _c(values, np.float64)
    W = (num_rows + tile_rows - 1) // tile_rows
    win = np.zeros(W + 1, np.int64)
    T = lib().orc_csr_to_bcsr_count(num_rows, _p(rp, _i64p), _p(ci, _i32p), tile_rows,
                                    tile_cols, _p(win, _i64p))
    cols = np.empty(T * tile_cols, np.int32)
    vals = np.empty(T * tile_rows * tile_cols, np.float64)
    lib().orc_csr_to_bcsr_fill(num_rows, _p(rp, _i64p), _p(ci, _i32p), _p(va, _f64p),
                               tile_rows, tile_cols, _p(win, _i64p), _p(cols, _i32p),
                               _p(vals, _f64p))
    return win, cols, vals


def ref_csr_to_bcsr(num_rows: int, row_ptr, col_idx, values, tile_rows: int = 16,
                    tile_cols: int = 8):
    """The reference's own converter (oracle/_ref, compiled from
    /root/reference/core/wrapper/convert_wrapper.cpp).  None if not built."""
    mod = _ref_module()
    if mod is None:
        return None
    import torch
    out = mod.csr_to_bcsr_cpu(int(num_rows), torch.as_tensor(_c(row_ptr, np.int64)),
                              torch.as_tensor(_c(col_idx, np.int32)),
                              torch.as_tensor(_c(values, np.float32)), int(tile_rows),
                              int(tile_cols))
    return tuple(t.numpy() for t in out)


_ref_mod = None


def _ref_module():
    global _ref_mod
    if _ref_mod is not None:
        return _ref_mod
    d = os.path.join(HERE, "_ref")
    if not os.path.isdir(d):
        return None
    so = [f for f in os.listdir(d) if f.startswith("ref_convert") and f.endswith(".so")]
    if not so:
        return None
    import torch  # noqa: F401  (the module links libtorch)
    spec = importlib.util.spec_from_file_location("ref_convert", os.path.join(d, so[0]))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    _ref_mod = m
    return m


def bcsr_to_dense(win, cols, vals, tile_rows: int, tile_cols: int, num_cols: int) -> np.ndarray:
    """Dense [16W x num_cols] float64 matrix of a BCSR graph (duplicates cannot
    occur: columns are unique per window)."""
    win = np.asarray(win); cols = np.asarray(cols); vals = np.asarray(vals, np.float64)
    W = len(win) - 1
    D = np.zeros((W * tile_rows, num_cols), np.float64)
    for w in range(W):
        for t in range(win[w], win[w + 1]):
            for c in range(tile_cols):
                col = cols[t * tile_cols + c]
                if col < 0 or col >= num_cols:
                    continue
                D[w * tile_rows:(w + 1) * tile_rows, col] = \
                    vals[t * tile_rows * tile_cols + c:(t + 1) * tile_rows * tile_cols:tile_cols]
    return D


# ----------------------------------------------------------------------------
# SpMM forward / transpose
# ----------------------------------------------------------------------------
def bcsr_spmm(win, cols, vals, tile_rows: int, tile_cols: int, X) -> Tuple[np.ndarray, np.ndarray]:
    """Y = A X and |A||X| in float64 (spmm_tc.cuh:113-193 semantics, all N
    columns).  X may be any float dtype; it is widened exactly."""
    win = _c(win, np.int64); cols = _c(cols, np.int32); vals = _c(vals, np.float64)
    X = _c(X, np.float64)
    if X.ndim != 2:
        raise ValueError("X must be 2-D")
    W = len(win) - 1
    N = X.shape[1]
    Y = np.empty((W * tile_rows, N), np.float64)
    Ya = np.empty_like(Y)
    lib().orc_bcsr_spmm_f64(W, _p(win, _i64p), _p(cols, _i32p), _p(vals, _f64p), tile_rows,
                            tile_cols, _p(X, _f64p), X.shape[0], N, N, _p(Y, _f64p),
                            _p(Ya, _f64p))
    return Y, Ya


def bcsr_spmm_t(win, cols, vals, tile_rows: int, tile_cols: int, G, num_cols: int):
    """G_in = A^T G and |A|^T|G| in float64 (spmm_tc.cuh:211-270 semantics
    without the 1e-9 skip / int32 / D>1024 quirks)."""
    win = _c(win, np.int64); cols = _c(cols, np.int32); vals = _c(vals, np.float64)
    G = _c(G, np.float64)
    W = len(win) - 1
    D = G.shape[1]
    if G.shape[0] < W * tile_rows:
        raise ValueError("G must have at least 16W rows")
    out = np.empty((num_cols, D), np.float64)
    outa = np.empty_like(out)
    lib().orc_bcsr_spmm_t_f64(W, _p(win, _i64p), _p(cols, _i32p), _p(vals, _f64p), tile_rows,
                              tile_cols, _p(G, _f64p), D, D, num_cols, _p(out, _f64p),
                              _p(outa, _f64p))
    return out, outa


def bcsr_spmm_f32_timed(win, cols, vals_f32, tile_rows: int, tile_cols: int, X_f32,
                        w_begin: int, w_end: int) -> np.ndarray:
    """fp32 CPU SpMM over windows [w_begin, w_end) (the timed CPU baseline)."""
    N = X_f32.shape[1]
    Y = np.empty(((w_end - w_begin) * tile_rows, N), np.float32)
    lib().orc_bcsr_spmm_f32(w_begin, w_end, _p(win, _i64p), _p(cols, _i32p),
                            _p(vals_f32, _f32p), tile_rows, tile_cols, _p(X_f32, _f32p),
                            X_f32.shape[0], X_f32.shape[1], N, _p(Y, _f32p))
    return Y


# ----------------------------------------------------------------------------
# Full-size checks on the stored element types (no float64 copy of A)
# ----------------------------------------------------------------------------
_DT = {"f32": (0, np.float32), "f16": (1, np.float16), "bf16": (2, np.uint16)}


def _typed(a, dt: str) -> np.ndarray:
    """a as a contiguous array of the element type dt ("f32", "f16", or
    "bf16" given as its raw uint16 bits)."""
    code, npt = _DT[dt]
    a = np.asarray(a)
    if dt == "bf16" and a.dtype == np.int16:
        a = a.view(np.uint16)
    if a.dtype != npt:
        raise TypeError(f"expected {npt.__name__} data for {dt}, got {a.dtype}")
    return np.ascontiguousarray(a)


def bcsr_spmm_windows(win, cols, vals, vdt: str, tile_cols: int, X, xdt: str, sel):
    """Rows of Y = A X and |A||X| (float64) for the windows in sel: output
    rows 16k..16k+15 belong to window sel[k] (spmm_tc.cuh:113-193 semantics,
    as bcsr_spmm).  vals and X keep their stored element type."""
    win = _c(win, np.int64); cols = _c(cols, np.int32); sel = _c(sel, np.int64)
    vals = _typed(vals, vdt)
    X = _typed(X, xdt)
    if X.ndim != 2:
        raise ValueError("X must be 2-D")
    N = X.shape[1]
    Y = np.empty((sel.size * 16, N), np.float64)
    Ya = np.empty_like(Y)
    lib().orc_bcsr_spmm_windows_f64(sel.size, _p(sel, _i64p), _p(win, _i64p), _p(cols, _i32p),
                                    vals.ctypes.data, _DT[vdt][0], 16, tile_cols, X.ctypes.data,
                                    _DT[xdt][0], X.shape[0], N, N, _p(Y, _f64p), _p(Ya, _f64p))
    return Y, Ya


def bcsr_spmv(win, cols, vals, vdt: str, tile_cols: int, v, v_abs, x_rows: int):
    """z = A v and |A| v_abs over all 16W rows (float64)."""
    win = _c(win, np.int64); cols = _c(cols, np.int32)
    vals = _typed(vals, vdt)
    v = _c(v, np.float64); v_abs = _c(v_abs, np.float64)
    W = len(win) - 1
    z = np.empty(W * 16, np.float64)
    za = np.empty_like(z)
    lib().orc_bcsr_spmv_f64(W, _p(win, _i64p), _p(cols, _i32p), vals.ctypes.data, _DT[vdt][0], 16,
                            tile_cols, _p(v, _f64p), _p(v_abs, _f64p), min(x_rows, v.size),
                            _p(z, _f64p), _p(za, _f64p))
    return z, za


def bcsr_spmv_t(win, cols, vals, vdt: str, tile_cols: int, u, u_abs, num_cols: int):
    """z = A^T u and |A|^T u_abs over num_cols outputs (float64); u has 16W
    entries."""
    win = _c(win, np.int64); cols = _c(cols, np.int32)
    vals = _typed(vals, vdt)
    u = _c(u, np.float64); u_abs = _c(u_abs, np.float64)
    W = len(win) - 1
    if u.size < 16 * W:
        raise ValueError("u must have 16W entries")
    z = np.empty(num_cols, np.float64)
    za = np.empty_like(z)
    lib().orc_bcsr_spmv_t_f64(W, _p(win, _i64p), _p(cols, _i32p), vals.ctypes.data, _DT[vdt][0], 16,
                              tile_cols, _p(u, _f64p), _p(u_abs, _f64p), num_cols, _p(z, _f64p),
                              _p(za, _f64p))
    return z, za


def bcsr_spmm_t_rows(win, cols, vals, vdt: str, tile_cols: int, G, gdt: str, num_cols: int, rows):
    """Rows `rows` (distinct column ids of A) of A^T G and |A|^T |G| in
    float64; G is [16W, D] of type gdt (spmm_tc.cuh:238-269 semantics)."""
    win = _c(win, np.int64); cols = _c(cols, np.int32); rows = _c(rows, np.int64)
    vals = _typed(vals, vdt)
    G = _typed(G, gdt)
    W = len(win) - 1
    if G.ndim != 2 or G.shape[0] < 16 * W:
        raise ValueError("G must be [>=16W, D]")
    D = G.shape[1]
    m = np.full(num_cols, -1, np.int32)
    m[rows] = np.arange(rows.size, dtype=np.int32)
    out = np.empty((rows.size, D), np.float64)
    outa = np.empty_like(out)
    lib().orc_bcsr_spmm_t_rows_f64(W, _p(win, _i64p), _p(cols, _i32p), vals.ctypes.data, _DT[vdt][0], 16,
                                   tile_cols, G.ctypes.data, _DT[gdt][0], D, D, num_cols, _p(m, _i32p),
                                   rows.size, _p(out, _f64p), _p(outa, _f64p))
    return out, outa


def num_threads() -> int:
    return int(lib().orc_num_threads())


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


# ----------------------------------------------------------------------------
# reindex (reindex.cuh:33-102)
# ----------------------------------------------------------------------------
def reindex_prune(in_cols, values, active_windows, tile_rows: int = 16, tile_cols: int = 8):
    """Returns (out_cols, values_after).  `values` is not modified; a pruned
    copy is returned (the reference prunes in place)."""
    ic = _c(in_cols, np.int32)
    va = _c(values, np.float32).copy()
    aw = _c(active_windows, np.int32)
    out = np.empty_like(ic)
    lib().orc_reindex_prune(_p(ic, _i32p), ic.size, _p(va, _f32p), _p(aw, _i32p), aw.size,
                            tile_rows, tile_cols, _p(out, _i32p))
    return out, va


# ----------------------------------------------------------------------------
# Philox + node-wise sampler + relabel (no reference counterpart)
# ----------------------------------------------------------------------------
def philox4x32_10(counter, key) -> np.ndarray:
    c = _c(counter, np.uint32)
    k = _c(key, np.uint32)
    o = np.empty(4, np.uint32)
    lib().orc_philox4x32_10(_p(c, _u32p), _p(k, _u32p), _p(o, _u32p))
    return o


def philox_draws(seed: int, nodes, draws) -> np.ndarray:
    n = _c(nodes, np.int64)
    d = _c(draws, np.uint32)
    o = np.empty(n.size, np.uint32)
    lib().orc_philox_draws(seed, _p(n, _i64p), _p(d, _u32p), n.size, _p(o, _u32p))
    return o


def sample_hop(indptr, indices, seed: int, frontier, k: int):
    """Floyd sampling of min(deg,k) neighbours per frontier node.  Returns
    (edge_dst_local int32[E], edge_src_global int64[E])."""
    ip = _c(indptr, np.int64)
    ix = _c(indices, np.int32)
    fr = _c(frontier, np.int64)
    if k < 1 or k > 64:
        raise ValueError("k must be in [1, 64]")
    cap = max(1, fr.size * k)
    dst = np.empty(cap, np.int32)
    src = np.empty(cap, np.int64)
    E = lib().orc_sample_hop(_p(ip, _i64p), _p(ix, _i32p), seed, _p(fr, _i64p), fr.size, k,
                             _p(dst, _i32p), _p(src, _i64p))
    return dst[:E].copy(), src[:E].copy()


def relabel(frontier, edge_src):
    """Returns (src_local int32[E], next_frontier int64[n_src])."""
    fr = _c(frontier, np.int64)
    es = _c(edge_src, np.int64)
    sl = np.empty(max(1, es.size), np.int32)
    nf = np.empty(max(1, fr.size + es.size), np.int64)
    n = lib().orc_relabel(_p(fr, _i64p), fr.size, _p(es, _i64p), es.size, _p(sl, _i32p),
                          _p(nf, _i64p))
    return sl[:es.size].copy(), nf[:n].copy()


# ----------------------------------------------------------------------------
# quantisation helpers (the same rounding the device applies)
# ----------------------------------------------------------------------------
def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even), returned as float32."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    nan = np.isnan(x)
    out = r.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def gcn_weight(deg_dst, deg_src) -> np.ndarray:
    """1/sqrt((deg_dst+1)(deg_src+1)) in float64 (exact product, correctly
    rounded sqrt and division), rounded once to float32."""
    p = (np.asarray(deg_dst, np.int64) + 1).astype(np.float64) * \
        (np.asarray(deg_src, np.int64) + 1).astype(np.float64)
    return (1.0 / np.sqrt(p)).astype(np.float32)


def coo_to_bcsr(num_rows: int, rows, cols, vals, tile_cols: int):
    """COO (duplicates: last in input order wins) -> BCSR through a stable
    (row, col) ordering and csr_to_bcsr (convert_wrapper.cpp:27-180)."""
    rows = np.asarray(rows, np.int64)
    cols = np.asarray(cols, np.int64)
    vals = np.asarray(vals, np.float64)
    order = np.lexsort((cols, rows))  # stable: ties keep input order
    r, c, v = rows[order], cols[order], vals[order]
    rp = np.zeros(num_rows + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=num_rows), out=rp[1:])
    return csr_to_bcsr(num_rows, rp, c.astype(np.int32), v, 16, tile_cols)


def sample_blocks(indptr, indices, seeds, fanouts, seed: int = 42, tile_cols: int = 16):
    """Host restatement of the node-wise sampler's batch: hop 0 from the
    seeds with fanouts[-1] (sampler.py:204 order), Floyd + relabel per hop,
    a BCSR block per hop with GCN weights from out-degrees.  Returns a list
    (input side first) of dicts with dst, src, val, src_local, src_nodes and
    the BCSR arrays (win, cols, vals as float32)."""
    ip = np.asarray(indptr, np.int64)
    deg = ip[1:] - ip[:-1]
    frontier = np.asarray(seeds, np.int64)
    out = []
    for k in reversed(list(fanouts)):
        dst, src = sample_hop(ip, indices, seed, frontier, k)
        val = gcn_weight(deg[frontier[dst]], deg[src])
        local, nxt = relabel(frontier, src)
        win, cols, vals = coo_to_bcsr(frontier.size, dst, local, val, tile_cols)
        out.insert(0, dict(dst=dst, src=src, val=val, src_local=local, src_nodes=nxt,
                           num_rows=frontier.size, num_cols=nxt.size, win=win, cols=cols,
                           vals=vals.astype(np.float32)))
        frontier = nxt
    return out


# ----------------------------------------------------------------------------
# window top-K sampling (sampling.cuh:65-579, sampling_wrapper.cu:58-438)
# ----------------------------------------------------------------------------
class _Hacs(ctypes.Structure):
    _fields_ = [("static_scores", ctypes.c_void_p), ("window_part_ids", ctypes.c_void_p),
                ("part_starts", ctypes.c_void_p), ("part_ends", ctypes.c_void_p),
                ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("delta", ctypes.c_float),
                ("gamma_bonus", ctypes.c_float), ("score_scale", ctypes.c_float),
                ("use_hacs", ctypes.c_int32), ("locality_enabled", ctypes.c_int32)]


def _window_lib():
    L = lib()
    if not getattr(L, "_window_protos", False):
        L.orc_window_topk.restype = None
        L.orc_window_topk.argtypes = [_i64p, _i32p, _f32p, ctypes.c_int32, _i32p, ctypes.c_int64,
                                      ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, _i32p, _i32p]
        L.orc_window_recompress.restype = None
        L.orc_window_recompress.argtypes = [_i64p, _i32p, _f32p, ctypes.c_int64, ctypes.c_int32,
                                            _i32p, ctypes.c_int64, ctypes.c_int32, _i32p, _i64p,
                                            _i32p, _f32p]
        L.orc_prepare_windows.restype = ctypes.c_int64
        L.orc_prepare_windows.argtypes = [_i32p, ctypes.c_int64, ctypes.c_int32, _i32p, _i32p]
        L._window_protos = True
    return L


def prepare_windows(seeds, tile_rows: int = 16):
    """(active_windows int32, masks int32) of seed ids (sampling_wrapper.cu:283-347)."""
    s = _c(seeds, np.int32)
    w = np.empty(max(1, s.size), np.int32)
    m = np.empty(max(1, s.size), np.int32)
    n = _window_lib().orc_prepare_windows(_p(s, _i32p), s.size, tile_rows, _p(w, _i32p), _p(m, _i32p))
    return w[:n].copy(), m[:n].copy()


def window_sample_layer(win, cols, vals, active, fanout: int, tile_cols: int = 8,
                        warps_per_block: int = 8, hacs: Optional[dict] = None):
    """One layer of the reference's window sampler.  Returns (out_win int64,
    out_cols int32, out_vals float32), sized exactly."""
    win = _c(win, np.int64); cols = _c(cols, np.int32); vals = _c(vals, np.float32)
    act = _c(active, np.int32)
    A = act.size
    S = ((fanout + 31) // 32) * 32
    sampled = np.empty(max(1, A * S), np.int32)
    tiles = np.empty(max(1, A), np.int32)
    keep = []
    hp = None
    if hacs is not None:
        arrs = {k: (None if hacs.get(k) is None else
                    _c(hacs[k], np.float32 if k == "static_scores" else np.int32))
                for k in ("static_scores", "window_part_ids", "part_starts", "part_ends")}
        keep = [a for a in arrs.values() if a is not None]
        h = _Hacs(*(None if arrs[k] is None else arrs[k].ctypes.data
                    for k in ("static_scores", "window_part_ids", "part_starts", "part_ends")),
                  hacs.get("alpha", 1.0), hacs.get("beta", 10.0), hacs.get("delta", 0.0),
                  hacs.get("gamma_bonus", 0.0), hacs.get("score_scale", 100.0),
                  int(hacs.get("use_hacs", 1)), int(hacs.get("locality_enabled", 0)))
        hp = ctypes.byref(h)
    _window_lib().orc_window_topk(_p(win, _i64p), _p(cols, _i32p), _p(vals, _f32p), tile_cols,
                                  _p(act, _i32p), A, fanout, warps_per_block, hp,
                                  _p(sampled, _i32p), _p(tiles, _i32p))
    del keep
    out_win = np.zeros(A + 1, np.int64)
    out_win[1:] = np.cumsum(tiles[:A])
    T = int(out_win[-1])
    oc = np.empty(max(1, T * tile_cols), np.int32)
    ov = np.empty(max(1, T * 16 * tile_cols), np.float32)
    _window_lib().orc_window_recompress(_p(win, _i64p), _p(cols, _i32p), _p(vals, _f32p), vals.size,
                                        tile_cols, _p(act, _i32p), A, fanout, _p(sampled, _i32p),
                                        _p(out_win, _i64p), _p(oc, _i32p), _p(ov, _f32p))
    return out_win, oc[:T * tile_cols].copy(), ov[:T * 16 * tile_cols].copy(), sampled[:A * S].reshape(A, S)


def window_sample_all_layers(win, cols, vals, seeds, fanouts, num_global_nodes: int,
                             tile_cols: int = 8, warps_per_block: int = 8,
                             hacs: Optional[dict] = None):
    """bcsr_sample_all_layers_wrapper (sampling_wrapper.cu:365-438): layers in
    sampling order, each [out_win, out_cols, out_vals, active, masks]."""
    active, masks = prepare_windows(seeds)
    out = []
    for i, f in enumerate(fanouts):
        ow, oc, ov, _ = window_sample_layer(win, cols, vals, active, f, tile_cols,
                                            warps_per_block, hacs)
        out.append([ow, oc, ov, active, masks])
        if i + 1 < len(fanouts):
            nxt = oc.copy()
            nxt[(nxt < 0) | (nxt >= num_global_nodes)] = -1
            active, masks = prepare_windows(nxt)
    return out


def repack_subgraph(win, cols, vals, num_nodes: int, tile_cols: int, window_ids, ratio: float,
                    perm=None, tile_rows: int = 16) -> dict:
    """numpy restatement of BCSRSampler.repack_subgraph (sampler/sampler.py:
    420-690), steps as in the reference: sort and filter the window ids
    (:433-436); gather the windows' tiles (:466-487); internal nodes, window
    then row order, below num_nodes (:492-497); valid neighbour columns,
    unique, minus internal (:503-524); the budget int(internal * ratio)
    with ``perm`` standing for the reference's torch.randperm draw
    (:529-538); input nodes internal + kept (:543); relabel, dropped and
    invalid columns -1 (:551-579); zero the values of -1 columns (:582-604);
    nan_to_num when a NaN is left, after the halo graph counted its edges
    (:607-639); the inner copy masking columns >= internal (:647-688).
    Returns the arrays of both graphs."""
    win = np.asarray(win, np.int64)
    cols = np.asarray(cols, np.int64)
    vals = np.asarray(vals)
    W = win.size - 1
    wid = np.sort(np.asarray(window_ids, np.int64))
    wid = wid[(wid >= 0) & (wid < W)]
    starts, ends = win[wid], win[wid + 1]
    lengths = ends - starts
    new_off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    tiles = (np.concatenate([np.arange(a, b) for a, b in zip(starts, ends)]).astype(np.int64)
             if wid.size else np.zeros(0, np.int64))
    raw_cols = cols.reshape(-1, tile_cols)[tiles].reshape(-1).copy()
    raw_vals = vals.reshape(-1, tile_rows, tile_cols)[tiles].reshape(-1).copy()
    internal = (np.repeat(wid, tile_rows) * tile_rows + np.tile(np.arange(tile_rows), wid.size)).astype(np.int64)
    internal = internal[internal < num_nodes]
    n_int = int(internal.size)
    valid = (raw_cols >= 0) & (raw_cols < num_nodes)
    raw_cols[~valid] = -1
    uniq = np.unique(raw_cols[valid])
    is_int = np.zeros(W * tile_rows, bool)
    is_int[internal] = True
    ext = uniq[~is_int[uniq]]
    budget = int(n_int * ratio)
    if ext.size > budget:
        if perm is None:
            raise ValueError("over budget: pass the permutation the reference would draw")
        kept = np.sort(ext[np.asarray(perm, np.int64)[:budget]])
    else:
        kept = ext
    final = np.concatenate([internal, kept]).astype(np.int64)
    g2l = np.full(max(num_nodes, 1), -1, np.int64)
    g2l[final] = np.arange(final.size)
    new_cols = np.full(raw_cols.shape, -1, np.int64)
    new_cols[valid] = g2l[raw_cols[valid]]
    T = tiles.size
    v3 = raw_vals.reshape(T, tile_rows, tile_cols)
    v3[np.broadcast_to((new_cols.reshape(T, tile_cols) == -1)[:, None, :], v3.shape)] = 0
    nnz_halo = int(np.count_nonzero(raw_vals))
    if np.isnan(raw_vals).any():
        raw_vals = np.nan_to_num(raw_vals, nan=0.0)
    inner_cols = new_cols.copy()
    inner_cols[inner_cols >= n_int] = -1
    inner_vals = raw_vals.copy()
    iv3 = inner_vals.reshape(T, tile_rows, tile_cols)
    iv3[np.broadcast_to((inner_cols.reshape(T, tile_cols) == -1)[:, None, :], iv3.shape)] = 0
    return {"window_ids": wid, "window_offset": new_off, "input_nodes": final, "num_internal": n_int,
            "halo_cols": new_cols.astype(np.int32), "halo_values": raw_vals, "halo_nnz": nnz_halo,
            "inner_cols": inner_cols.astype(np.int32), "inner_values": inner_vals,
            "inner_nnz": int(np.count_nonzero(inner_vals)), "num_external": int(ext.size)}
