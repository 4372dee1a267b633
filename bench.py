#!/usr/bin/env python3
"""Benchmark of the Graph_RWS hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c3] [--gpus 1]

A step is one BCSR SpMM forward Y = A X over the whole synthetic graph of the
chosen BASELINE config (default c3: SBM, 232,965 nodes, ~114.6M nnz, X
[n, 608] float16, 16x16 tiles), inputs resident in HBM.  Prints ONE JSON
line: value = useful SpMM GFLOP/s (2 nnz N / t), with the effective HBM
bandwidth over the algorithmic bytes, a live roofline object for the SpMM
kernel (HIP events on the launch stream) and a CPU baseline (the oracle's
fp32 BCSR SpMM on host cores over a bounded sample of the same windows).
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import platform
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16/bf16

# Bytes per SpMM leaving the L2s, measured with rocprofv3 --pmc (FETCH_SIZE x2.0
# and WRITE_SIZE x1.0, both scaled by a 1 GiB device copy; Infinity-Cache hits
# included, no counter separates them); bench.py cannot read counters itself,
# so the figure of the profiled workload is recorded here and reported only for
# that exact workload.  Sources: the profile file named with each figure
MEASURED_TRAFFIC = {
    # (config, N, x dtype, tile cols, A format): (bytes per SpMM, profile file)
    # grouped tiles, 4 windows per group, slab pairs staged by direct loads
    # into LDS: FETCH 16.88M KiB x2, WRITE 0.277M KiB
    ("c3", 608, "f16", 16, "grouped tiles (4 windows)"): (34.86e9, "profiles/spmm_grp2d_c3_n608_f16.md"),
    # SpMM kernel (351.0 MB read, 55.1 MB written) plus the split-window fixup (14.6 MB)
    ("c2", 128, "f16", 16, "packed tiles"): (420.7e6, "profiles/spmm_buf_c2_n128_f16.md"),
    # SpMM kernel (24.96 GB read, 0.56 GB written) plus the fixup (13 MB)
    ("c4", 112, "bf16", 16, "packed tiles"): (25.534e9, "profiles/spmm_buf_c4_n112_bf16.md"),
}


# HBM bytes of one device BCSR build (the window sort and the fill), measured
# the same way (FETCH_SIZE x2.0 + WRITE_SIZE x1.0 per dispatch), for the
# profiled workload only
BUILD_TRAFFIC = {
    # (config, path): (bytes per build, profile file)
    ("c3", "window by window"): (6.19e9, "profiles/bcsr_build_c3_f16.md"),
}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def build_graph(cfg: str, tc: int, vdt: torch.dtype, dev: torch.device):
    from graph_rws_amd import synth
    from graph_rws_amd.data import BCSRGraph
    t0 = time.time()
    g = synth.config_graph(cfg, device=dev)
    t1 = time.time()
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes,
                           tile_cols=tc, device=dev, values_dtype=vdt)
    torch.cuda.synchronize(dev)
    t2 = time.time()
    return g, G, t1 - t0, t2 - t1


def bench_build(g, dev, cpu: bool, reps: int = 5, cfg: str = "c3") -> dict:
    """The device BCSR build (csr_to_bcsr, H3) of the headline graph: CSR
    (int64 row pointer, int32 columns, f32 values) -> 16x16 BCSR with f16
    values, and the build of its transpose (the backward's operand).  Wall
    time per build (each build synchronises to size its outputs), median of
    `reps`.  Bytes the algorithm moves: the CSR read; window by window, the
    per-edge records and distinct columns written and read back (24 B per
    edge); with the global sort, per radix pass the keys read by the
    histogram (8 B) and keys + payload read and written by the scatter (24 B)
    per edge and the flags/scans over the sorted edges (~16 B per edge); the
    BCSR written once."""
    from graph_rws_amd import builder
    n, nnz = g.num_nodes, g.nnz

    def timed(fn):
        fn()
        torch.cuda.synchronize(dev)
        ts, out = [], None
        for _ in range(reps):
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize(dev)
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2], out

    t_fwd, (win, cols, vals) = timed(lambda: builder.csr_to_bcsr_device(
        n, n, g.row_ptr, g.col_idx, g.values, tile_cols=16, values_dtype=torch.float16))
    W, T = win.numel() - 1, cols.numel() // 16
    # the path the library takes (csrc/bcsr_build.hip): window by window (in
    # LDS up to 16,384 edges a window, larger windows by one work-group from
    # global scratch) unless a window holds more than 2^27 edges, then one
    # global radix sort over (window, column, row) keys
    idx = torch.clamp(torch.arange(0, n + 16, 16, device=g.row_ptr.device), max=n)
    per_window = int(torch.diff(g.row_ptr[idx]).max()) <= (1 << 27)
    out_bytes = 8 * (W + 1) + 4 * T * 16 + 2 * T * 256
    if per_window:
        # row pointers, columns and values read; one 8-byte record per edge
        # and the distinct columns (4 B) written and read back by the fill
        passes = 0
        b_alg = 8 * (n + 1) + 8 * nnz + 24 * nnz + out_bytes
    else:
        bits = max(1, (W - 1).bit_length()) + max(1, (n - 1).bit_length()) + 4
        passes = -(-bits // 8)
        b_alg = 8 * (n + 1) + 8 * nnz + passes * 32 * nnz + 16 * nnz + out_bytes
    t_tr, _ = timed(lambda: builder.transpose_arrays(win, cols, vals, 16, n))
    gbs = b_alg / t_fwd / 1e9
    r = {"workload": f"device BCSR build of the {nnz:,}-edge headline graph: CSR -> 16x16 BCSR, f16 values",
         "ms": round(1e3 * t_fwd, 3), "edges_per_s": round(nnz / t_fwd, 1),
         "path": "window by window" if per_window else "global radix sort", "radix_passes": passes,
         "transpose_ms": round(1e3 * t_tr, 3),
         "transpose_how": "BCSR(A) -> COO -> BCSR(A^T): the COO grouped by window (radix sort over the window "
                          "bits), then built window by window",
         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": int(b_alg),
                      "note": "algorithmic bytes of the path taken: the CSR read, the BCSR written once, and "
                              "the workspace round trip (window by window: 24 B per edge; global sort: "
                              "32 B per edge per radix pass + 16); wall time including the build's syncs"}}
    traffic = BUILD_TRAFFIC.get((cfg, r["path"]))
    if traffic is not None:
        r["roofline"]["traffic"] = traffic[0]
        r["roofline"]["traffic_source"] = traffic[1]
    if cpu:
        import oracle
        rows = n
        e = int(g.row_ptr[rows])
        rp = g.row_ptr[:rows + 1].cpu().numpy()
        ci = g.col_idx[:e].cpu().numpy()
        va = g.values[:e].float().cpu().numpy()
        kind, fn = "reference", lambda: oracle.ref_csr_to_bcsr(rows, rp, ci, va, 16, 16)
        if oracle.ref_csr_to_bcsr(16, rp[:17], ci[:int(rp[16])], va[:int(rp[16])], 16, 16) is None:
            from graph_rws_amd import core
            kind = "port"
            fn = lambda: core.csr_to_bcsr_cpu(rows, torch.from_numpy(rp), torch.from_numpy(ci),
                                              torch.from_numpy(va), 16, 16)
        t0 = time.perf_counter()
        fn()
        t_cpu = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(e / t_cpu, 1), "unit": "edges/s", "cores": os.cpu_count(),
                             "kind": kind,
                             "sample": f"rows 0..{rows} ({e:,} edges) through "
                                       + ("the reference's csr_to_bcsr_cpu (convert_wrapper.cpp, compiled "
                                          "into oracle/_ref, OpenMP)" if kind == "reference"
                                          else "the host converter (csrc/abi.cpp, OpenMP)")
                                       + f", {t_cpu:.2f} s"}
    del win, cols, vals
    torch.cuda.empty_cache()
    return r


def alg_bytes(G, N: int, s_x: int, s_y: int, packed=None, plan=None, grouped=None) -> dict:
    """Bytes one SpMM must move, two ways.

    compulsory: every array the kernel reads, read once, in the format it
    actually reads (packed tiles when the product uses them), every
    referenced X row read once, Y written once.  This is the roofline's
    numerator: a kernel cannot move less.

    gather model: B = 8(W+1) + 4 T tc + s_a T 16 tc + s_x U N + s_y 16 W N,
    each referenced X row counted once per window that references it (no
    reuse across windows).  The caches serve those re-references, so this
    count is modelled L2-side traffic, not a bound on DRAM bytes."""
    W, T, tc = G.num_windows, G.num_tiles, G.tile_cols
    cols = G.original_col_indices
    valid = cols[cols >= 0]
    U = int(valid.numel())
    rows_ref = int(torch.unique(valid[valid < G.num_cols]).numel()) if U else 0
    s_a = G.values_condensed.element_size()
    parts = {
        "win_off": 8 * (W + 1),
        "cols": 4 * T * tc,
        "vals": s_a * T * 16 * tc,
        "x_gather": s_x * U * N,
        "y": s_y * 16 * W * N,
    }
    parts["total"] = sum(parts.values())
    parts["U"] = U
    if grouped is not None:
        # group offsets, union columns, sub-tile headers and values: all the kernel reads of A
        a_read = grouped.nbytes()
        parts["compulsory"] = a_read + s_x * rows_ref * N + parts["y"]
        parts["compulsory_detail"] = {"a_grouped": a_read, "a_format": f"grouped ({grouped.group_size} windows)",
                                      "x_rows_referenced": rows_ref, "x_once": s_x * rows_ref * N}
        return parts
    a_read = (48 * T + s_a * packed.num_values) if packed is not None else parts["vals"]
    items = 16 * plan.num_items if plan is not None else 0
    parts["compulsory"] = (parts["win_off"] + parts["cols"] + a_read + s_x * rows_ref * N + parts["y"]
                           + items)
    parts["compulsory_detail"] = {"a_values": a_read, "a_format": "packed" if packed is not None else "dense",
                                  "x_rows_referenced": rows_ref, "x_once": s_x * rows_ref * N,
                                  "plan_items": items}
    return parts


def row_gather_ceiling(dev, rows: int, pitch_bytes: int, segments: int, n_idx: int, reps: int = 5) -> float:
    """GB/s of grws_probe_row_gather: n_idx random rows (uniform over
    `rows`, seeded) of segments * 128 bytes each from a table of rows x
    pitch_bytes, the SpMM's X-read pattern with nothing else around it.
    Median of reps after one warm-up, HIP events on the stream."""
    from graph_rws_amd.core import _lib as L
    n_idx = n_idx // 8 * 8
    table = torch.zeros(rows * pitch_bytes // 4, dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    idx = torch.randint(0, rows, (n_idx,), device=dev, dtype=torch.int32, generator=gen)
    blocks = 4096
    out = torch.empty(4 * blocks, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev)

    def run():
        L.call("grws_probe_row_gather", L.ptr(table), rows, pitch_bytes, segments, L.ptr(idx), n_idx, L.ptr(out),
               blocks, L.stream_of(dev))

    run()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        run()
        e1.record(s)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1))
    ts.sort()
    del table, idx, out
    return n_idx * segments * 128 / (ts[len(ts) // 2] / 1e3) / 1e9


def copy_peak(dev, nbytes: int = 1 << 30, reps: int = 5) -> float:
    """Read+write GB/s of a device-to-device copy of nbytes (torch's copy
    kernel), median of reps after one warm-up, HIP events on the stream."""
    a = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    s = torch.cuda.current_stream(dev)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        b.copy_(a)
        e1.record(s)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1))
    ts.sort()
    del a, b
    torch.cuda.empty_cache()
    return 2 * nbytes / ts[len(ts) // 2] / 1e6


def cpu_baseline(g, G, X: torch.Tensor, Y: torch.Tensor, rtol: float, budget_s: float = 12.0) -> dict:
    """The CPU path beside the headline, and the check of the timed Y.

    Timed: torch.sparse CSR fp32 A @ X over the whole graph (the CPU SpMM
    the baseline plan names; the reported value), and the oracle's fp32
    BCSR SpMM (the reference kernel's arithmetic on host cores) over the
    first windows until ~budget_s (reported beside it).  Untimed, two tiers:

    * contract (north_star): every timed window of the GPU's Y against the
      fp32 oracle, |Y - Y_cpu| <= (rtol + 2e-4) |A||X| (the fp32 sum's own
      error is far below 2e-4 here), and a projection of every row onto a
      seeded r in float64, |Y r - A (X r)| <= rtol |A| (|X| |r|);
    * tight (the arithmetic's own bound, so that a dropped or repeated term
      fails): 16-bit products are exact in fp32 and row i's k_i non-zero
      terms make at most k_i - 1 fp32 roundings (2 k_i 2^-24 |A||X| with a
      truncating adder), the oracle's fp32 sum at most k_i 2^-24 |A||X|
      more, then one rounding to the output type (u_out |Y|):
      |Y - Y_cpu| <= u_out |Y_cpu| + (3 k_i + 1) 2^-24 |A||X| + k_i 2^-126
      + s_out, and on the projection u_out (1 + 2 u_out) |Y| |r| +
      2 k_i 2^-24 |A| (|X| |r|) (+ the same small terms)."""
    import numpy as np
    import oracle
    from graph_rws_amd.core.ops import host_threads
    oracle.set_num_threads(host_threads())
    win = G.window_offset.cpu().numpy()
    cols = G.original_col_indices.cpu().numpy()
    vals = G.values_condensed.float().cpu().numpy()
    vabs = np.abs(vals)
    Xh = X.float().cpu().numpy()
    Xabs = np.abs(Xh)
    Yd = Y.float().cpu().numpy()
    rp = g.row_ptr.cpu().numpy()
    W = G.num_windows
    N = Xh.shape[1]
    ydt = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[Y.dtype]
    u_out = {"f16": 2.0 ** -11, "bf16": 2.0 ** -8, "f32": 2.0 ** -24}[ydt]
    s_out = {"f16": 2.0 ** -25, "bf16": 2.0 ** -134, "f32": 2.0 ** -150}[ydt]
    exact_products = X.dtype != torch.float32 and G.values_condensed.dtype != torch.float32
    c_dev = 2.0 if exact_products else 3.0
    k_rows = _row_nonzeros(G)  # non-zero values per output row, [16W] int64
    done, t_total, nnz = 0, 0.0, 0
    worst = 0.0
    worst_t = 0.0
    step = 64
    oracle.bcsr_spmm_f32_timed(win, cols, vals, 16, G.tile_cols, Xh, 0, min(W, 4))  # warm
    while done < W and t_total < budget_s:
        e = min(W, done + step)
        t0 = time.perf_counter()
        Yc = oracle.bcsr_spmm_f32_timed(win, cols, vals, 16, G.tile_cols, Xh, done, e)
        t_total += time.perf_counter() - t0
        Ya = oracle.bcsr_spmm_f32_timed(win, cols, vabs, 16, G.tile_cols, Xabs, done, e)
        err = np.abs(Yd[16 * done:16 * e].astype(np.float64) - Yc)
        worst = max(worst, float(np.max(err / np.maximum((rtol + 2e-4) * Ya, 1e-30))))
        k = k_rows[16 * done:16 * e, None].astype(np.float64)
        tb = (u_out * np.abs(Yc) + ((c_dev + 1) * k + 1) * 2.0 ** -24 * Ya.astype(np.float64) * (1 + 1e-4)
              + k * 2.0 ** -126 + s_out)
        worst_t = max(worst_t, float(np.max(err / tb)))
        nnz += int(rp[min(e * 16, g.num_nodes)] - rp[min(done * 16, g.num_nodes)])
        done = e
        step = min(step * 2, 4096)
    gflops = 2.0 * nnz * N / t_total / 1e9
    # projection of every row, float64
    r = np.random.default_rng(17).standard_normal(N)
    v = Xh.astype(np.float64) @ r
    va = Xabs.astype(np.float64) @ np.abs(r)
    z, za = oracle.bcsr_spmv(win, cols, vals, "f32", G.tile_cols, v, va, Xh.shape[0])
    Y64 = Yd.astype(np.float64)
    yr = Y64 @ r
    ya_r = np.abs(Y64) @ np.abs(r)
    del Y64
    perr = np.abs(yr - z)
    proj = float(np.max(perr / np.maximum(rtol * za, 1e-300)))
    k = k_rows.astype(np.float64)
    ptb = (u_out * (1 + 2 * u_out) * ya_r + (c_dev + 1e-6) * k * 2.0 ** -24 * za * (1 + 1e-3)
           + (k * 2.0 ** -126 + s_out) * float(np.abs(r).sum()) + 1e-12 * (za + ya_r))
    proj_t = float(np.max(perr / ptb))
    parity = {"pass": bool(worst <= 1.0 and proj <= 1.0 and worst_t <= 1.0 and proj_t <= 1.0),
              "elementwise": f"windows 0..{done} of {W} against the fp32 oracle, bound (rtol + 2e-4) |A||X|, "
                             f"rtol {rtol}",
              "elementwise_worst_err_over_bound": round(worst, 5),
              "projection": f"all {16 * W} rows: Y r against A (X r) in float64, bound rtol |A| (|X| |r|)",
              "projection_worst_err_over_bound": round(proj, 5),
              "tight_tier": "the arithmetic's own bound: u_out |Y| + (C + 1) k_i 2^-24 |A||X| elementwise, "
                            f"C = {c_dev:g}, u_out = 2^{int(np.log2(u_out))}; k_i = row i's non-zeros",
              "tight_elementwise_worst_err_over_bound": round(worst_t, 5),
              "tight_projection_worst_err_over_bound": round(proj_t, 5)}
    del vals, vabs, Xabs, Yd
    # torch.sparse CSR fp32 over the whole graph: the CPU SpMM this product is
    # measured against (the same A @ X on the host cores)
    torch.set_num_threads(host_threads())
    A = torch.sparse_csr_tensor(g.row_ptr.cpu(), g.col_idx.cpu().long(), g.values.cpu().float(),
                                size=(g.num_nodes, g.num_nodes))
    Xt = torch.from_numpy(Xh)
    t0 = time.perf_counter()
    A @ Xt
    t_first = time.perf_counter() - t0
    ts = [t_first]
    if t_first < 10.0:
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            A @ Xt
            ts.append(time.perf_counter() - t0)
        ts.sort()
    t_sp = ts[len(ts) // 2]
    return {"value": round(2.0 * g.nnz * N / t_sp / 1e9, 3), "unit": "GFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": "torch.sparse_csr fp32 A @ X over the whole graph (the CPU SpMM of the baseline "
                      f"plan), {1e3 * t_sp:.1f} ms, "
                      + ("median of 3 after 1 warm-up" if len(ts) == 3 else "one run"),
            "oracle_port": {"value": round(gflops, 3), "unit": "GFLOP/s", "cores": int(oracle.num_threads()),
                            "sample": f"windows 0..{done} of {W} ({nnz} nnz, {100.0 * done / W:.1f}% of "
                                      f"the graph), fp32, {t_total:.1f} s; oracle/grws_oracle.c "
                                      "orc_bcsr_spmm_f32 (the reference kernel's arithmetic)"},
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "torch_threads": torch.get_num_threads(), "parity": parity}


def _row_nonzeros(G) -> "np.ndarray":
    """Non-zero stored values of every output row of G, [16W] int64 (host),
    counted on the device."""
    T, tc, W = G.num_tiles, G.tile_cols, G.num_windows
    v = G.values_condensed.view(T, 16, tc)
    cnt = (v != 0).sum(dim=2)  # [T, 16]
    cs = torch.zeros((T + 1, 16), dtype=torch.int64, device=v.device)
    torch.cumsum(cnt, dim=0, out=cs[1:])
    w = G.window_offset
    k = (cs[w[1:]] - cs[w[:-1]]).reshape(-1).cpu().numpy()
    del cs, cnt
    return k


def sampling_bytes(blk) -> int:
    """Algorithmic bytes of one sampled hop: 16 F + 36 E plus its BCSR block
    (window offsets, column slots, values)."""
    F, E, T, tc = blk.num_rows, blk.num_sampled_edges, blk.num_tiles, blk.tile_cols
    W = (F + 15) // 16
    return (16 * F + 36 * E + 8 * (W + 1) + 4 * T * tc
            + blk.values_condensed.element_size() * T * 16 * tc)


def bench_sampling(dev, batches: int, warmup: int, cpu: bool) -> dict:
    """c5: one batch = 1,024 distinct uniform seeds, 3 hops with fanouts
    [15, 10, 5] (hop 0 from the seeds draws 5), Philox seed 42, unique +
    relabel and a 16x16 BCSR block per hop, on the 111M-node, ~1.6B-edge
    power-law CSR resident in HBM.  Rate = sampled edges / batch wall time
    (the batch synchronises the stream at its end)."""
    from graph_rws_amd import synth
    from graph_rws_amd.sampler import NeighborSampler
    c = synth.C5
    t0 = time.time()
    g = synth.c5_graph(device=dev)
    torch.cuda.synchronize(dev)
    t_gen = time.time() - t0
    s = NeighborSampler(c["fanouts"], seed=c["philox_seed"], tile_cols=16)
    seed_sets = [synth.distinct_seeds(g.num_nodes, c["batch"], seed=1000 + b, device=dev)
                 for b in range(warmup + batches)]
    for b in range(warmup):
        s.sample_layers(g.row_ptr, g.col_idx, seed_sets[b])
    torch.cuda.synchronize(dev)
    edges, times, blocks = 0, [], None
    b_alg = 0
    gc.collect()
    for b in range(warmup, warmup + batches):
        t1 = time.perf_counter()
        blocks = s.sample_layers(g.row_ptr, g.col_idx, seed_sets[b])
        torch.cuda.synchronize(dev)
        times.append(time.perf_counter() - t1)
        edges += sum(x.num_sampled_edges for x in blocks)
        b_alg += sum(sampling_bytes(x) for x in blocks)
    total = sum(times)
    sgbs = b_alg / total / 1e9
    out = {
        "mode": "eager (grws_sample_blocks per batch); the captured mode below replays the same call "
                "from a HIP graph and is the one the mini-batch engine runs",
        "workload": "c5 mini-batch sampling (Philox fanout [15,10,5], unique+relabel, per-hop BCSR)",
        "graph": {"nodes": g.num_nodes, "edges": g.nnz, "indptr": "int64", "indices": "int32"},
        "batches": batches, "seeds_per_batch": c["batch"],
        "sampled_edges_per_s": round(edges / total, 1),
        "batch_ms": round(1e3 * total / batches, 4),
        "edges_per_batch": round(edges / batches, 1),
        "hop_edges_last_batch": [x.num_sampled_edges for x in blocks],
        "input_nodes_last_batch": int(blocks[0].num_cols),
        "generate_s": round(t_gen, 2),
        "dispatches_per_batch": 4 * len(c["fanouts"]) + 2,
        "host_syncs_per_batch": 1,
        "roofline_eager": {"bound": "hbm (random 8-64 B reads: latency bound in practice)",
                     "achieved": round(sgbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(sgbs / HBM_PEAK_GBS, 5),
                     "bytes_per_batch": round(b_alg / batches),
                     "bytes": "per hop 16 F + 36 E (indptr pair and frontier id per node; per edge the "
                              "index, the source's degree, three relabel passes of 8 B) plus the block "
                              "written"},
    }
    # the same plain call replayed from a HIP graph (NeighborSampler(capture=
    # True): grws_sample_blocks_enqueue captured once per batch shape, the
    # outputs copied out of the static buffers in one launch)
    sp = NeighborSampler(c["fanouts"], seed=c["philox_seed"], tile_cols=16, capture=True)
    for b in range(warmup):
        sp.sample_layers(g.row_ptr, g.col_idx, seed_sets[b])
    torch.cuda.synchronize(dev)
    tp, pe, pb = [], 0, 0
    for b in range(warmup, warmup + batches):
        t1 = time.perf_counter()
        bl = sp.sample_layers(g.row_ptr, g.col_idx, seed_sets[b])
        torch.cuda.synchronize(dev)
        tp.append(time.perf_counter() - t1)
        pe += sum(x.num_sampled_edges for x in bl)
        pb += sum(sampling_bytes(x) for x in bl)
    tpt = sum(tp)
    out["captured"] = {
        "batch_ms": round(1e3 * tpt / batches, 4),
        "sampled_edges_per_s": round(pe / tpt, 1),
        "replays": sum(x.replays for x in sp._captures.values()),
        "note": "the plain call replayed from a HIP graph captured in the warm-up (the engine's mode); per "
                "batch one launch staging the seeds and their count, the replay, the counters read back (the "
                "batch's one sync) and one copy launch for the outputs"}
    # the record's roofline: the captured call, the mode the engine runs
    out["roofline"] = {"bound": "hbm (random 8-64 B reads: latency bound in practice)",
                       "mode": "captured (replayed from a HIP graph)",
                       "achieved": round(pb / tpt / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(pb / tpt / 1e9 / HBM_PEAK_GBS, 5), "bytes_per_batch": round(pb / batches),
                       "bytes": "per hop 16 F + 36 E (indptr pair and frontier id per node; per edge the "
                                "index, the source's degree, three relabel passes of 8 B) plus the block "
                                "written"}
    del sp
    # the mini-batch engine's call: the same batches with the transposes of
    # the blocks whose backward multiplies by A^T (layers 1 and 2 of the
    # 3-layer model) built in the same device call
    want = [False, True, True]
    for b in range(warmup):
        s.sample_layers(g.row_ptr, g.col_idx, seed_sets[b], transposes=want)
    torch.cuda.synchronize(dev)
    tt = []
    for b in range(warmup, warmup + batches):
        t1 = time.perf_counter()
        s.sample_layers(g.row_ptr, g.col_idx, seed_sets[b], transposes=want)
        torch.cuda.synchronize(dev)
        tt.append(time.perf_counter() - t1)
    out["with_transposes"] = {
        "transposes": "layers 1 and 2 (grws_sample_blocks_transposed)",
        "batch_ms": round(1e3 * sum(tt) / batches, 4),
        "host_syncs_per_batch": 1,
        "note": "per transposed hop: slot keys, a 2-pass radix sort by source window, the windows' "
                "slot ranges, tiles per window, a scan and the fill"}
    # the same call replayed from a HIP graph (NeighborSampler(capture=True):
    # grws_sample_blocks_enqueue captured once, the outputs copied out of the
    # static buffers in one launch)
    sc = NeighborSampler(c["fanouts"], seed=c["philox_seed"], tile_cols=16, capture=True)
    for b in range(warmup):
        sc.sample_layers(g.row_ptr, g.col_idx, seed_sets[b], transposes=want)
    torch.cuda.synchronize(dev)
    tc_ = []
    for b in range(warmup, warmup + batches):
        t1 = time.perf_counter()
        sc.sample_layers(g.row_ptr, g.col_idx, seed_sets[b], transposes=want)
        torch.cuda.synchronize(dev)
        tc_.append(time.perf_counter() - t1)
    out["with_transposes_captured"] = {
        "batch_ms": round(1e3 * sum(tc_) / batches, 4),
        "replays": sum(x.replays for x in sc._captures.values()),
        "note": "the transposed call replayed from a HIP graph captured in the warm-up; per batch a "
                "seed copy, the replay, the counters read back (the batch's one sync) and one copy "
                "launch for the outputs"}
    if cpu:
        import numpy as np
        import oracle
        ip = g.row_ptr.cpu().numpy()
        ix = g.col_idx.cpu().numpy()
        seeds = seed_sets[-1].cpu().numpy()
        t1 = time.perf_counter()
        ref = oracle.sample_blocks(ip, ix, seeds, c["fanouts"], seed=c["philox_seed"], tile_cols=16)
        t_cpu = time.perf_counter() - t1
        e_cpu = sum(int(r["dst"].size) for r in ref)
        same = all(
            np.array_equal(b.src_nodes.cpu().numpy(), r["src_nodes"])
            and np.array_equal(b.window_offset.cpu().numpy(), r["win"])
            and np.array_equal(b.original_col_indices.cpu().numpy(), r["cols"])
            and np.array_equal(b.values_condensed.cpu().numpy(), r["vals"])
            for b, r in zip(blocks, ref))
        out["bit_exact_vs_oracle_last_batch"] = bool(same)
        out["cpu_baseline"] = {
            "value": round(e_cpu / t_cpu, 1), "unit": "sampled edges/s",
            "cores": int(oracle.num_threads()),
            "kind": "port",
            "sample": f"one batch ({e_cpu} edges): oracle.sample_blocks (grws_oracle.c Floyd + "
                      f"relabel on 1 thread, numpy weights, C csr_to_bcsr on OpenMP threads), "
                      f"{t_cpu:.2f} s"}
        del ip, ix
    del g
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# GCN step / epoch (models/model.py:212-266, helper/engine.py:44-83)
# ---------------------------------------------------------------------------
GCN_CONFIGS = {
    # config: (feature dim, padded dim, feature kind, hidden, classes, layers, dtype name)
    "c1": (1433, 1433, "binary", 16, 7, 2, "f32"),
    "c3": (602, 608, "normal", 256, 41, 3, "f16"),
    "c4": (100, 112, "normal", 256, 47, 3, "bf16"),
}


class _CpuSpmm(torch.autograd.Function):
    """A @ X on host cores with torch.sparse CSR and a precomputed CSR of A^T
    for the backward (the same cached-transpose scheme as the GPU path)."""

    @staticmethod
    def forward(ctx, A, AT, x):
        ctx.AT = AT
        return A @ x

    @staticmethod
    def backward(ctx, g):
        return None, None, ctx.AT @ g


class _CpuGCN(torch.nn.Module):
    """GCN_BCSR's arithmetic (layer.py:95-191, model.py:212-266) on torch
    CPU tensors in float32: h = A (h Wn) + h Ws, then ReLU, LayerNorm and
    dropout between layers."""

    def __init__(self, dims, dropout):
        super().__init__()
        self.wn = torch.nn.ParameterList(torch.nn.Parameter(torch.empty(a, b)) for a, b in zip(dims, dims[1:]))
        self.ws = torch.nn.ParameterList(torch.nn.Parameter(torch.empty(a, b)) for a, b in zip(dims, dims[1:]))
        for p in list(self.wn) + list(self.ws):
            torch.nn.init.xavier_uniform_(p)
        self.norms = torch.nn.ModuleList(torch.nn.LayerNorm(d) for d in dims[1:-1])
        self.dropout = torch.nn.Dropout(dropout)

    def forward(self, A, AT, x):
        h = x
        for l in range(len(self.wn)):
            h = _CpuSpmm.apply(A, AT, h @ self.wn[l]) + h @ self.ws[l]
            if l < len(self.wn) - 1:
                h = self.dropout(self.norms[l](torch.relu(h)))
        return h


def cpu_gcn_epoch(g, X, labels, train_idx, dims, dropout: float) -> float:
    """Seconds of one CPU training epoch (forward, CE loss, backward,
    clip_grad_norm_(1.0), Adam) on the same graph and features."""
    import numpy as np
    import scipy.sparse as sps
    n = g.num_nodes
    rp, ci, va = g.row_ptr.cpu(), g.col_idx.cpu(), g.values.cpu()
    A = torch.sparse_csr_tensor(rp, ci.long(), va, size=(n, n))
    At = sps.csr_matrix((va.numpy(), ci.numpy(), rp.numpy()), shape=(n, n)).T.tocsr()
    AT = torch.sparse_csr_tensor(torch.from_numpy(At.indptr.astype(np.int64)),
                                 torch.from_numpy(At.indices.astype(np.int64)),
                                 torch.from_numpy(At.data), size=(n, n))
    model = _CpuGCN(dims, dropout)
    opt = torch.optim.Adam(model.parameters(), lr=0.01)
    x = X.float().cpu()
    lab, idx = labels.cpu(), train_idx.cpu()
    t0 = time.perf_counter()
    opt.zero_grad()
    out = model(A, AT, x)
    loss = torch.nn.functional.cross_entropy(out[idx], lab[idx])
    loss.backward()
    torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
    opt.step()
    return time.perf_counter() - t0


def bench_gcn_graphed(G, X, labels, train_idx, d_pad, hidden, classes, layers, dt, dev, epochs: int,
                      warmup: int) -> dict:
    """The same step captured once on a HIP graph and replayed
    (GraphedFullStep): a fresh model of the same init, Adam with
    capturable=True; median over at least 20 replays."""
    from graph_rws_amd.helper import GraphedFullStep
    from graph_rws_amd.models import GCN_BCSR
    torch.manual_seed(13)
    model_g = GCN_BCSR(d_pad, hidden, classes, layers, dropout=0.5, use_checkpoint=False).to(dev)
    opt_g = torch.optim.Adam(model_g.parameters(), lr=0.01, capturable=True)
    step = GraphedFullStep(model_g, G, X, labels, train_idx, opt_g, dev, warmup=max(2, warmup),
                           autocast_dtype=None if dt == torch.float32 else dt)
    n_g = max(epochs, 20)
    step()
    torch.cuda.synchronize(dev)
    tg = []
    for _ in range(n_g):
        t0 = time.perf_counter()
        loss_g, _ = step()
        torch.cuda.synchronize(dev)
        tg.append(time.perf_counter() - t0)
    tg.sort()
    return {"epoch_ms": round(1e3 * tg[len(tg) // 2], 3), "epoch_ms_min": round(1e3 * tg[0], 3),
            "epochs": n_g, "final_loss": round(float(loss_g), 4),
            "how": "the same step captured once on a HIP graph (torch.cuda.graph) and replayed"}


def bench_gcn(cfg: str, dev, epochs: int, warmup: int, cpu: bool, graphed: bool = True) -> dict:
    """Full-graph training epochs of GCN_BCSR on config `cfg` (c1: the tiny
    fp32 step; c3, c4: 3 layers, hidden 256, autocast to the config dtype,
    BCSR values in that dtype, 16x16 tiles).  Epoch = forward + loss +
    backward + clip + Adam, synchronised at its end."""
    from graph_rws_amd import synth
    from graph_rws_amd.data import BCSRGraph
    from graph_rws_amd.helper import train_epoch_full
    from graph_rws_amd.models import GCN_BCSR
    d_raw, d_pad, kind, hidden, classes, layers, dname = GCN_CONFIGS[cfg]
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dname]
    g = synth.config_graph(cfg, device=dev)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes,
                           tile_cols=16, device=dev, values_dtype=dt)
    X = synth.features(g.num_nodes, d_raw, pad_to=d_pad, kind=kind, seed=11, device=dev).to(dt)
    gen = torch.Generator(device=dev)
    gen.manual_seed(12)
    labels = torch.randint(0, classes, (g.num_nodes,), generator=gen, device=dev)
    train_idx = torch.nonzero(torch.rand(g.num_nodes, generator=gen, device=dev) < 0.66).view(-1)
    torch.manual_seed(13)
    model = GCN_BCSR(d_pad, hidden, classes, layers, dropout=0.5, use_checkpoint=False).to(dev)
    opt = torch.optim.Adam(model.parameters(), lr=0.01)

    def epoch():
        if dt == torch.float32:
            return train_epoch_full(model, G, X, labels, train_idx, opt, dev, sync=False)
        with torch.autocast("cuda", dtype=dt):
            return train_epoch_full(model, G, X, labels, train_idx, opt, dev, sync=False)

    for _ in range(warmup):
        epoch()
    torch.cuda.synchronize(dev)
    times = []
    for _ in range(epochs):
        t0 = time.perf_counter()
        loss, _ = epoch()
        torch.cuda.synchronize(dev)
        times.append(time.perf_counter() - t0)
    times.sort()
    out = {"workload": f"{cfg} full-graph GCN_BCSR epoch (fwd+bwd+clip+Adam)",
           "nodes": g.num_nodes, "nnz": g.nnz, "features": d_pad, "hidden": hidden,
           "classes": classes, "layers": layers, "dtype": dname, "tile": "16x16",
           "epochs": epochs, "epoch_ms": round(1e3 * times[len(times) // 2], 3),
           "epoch_ms_min": round(1e3 * times[0], 3), "final_loss": round(float(loss), 4)}
    if graphed:
        out["graphed"] = bench_gcn_graphed(G, X, labels, train_idx, d_pad, hidden, classes, layers, dt,
                                           dev, epochs, warmup)
    if cpu:
        torch.set_num_threads(os.cpu_count() or 1)
        dims = [d_pad] + [hidden] * (layers - 1) + [classes]
        if cfg == "c1":
            cpu_gcn_epoch(g, X, labels, train_idx, dims, 0.5)  # warm-up
            ts = sorted(cpu_gcn_epoch(g, X, labels, train_idx, dims, 0.5) for _ in range(3))
            t_cpu, note = ts[1], "median of 3 after 1 warm-up"
        else:
            t_cpu, note = cpu_gcn_epoch(g, X, labels, train_idx, dims, 0.5), "one epoch"
        out["cpu_baseline"] = {"value": round(1e3 * t_cpu, 2), "unit": "ms per epoch",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"{note}: the same model arithmetic in fp32 on "
                                         "torch.sparse CSR (A and a precomputed A^T) over the "
                                         "whole graph"}
    del G, X, model, opt, g
    torch.cuda.empty_cache()
    return out


def bench_minibatch(dev, batches: int, warmup: int) -> dict:
    """c5 mini-batch training: per batch, 1,024 seeds, NeighborSampler
    ([15,10,5], Philox seed 42), the input features gathered from the
    111M x 128 fp16 matrix in HBM, then a 3-layer GCN_BCSR step (hidden 256,
    172 classes, fp16 autocast, CE loss, clip, Adam), sampling pipelined one
    batch ahead on a side stream (train_epoch_node_sampling).  Timed twice
    on the same seeds: the eager step, and the step replayed from HIP graphs
    captured per bucket of batch shapes (GraphedBlockStep).  A third,
    untimed pass times each forward SpMM with events (the SpMM column)."""
    from graph_rws_amd import synth
    from graph_rws_amd.core import ops as _ops
    from graph_rws_amd.helper import EpochTimer, GraphedBlockStep, train_epoch_node_sampling
    from graph_rws_amd.models import GCN_BCSR
    from graph_rws_amd.sampler import NeighborSampler
    c = synth.C5
    t0 = time.time()
    g = synth.c5_graph(device=dev)
    X = synth.features(g.num_nodes, c["feat"], dtype=torch.float16, seed=31, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(32)
    labels = torch.randint(0, c["classes"], (g.num_nodes,), generator=gen, device=dev)
    torch.cuda.synchronize(dev)
    t_gen = time.time() - t0
    torch.manual_seed(33)
    model = GCN_BCSR(c["feat"], 256, c["classes"], 3, dropout=0.5, use_checkpoint=False).to(dev)
    # torch's fused Adam (one kernel per step instead of ~17 foreach kernels),
    # stepping on the device so that the step can be captured
    opt = torch.optim.Adam(model.parameters(), lr=0.003, capturable=True, fused=True)
    # batches replayed from HIP graphs on both sides: the sampler's call
    # (one capture per bucket of 64 seed counts) and the model step
    sampler = NeighborSampler(c["fanouts"], seed=c["philox_seed"], tile_cols=16,
                              values_dtype=torch.float16, capture=True)
    graphed = GraphedBlockStep(model, opt, dev, autocast_dtype=torch.float16)

    def run(nb, seed, step=None):
        idx = synth.distinct_seeds(g.num_nodes, c["batch"] * nb, seed=seed, device=dev).cpu()
        timer = EpochTimer()
        e0, b0 = sampler.total_edges, sampler.total_batches
        torch.cuda.synchronize(dev)
        t = time.perf_counter()
        with torch.autocast("cuda", dtype=torch.float16):
            loss, _ = train_epoch_node_sampling(model, g, X, labels, idx, opt, dev, sampler,
                                                batch_size=c["batch"], timer=timer, pipeline=True,
                                                graphed=step)
        torch.cuda.synchronize(dev)
        return (time.perf_counter() - t, sampler.total_edges - e0, sampler.total_batches - b0,
                loss, timer.get_epoch_stats())

    # the objects earlier legs left are moved out of the collector's reach
    # (gc.freeze): a full collection over them inside a timed epoch cost
    # ~0.5 ms per batch
    gc.collect()
    gc.freeze()
    # warm-up epochs on other seed sets: GEMM kernels for the batch shapes
    # seen load lazily (a one-off stall of tens of ms on first use), and the
    # graphed step captures the buckets these shapes fall in
    for e in range(2):
        run(warmup, 40 + e)
    wall, edges, nb, loss, stats = run(batches, 42)
    # graphed warm-up epochs until one captures no new bucket (at most 6)
    for e in range(6):
        c0 = graphed.captures
        run(warmup, 50 + e, graphed)
        if e >= 1 and graphed.captures == c0:
            break
    cap0 = graphed.captures
    g_wall, g_edges, g_nb, g_loss, g_stats = run(batches, 42, graphed)
    g_caps = graphed.captures - cap0
    # the SpMM column: each forward SpMM timed with events (a sync per call)
    _ops.TIMING = True
    try:
        _, _, _, _, t_stats = run(min(batches, 10), 43)
    finally:
        _ops.TIMING = False
    out = {"workload": "c5 mini-batch GCN step (sample + feature gather + fwd/bwd/Adam), pipelined",
           "graph": {"nodes": g.num_nodes, "edges": g.nnz}, "features": [g.num_nodes, c["feat"], "f16"],
           "batches": g_nb, "warmup": f"2 eager + {e + 1} graphed epochs x {warmup} batches (until one captured no new bucket)",
           "batch_ms": round(1e3 * g_wall / g_nb, 3),
           "step": "replayed from HIP graphs (GraphedBlockStep); the sampler's call too (capture=True)",
           "sampler_replays": sum(x.replays for x in sampler._captures.values()),
           "sampled_edges_per_s_in_training": round(g_edges / g_wall, 1),
           "edges_per_batch": round(g_edges / g_nb, 1), "final_loss": round(float(g_loss), 4),
           "stage_ms_per_batch": {k: round(v, 3) for k, v in g_stats.items() if k != "SpMM"},
           "buckets_captured": graphed.captures, "captures_in_timed_epoch": g_caps,
           "eager": {"step": "eager model step (the sampler's call still replayed)",
                     "batch_ms": round(1e3 * wall / nb, 3), "final_loss": round(float(loss), 4),
                     "sampled_edges_per_s_in_training": round(edges / wall, 1),
                     "stage_ms_per_batch": {k: round(v, 3) for k, v in stats.items() if k != "SpMM"}},
           "spmm_fwd_ms_per_call": round(t_stats["SpMM"], 4),
           "spmm_note": "SpMM: mean event-timed ms of one forward block SpMM, from a separate eager pass "
                        "of 10 batches with a sync per call (3 per batch); the timed epochs do not sync",
           "generate_s": round(t_gen, 2)}
    del g, X, labels, model, opt, graphed
    gc.unfreeze()
    torch.cuda.empty_cache()
    return out


def bench_dps(dev, cpu: bool, reps: int = 10) -> dict:
    """The next-row extensions: the halo repack of BCSRSampler.repack_subgraph
    (sampler.py:420-690) on c3 (a batch of 256 random windows = 4,096 seed
    rows, external budget 5x, the reference's default), the reference's
    window top-K sampler on c2, and loading a BCSR cache in the reference's
    on-disk layout (data_loader.py:282-406) into HBM, on c2 (page cache warm:
    host-memory-to-HBM rate, not the disk)."""
    import tempfile

    import numpy as np
    from graph_rws_amd import synth
    from graph_rws_amd.data import BCSRGraph, load_bcsr_bins, save_bcsr_bins
    from graph_rws_amd.sampler import BCSRSampler
    out = {}
    g = synth.config_graph("c3", device=dev)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=dev, values_dtype=torch.float16)
    del g
    s = BCSRSampler([5, 5], tile_cols=16)
    gen = torch.Generator(device="cpu").manual_seed(77)
    wids = torch.randperm(G.num_windows, generator=gen)[:256].to(dev)
    torch.manual_seed(78)
    sub = s.repack_subgraph(G, wids)  # warm-up
    torch.cuda.synchronize(dev)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        sub = s.repack_subgraph(G, wids)
        torch.cuda.synchronize(dev)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    T = int(sub.window_offset[-1])
    moved = T * 16 * 4 + T * 256 * 2 * 3 + T * 16 * 4 * 2  # cols read; values read + 2 writes; cols 2 writes
    r = {"workload": "c3 repack_subgraph: 256 random windows (4,096 rows), max_external_ratio 5.0, f16 values",
         "ms": round(1e3 * ts[len(ts) // 2], 3), "tiles": T, "internal_nodes": sub.num_internal_nodes,
         "input_nodes": int(sub.original_node_ids.numel()), "tile_gb_moved": round(moved / 1e9, 4),
         "note": "median of %d; includes the host syncs and torch.randperm of the over-budget draw" % reps}
    if cpu:
        import oracle
        win = G.window_offset.cpu().numpy()
        cols = G.original_col_indices.cpu().numpy()
        vals = G.values_condensed.float().cpu().numpy()
        ref0 = oracle.repack_subgraph(win, cols, vals, G.num_nodes, 16, wids.cpu().numpy(), 1e18)
        perm = np.random.default_rng(0).permutation(ref0["num_external"])
        t0 = time.perf_counter()
        oracle.repack_subgraph(win, cols, vals, G.num_nodes, 16, wids.cpu().numpy(), 5.0, perm=perm)
        t_cpu = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": round(1e3 * t_cpu, 2), "unit": "ms per repack", "cores": 1, "kind": "port",
                             "sample": "the same batch through oracle.repack_subgraph (numpy, one thread, "
                                       "graph arrays already in host memory)"}
    out["repack"] = r
    del G, sub
    torch.cuda.empty_cache()
    g = synth.config_graph("c2", device=dev)
    G2 = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                            device=dev)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "c2.pt")
        save_bcsr_bins(G2, path)
        load_bcsr_bins(path, device=dev, values_dtype=torch.float16)  # warm the page cache
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        H, _ = load_bcsr_bins(path, device=dev, values_dtype=torch.float16)
        torch.cuda.synchronize(dev)
        t_load = time.perf_counter() - t0
        nbytes = 8 * H.window_offset.numel() + 4 * H.original_col_indices.numel() + 4 * H.values_condensed.numel()
        same = bool(torch.equal(H.values_condensed, G2.values_condensed.half()))
    # the reference's own sampler (window top-K, BCSRSampler.sample_layers,
    # sampler.py:186-279) on c2 with its defaults: 16x8 tiles, f32 values,
    # 1,024 seeds, fanouts [15, 10, 5] (5 drawn first)
    G8 = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=8, device=dev)
    ws = BCSRSampler([15, 10, 5], tile_cols=8, verbose=False)
    seed_sets = [synth.distinct_seeds(g.num_nodes, 1024, seed=500 + b, device=dev) for b in range(23)]
    for b in range(3):
        ws.sample_layers(G8, seed_sets[b])
    torch.cuda.synchronize(dev)
    tw = []
    for b in range(3, 23):
        t0 = time.perf_counter()
        layers = ws.sample_layers(G8, seed_sets[b])
        torch.cuda.synchronize(dev)
        tw.append(time.perf_counter() - t0)
    tiles = [int(x.window_offset[-1]) for x in layers]
    # algorithmic bytes of the last batch: per layer the active windows'
    # input tiles read once (column ids and values), the sampled tiles
    # written (column ids and values), the layer's seed ids read and its
    # active windows and masks written
    woff = G8.window_offset
    s_v = G8.values_condensed.element_size()
    tile_b = 8 * 4 + 16 * 8 * s_v
    wb = 0
    n_ids = 1024
    for x in reversed(layers):  # the hop from the seeds first
        act = x.active_windows.long()
        wb += int((woff[act + 1] - woff[act]).sum()) * tile_b + int(x.window_offset[-1]) * tile_b
        wb += 4 * n_ids + 8 * act.numel()
        n_ids = 8 * int(x.window_offset[-1])
    bms = 1e3 * sum(tw) / len(tw)
    wr = {"workload": "c2 window top-K sampling (BCSRSampler, 16x8 tiles, f32 values, 1,024 seeds, fanouts "
                      "[15,10,5]): prepare windows, top-K per window, recompress, per layer",
          "batch_ms": round(bms, 4), "batches": len(tw),
          "tiles_last_batch": tiles, "active_windows_last_batch": [int(x.active_windows.numel()) for x in layers],
          "host_syncs_per_batch": 1,
          "roofline": {"bound": "hbm (per-window selection: latency bound in practice)",
                       "achieved": round(wb / (bms / 1e3) / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(wb / (bms / 1e3) / 1e9 / HBM_PEAK_GBS, 5), "bytes_per_batch": wb,
                       "bytes": "per layer: the active windows' input tiles read once (column ids and values), "
                                "the sampled tiles written, the seed ids read, the windows and masks written"}}
    # the same batches with BCSRSampler(capture=True): the call captured once
    # in a HIP graph (CapturedWindowSampler) and replayed per batch
    wsc = BCSRSampler([15, 10, 5], tile_cols=8, verbose=False, capture=True)
    for b in range(3):
        wsc.sample_layers(G8, seed_sets[b])
    torch.cuda.synchronize(dev)
    tc_ = []
    for b in range(3, 23):
        t0 = time.perf_counter()
        layers_c = wsc.sample_layers(G8, seed_sets[b])
        torch.cuda.synchronize(dev)
        tc_.append(time.perf_counter() - t0)
    cms = 1e3 * sum(tc_) / len(tc_)
    cap = next(iter(wsc._captures.values()))[1]
    wr["captured"] = {
        "batch_ms": round(cms, 4), "batches": len(tc_), "replays": cap.replays,
        "equals_eager_last_batch": all(
            torch.equal(x.window_offset, y.window_offset) and torch.equal(x.original_col_indices, y.original_col_indices)
            and torch.equal(x.values_condensed, y.values_condensed) and torch.equal(x.active_windows, y.active_windows)
            for x, y in zip(layers_c, layers)),
        "roofline_frac": round(wb / (cms / 1e3) / 1e9 / HBM_PEAK_GBS, 5),
        "note": "BCSRSampler(capture=True): grws_window_sample_layers_enqueue captured once and replayed per "
                "batch; per batch one seed copy, the replay, the counts read back (the batch's one sync) and one "
                "copy launch for the outputs"}
    del wsc, cap
    if cpu:
        import oracle
        seeds = seed_sets[-1].cpu().numpy()
        win8 = G8.window_offset.cpu().numpy()
        cols8 = G8.original_col_indices.cpu().numpy()
        vals8 = G8.values_condensed.cpu().numpy()
        t0 = time.perf_counter()
        ref = oracle.window_sample_all_layers(win8, cols8, vals8, seeds, [5, 10, 15], g.num_nodes)
        t_cpu = time.perf_counter() - t0
        same = all(np.array_equal(x.window_offset.cpu().numpy(), r[0])
                   and np.array_equal(x.original_col_indices.cpu().numpy(), r[1])
                   and np.array_equal(x.values_condensed.cpu().numpy(), r[2])
                   for x, r in zip(reversed(layers), ref))
        wr["bit_exact_vs_oracle_last_batch"] = same
        wr["cpu_baseline"] = {"value": round(1e3 * t_cpu, 2), "unit": "ms per batch", "cores": oracle.num_threads(),
                              "kind": "port", "sample": "the last batch through oracle.window_sample_all_layers "
                                                        "(C restatement; graph arrays in host memory)"}
    out["window_sampling"] = wr
    del G8
    out["bcsr_load"] = {"workload": "c2 BCSR cache (reference layout, f32 values) -> HBM, values to f16 on "
                                    "the device", "file_bytes": nbytes, "ms": round(1e3 * t_load, 2),
                        "gb_per_s": round(nbytes / t_load / 1e9, 2), "round_trip_equal": same}
    del G2, H, g
    torch.cuda.empty_cache()
    return out


def cpu_spmm_c2(g, reps: int = 5) -> dict:
    """torch.sparse CSR fp32 A X and A^T G (N=128) on the host cores, the CPU
    path beside the c2 microbenchmark: median of `reps` after one warm-up."""
    torch.set_num_threads(os.cpu_count() or 1)
    n = g.num_nodes
    A = torch.sparse_csr_tensor(g.row_ptr.cpu(), g.col_idx.cpu().long(), g.values.cpu().float(),
                                size=(n, n))
    AT = A.t().to_sparse_csr()
    X = torch.randn(n, 128, generator=torch.Generator().manual_seed(23))
    out = {}
    for name, M in (("fwd", A), ("bwd", AT)):
        M @ X
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            M @ X
            ts.append(time.perf_counter() - t0)
        ts.sort()
        out[name] = {"ms": round(1e3 * ts[len(ts) // 2], 3),
                     "gflops": round(2.0 * g.nnz * 128 / ts[len(ts) // 2] / 1e9, 2)}
    return {"value": out, "unit": "ms per product", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"whole graph, fp32, torch.sparse CSR (A and a precomputed A^T), median of {reps}"}


def bench_spmm_c2(dev, reps: int = 20, cpu: bool = False) -> dict:
    """c2 SpMM microbenchmark: forward A X and backward A^T G (G like X),
    X [169,343 x 128] in bf16 and f16, 16x16 tiles."""
    from graph_rws_amd import synth
    from graph_rws_amd.data import BCSRGraph
    g = synth.config_graph("c2", device=dev)
    res = {"workload": "c2 SpMM forward A*X and backward A^T*G", "nodes": g.num_nodes,
           "nnz": g.nnz, "N": 128}
    for dname, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes,
                               tile_cols=16, device=dev, values_dtype=dt)
        X = synth.features(g.num_nodes, 128, seed=21, device=dev).to(dt)
        Gr = synth.features(16 * G.num_windows, 128, seed=22, device=dev).to(dt)
        AT = G.transpose()
        r = {}
        for name, M, inp in (("fwd", G, X), ("bwd", AT, Gr)):
            out = torch.empty((16 * M.num_windows, 128), dtype=dt, device=dev)
            for _ in range(3):  # builds the plan, then the packed tiles
                M.spmm(inp, out=out)
            torch.cuda.synchronize(dev)
            # every per-graph cache must exist before timing: a build inside
            # the timed loop would be a host sync and a pass over the graph
            plan = M.spmm_plan(128)
            packed = M.packed_tiles()
            assert packed is not None, f"c2 {dname} {name}: packed tiles not built in the warm-up"
            s = torch.cuda.current_stream(dev)
            gc.collect()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(reps)]
            for e0, e1 in ev:
                e0.record(s)
                M.spmm(inp, out=out)
                e1.record(s)
            torch.cuda.synchronize(dev)
            per = sorted(e0.elapsed_time(e1) for e0, e1 in ev)
            ms = per[len(per) // 2]
            B = alg_bytes(M, 128, 2, 2, packed=packed, plan=plan)
            r[name] = {"ms": round(ms, 4), "ms_min": round(per[0], 4), "ms_max": round(per[-1], 4),
                       "reps": reps, "gflops": round(2.0 * g.nnz * 128 / ms / 1e6, 1),
                       "compulsory_bytes": B["compulsory"],
                       "compulsory_gbps": round(B["compulsory"] / ms / 1e6, 1),
                       "frac_hbm_peak": round(B["compulsory"] / ms / 1e6 / HBM_PEAK_GBS, 4),
                       "gather_model_bytes": B["total"],
                       "gather_model_gbps": round(B["total"] / ms / 1e6, 1),
                       "plan": {"items": plan.num_items if plan is not None else M.num_windows,
                                "split_windows": plan.num_split if plan is not None else 0}}
            tk = ("c2", 128, dname, 16, "packed tiles")
            if name == "fwd" and tk in MEASURED_TRAFFIC:
                r[name]["traffic"] = MEASURED_TRAFFIC[tk][0]
                r[name]["traffic_gbs"] = round(MEASURED_TRAFFIC[tk][0] / ms / 1e6, 1)
                r[name]["traffic_source"] = MEASURED_TRAFFIC[tk][1]
        res[dname] = r
        del G, X, Gr, AT
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = cpu_spmm_c2(g)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3", choices=["c2", "c3", "c4"])
    ap.add_argument("--dtype", default=None, choices=["f16", "bf16", "f32"])
    ap.add_argument("--tile-cols", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sampling", action="store_true")
    ap.add_argument("--no-build", action="store_true", help="skip the device BCSR build record")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run 5 device-to-device copies of BYTES (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--sampling-batches", type=int, default=20)
    ap.add_argument("--no-gcn", action="store_true")
    ap.add_argument("--no-minibatch", action="store_true")
    ap.add_argument("--no-dps", action="store_true", help="skip the repack / BCSR-cache leg")
    ap.add_argument("--minibatch-batches", type=int, default=40)
    ap.add_argument("--gcn-epochs", type=int, default=5)
    ap.add_argument("--gcn-configs", default="c1,c3,c4")
    ap.add_argument("--no-gcn-graphed", action="store_true",
                    help="skip the GCN legs' captured-graph replays")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the hot path is a single-GPU "
              "kernel; the multi-GPU sharding is a design note). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    if args.calibrate_copy > 0:
        a = torch.ones(args.calibrate_copy, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize(dev)
        ms = (time.perf_counter() - t0) * 200.0
        print(json.dumps({"copy_bytes": args.calibrate_copy, "copies": 5, "ms_per_copy": round(ms, 4),
                          "gbps_read_plus_write": round(2 * args.calibrate_copy / ms / 1e6, 1)}))
        return
    from graph_rws_amd.core import _lib
    _lib.load()
    copy_gbs = copy_peak(dev)

    cfg = args.config
    spec = {"c2": (128, 128, "f16"), "c3": (602, 608, "f16"), "c4": (100, 112, "bf16")}[cfg]
    d_raw, N, ddef = spec
    dname = args.dtype or ddef
    xdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dname]

    g, G, t_gen, t_build = build_graph(cfg, args.tile_cols, xdt, dev)
    from graph_rws_amd import synth
    from graph_rws_amd.data import aligned_rows
    # rows stored at a 128-byte multiple pitch (608 fp16 -> 640): same values,
    # every gathered row segment starts on a cache line
    X = aligned_rows(synth.features(g.num_nodes, d_raw, pad_to=N, seed=7, device=dev).to(xdt))
    plan = G.spmm_plan(N)
    Y = torch.empty((16 * G.num_windows, N), dtype=xdt, device=dev)
    stream = torch.cuda.current_stream(dev)

    # the graph's packed tiles are built on its second product (a warm-up
    # call), like the plan; the build is timed once on its own for the record
    from graph_rws_amd.core import ops as _ops
    torch.cuda.synchronize(dev)
    tp = time.perf_counter()
    _pk = _ops.pack_tiles(G.window_offset, G.original_col_indices, G.values_condensed, G.tile_cols)
    torch.cuda.synchronize(dev)
    t_pack = time.perf_counter() - tp
    del _pk
    # the graph's first product (window by window on the dense tiles) and
    # its second (which builds the grouped tiles first), each timed once
    first_ms = []
    for _ in range(2):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        G.spmm(X, out=Y)
        e1.record(stream)
        e1.synchronize()
        first_ms.append(e0.elapsed_time(e1))
    for _ in range(max(0, args.warmup - 2)):
        G.spmm(X, out=Y)
    torch.cuda.synchronize(dev)
    grouped = G.grouped_tiles(X.shape[0], N) if N >= _ops.GROUP_MIN_N else None
    if grouped is not None:
        a_format = f"grouped tiles ({grouped.group_size} windows)"
    else:
        a_format = "packed tiles" if G.packed_tiles() is not None else "dense tiles"
    t_group = None
    if grouped is not None:  # its build, timed once on its own for the record
        torch.cuda.synchronize(dev)
        tq = time.perf_counter()
        _gq = _ops.group_tiles(G.window_offset, G.original_col_indices, G.values_condensed, G.tile_cols,
                               X.shape[0], group_size=grouped.group_size)
        torch.cuda.synchronize(dev)
        t_group = time.perf_counter() - tq
        del _gq
    gc.collect()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        G.spmm(X, out=Y)
        b.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms = [a.elapsed_time(b) for a, b in ev]
    ms_avg = sum(ms) / len(ms)
    ms_step = wall * 1000.0 / args.steps

    nnz = g.nnz
    flops = 2.0 * nnz * N
    gflops = flops / (ms_step / 1e3) / 1e9
    packed = G.packed_tiles() if grouped is None else None
    B = alg_bytes(G, N, X.element_size(), Y.element_size(), packed=packed, plan=plan, grouped=grouped)
    comp_gbs = B["compulsory"] / (ms_avg / 1e3) / 1e9
    gather_gbs = B["total"] / (ms_avg / 1e3) / 1e9
    issued = (2.0 * grouped.num_slabs * grouped.group_size * 256 * N if grouped is not None
              else 2.0 * G.num_tiles * 16 * G.tile_cols * N)
    tkey = (cfg, N, dname, G.tile_cols, a_format)
    traffic = MEASURED_TRAFFIC.get(tkey, (None, None))
    # the rate at which random X row segments come from beyond the L2s (a
    # table of X's rows and pitch) and from one XCD's L2 (1,600 rows), in
    # the kernels' gather shape: 640-byte segments (a 320-column chunk of
    # 16-bit X) where the pitch holds them, else 128-byte ones
    pitch_b = X.stride(0) * X.element_size()
    g_segs = 5 if pitch_b >= 640 else 1
    ceil_miss = row_gather_ceiling(dev, X.shape[0], pitch_b, g_segs, 16_000_000)
    ceil_l2 = row_gather_ceiling(dev, 1600, pitch_b, g_segs, 16_000_000)
    traffic_gbs = traffic[0] / (ms_avg / 1e3) / 1e9 if traffic[0] else None

    out = {
        "metric": "BCSR SpMM GFLOP/s + HBM GB/s (% peak); GCN epoch ms; sampled edges/s",
        "value": round(gflops, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic (seeded generators in graph_rws_amd/synth.py; random features)",
        "config": {
            "workload": f"{cfg} BCSR SpMM forward Y=A*X",
            "graph": synth.CONFIGS[cfg]["kind"],
            "nodes": g.num_nodes, "nnz": nnz, "windows": G.num_windows, "tiles": G.num_tiles,
            "tile": f"16x{G.tile_cols}", "N": N, "x_dtype": dname, "x_row_pitch": X.stride(0),
            "values_dtype": str(G.values_condensed.dtype).replace("torch.", ""),
            "a_format": a_format,
            "plan": ({"groups": grouped.num_groups, "union_slabs": grouped.num_slabs,
                      "union_over_window_slots": round(grouped.slot_ratio, 4),
                      "longest_group_slabs": grouped.max_group_slabs} if grouped is not None else
                     {"items": plan.num_items, "split_windows": plan.num_split,
                      "slabs_per_item": plan.slabs_per_item}),
        },
        "alg_bytes": B,
        "roofline": {
            "bound": "hbm",
            # 16-bit X runs the buffer-load kernel, fp32 X the element-masked
            # one; 4-window groups multiply slab pairs (spmm_grp2d_kernel)
            "kernel": (_ops.grouped_kernel(grouped.group_size) if grouped is not None else
                       "spmm_buf_kernel" if dname in ("f16", "bf16") else "spmm_fwd_kernel"),
            # compulsory bytes (A in the format read, X and Y once) per product
            # over the product's kernel time (HIP events on the launch stream)
            "achieved": round(comp_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(comp_gbs / HBM_PEAK_GBS, 4),
            "bytes": B["compulsory"],
            "peak_measured_copy": round(copy_gbs, 1),
            "frac_of_measured_copy": round(comp_gbs / copy_gbs, 4),
            "traffic": traffic[0],
            "traffic_source": traffic[1],
            "traffic_over_compulsory": round(traffic[0] / B["compulsory"], 2) if traffic[0] else None,
            "traffic_gbs": round(traffic_gbs, 1) if traffic_gbs else None,
            # grws_probe_row_gather: the kernel's L2-miss traffic against the
            # rate the chip serves random row segments from beyond the L2s
            "row_gather_ceiling": {"l2_miss_gbs": round(ceil_miss, 1), "l2_resident_gbs": round(ceil_l2, 1),
                                   "segment_bytes": 128 * g_segs, "table_rows": int(X.shape[0]),
                                   "pitch_bytes": int(pitch_b)},
            "traffic_frac_of_row_gather_ceiling": round(traffic_gbs / ceil_miss, 3) if traffic_gbs else None,
            "gather_model": {"bytes": B["total"], "gbs": round(gather_gbs, 1),
                             "note": "modelled L2-side bytes: each gathered X row counted once per "
                                     "window that references it; the caches serve re-references, so "
                                     "this rate can exceed the DRAM peak"},
            "kernel_ms_avg": round(ms_avg, 4),
            "kernel_ms_min": round(min(ms), 4),
            "kernel_ms_max": round(max(ms), 4),
            "mfma_issued_tflops": round(issued / (ms_avg / 1e3) / 1e12, 2),
            "mfma_frac": round(issued / (ms_avg / 1e3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        },
        "setup_s": {"generate": round(t_gen, 2), "bcsr_build": round(t_build, 2),
                    "pack_tiles": round(t_pack, 4),
                    "group_tiles": round(t_group, 4) if t_group is not None else None},
        # once per graph, outside the timed steps: the graph's first product
        # runs window by window on the dense tiles; its second builds the
        # grouped (or packed) tiles and then multiplies over them
        "first_products_ms": {"first_window_by_window": round(first_ms[0], 4),
                              "second_incl_tile_build": round(first_ms[1], 4),
                              "group_tiles_build_ms": round(1e3 * t_group, 3) if t_group is not None else None},
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline(g, G, X, Y, 1e-2 if dname != "f32" else 1e-5)
        out["parity"] = cb.pop("parity")
        out["cpu_baseline"] = cb
    else:
        out["parity"] = {"pass": None, "note": "not checked (--no-cpu-baseline)"}
    if not args.no_build:
        out["bcsr_build"] = bench_build(g, dev, not args.no_cpu_baseline, cfg=cfg)
    if not args.no_sampling:
        del G, X, Y, g, plan
        torch.cuda.empty_cache()
        out["sampling"] = bench_sampling(dev, args.sampling_batches, 3, not args.no_cpu_baseline)
    if not args.no_gcn:
        out["spmm_c2"] = bench_spmm_c2(dev, cpu=not args.no_cpu_baseline)
        out["gcn"] = {c: bench_gcn(c, dev, args.gcn_epochs, 2, not args.no_cpu_baseline,
                                   graphed=not args.no_gcn_graphed)
                      for c in args.gcn_configs.split(",") if c}
    if not args.no_dps:
        out["dps"] = bench_dps(dev, not args.no_cpu_baseline)
    if not args.no_minibatch:
        out["minibatch"] = bench_minibatch(dev, args.minibatch_batches, 20)
    # parity last, so that the tail of the line shows it; a failed check
    # fails the run
    out["parity"] = out.pop("parity")
    print(json.dumps(out), flush=True)
    if out["parity"]["pass"] is False:
        print("bench.py: the timed product failed its parity check", file=sys.stderr)
        sys.exit(3)


if __name__ == "__main__":
    main()
