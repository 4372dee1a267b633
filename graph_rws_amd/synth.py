"""Seeded synthetic graphs of the shapes BASELINE.json names.

The reference loads real datasets through DGL/OGB (data/data_loader.py), which
need the network; the benchmark configurations are synthetic instead.  Every
graph here is symmetric, deduplicated, has a self-loop on every node and
carries GCN weights D^-1/2 (A+I) D^-1/2 with D the in-degree including the
self-loop -- the closed form of data/data_loader.py:974-986.  Generators run
with torch on any device (use the GPU for the large configurations) and are
deterministic for a given (seed, device type).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class CSRGraph:
    num_nodes: int
    row_ptr: torch.Tensor   # int64 [n+1]
    col_idx: torch.Tensor   # int32 [nnz], ascending within a row
    values: torch.Tensor    # float32 [nnz]

    @property
    def nnz(self) -> int:
        return int(self.col_idx.numel())

    def to(self, device) -> "CSRGraph":
        return CSRGraph(self.num_nodes, self.row_ptr.to(device), self.col_idx.to(device),
                        self.values.to(device))


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _finish(n: int, u: torch.Tensor, v: torch.Tensor, device) -> CSRGraph:
    """Symmetrise, deduplicate, add self-loops, sym-normalise, build CSR."""
    keep = u != v
    u, v = u[keep], v[keep]
    key = torch.cat([u * n + v, v * n + u])
    key = torch.unique(key)
    loops = torch.arange(n, device=device, dtype=torch.int64) * (n + 1)
    key = torch.unique(torch.cat([key, loops]))  # sorted by (row, col)
    rows = key // n
    cols = key % n
    deg = torch.bincount(rows, minlength=n).to(torch.float32)  # symmetric: in == out
    norm = deg.clamp(min=1).pow(-0.5)
    vals = norm[rows] * norm[cols]
    row_ptr = torch.zeros(n + 1, dtype=torch.int64, device=device)
    row_ptr[1:] = torch.cumsum(torch.bincount(rows, minlength=n), 0)
    return CSRGraph(n, row_ptr, cols.to(torch.int32), vals.to(torch.float32))


def _draw_unique_pairs(n: int, target: int, sampler, device) -> tuple:
    """Draws undirected pairs with `sampler(m) -> (u, v)` until `target`
    distinct unordered non-loop pairs exist, then keeps exactly `target`."""
    have = torch.empty(0, dtype=torch.int64, device=device)
    m = int(target * 1.15) + 16
    for _ in range(12):
        u, v = sampler(m)
        a = torch.minimum(u, v)
        b = torch.maximum(u, v)
        k = a * n + b
        k = k[a != b]
        have = torch.unique(torch.cat([have, k]))
        if have.numel() >= target:
            break
        m = int((target - have.numel()) * 1.5) + 16
    if have.numel() > target:
        # deterministic subset: keep the pairs with the smallest hashed key
        h = (have * 0x9E3779B97F4A7C15) & 0x7FFFFFFFFFFFFFFF
        idx = torch.argsort(h)[:target]
        have = have[idx]
    return have // n, have % n


def chung_lu(n: int, num_directed_edges: int, gamma: float, seed: int = 0,
             max_degree: Optional[float] = None, device="cpu") -> CSRGraph:
    """Chung-Lu power-law graph: endpoint i drawn with probability proportional
    to w_i = (i+1)^(-1/(gamma-1)) (capped at max_degree in expected degree).
    `num_directed_edges` counts both directions of every non-loop edge; a
    self-loop is then added to every node."""
    device = torch.device(device)
    g = _gen(seed, device)
    i = torch.arange(n, device=device, dtype=torch.float64)
    w = (i + 1.0).pow(-1.0 / (gamma - 1.0))
    w = w / w.sum() * num_directed_edges
    if max_degree is not None:
        w = w.clamp(max=float(max_degree))
    cdf = torch.cumsum(w / w.sum(), 0)
    cdf[-1] = 1.0
    # scramble ids so heavy nodes are spread over the id range
    perm = torch.randperm(n, generator=g, device=device)

    def sampler(m):
        r = torch.rand(2, m, generator=g, device=device, dtype=torch.float64)
        s = torch.searchsorted(cdf, r).clamp(max=n - 1)
        return perm[s[0]], perm[s[1]]

    u, v = _draw_unique_pairs(n, num_directed_edges // 2, sampler, device)
    return _finish(n, u, v, device)


def sbm(n: int, communities: int, intra_fraction: float, num_directed_edges: int,
        seed: int = 0, device="cpu") -> CSRGraph:
    """Stochastic block model with contiguous community ids (community c holds
    nodes [c*n/k, (c+1)*n/k)); a drawn edge is intra-community with
    probability `intra_fraction`, else uniform over all nodes."""
    device = torch.device(device)
    g = _gen(seed, device)
    bounds = torch.tensor([(c * n) // communities for c in range(communities + 1)],
                          device=device, dtype=torch.int64)

    def sampler(m):
        r = torch.rand(4, m, generator=g, device=device, dtype=torch.float64)
        intra = r[0] < intra_fraction
        c = (r[1] * communities).long().clamp(max=communities - 1)
        lo = bounds[c]
        size = (bounds[c + 1] - lo).to(torch.float64)
        ui = lo + (r[2] * size).long()
        vi = lo + (r[3] * size).long()
        r2 = torch.rand(2, m, generator=g, device=device, dtype=torch.float64)
        uu = (r2[0] * n).long().clamp(max=n - 1)
        vv = (r2[1] * n).long().clamp(max=n - 1)
        return torch.where(intra, ui, uu), torch.where(intra, vi, vv)

    u, v = _draw_unique_pairs(n, num_directed_edges // 2, sampler, device)
    return _finish(n, u, v, device)


def random_graph(n: int, avg_degree: float, seed: int = 0, device="cpu") -> CSRGraph:
    """Uniform random symmetric graph (small parity cases)."""
    device = torch.device(device)
    g = _gen(seed, device)

    def sampler(m):
        r = torch.randint(0, n, (2, m), generator=g, device=device)
        return r[0], r[1]

    target = max(1, int(n * avg_degree / 2))
    target = min(target, n * (n - 1) // 2)
    u, v = _draw_unique_pairs(n, target, sampler, device)
    return _finish(n, u, v, device)


def features(n: int, d: int, pad_to: Optional[int] = None, dtype=torch.float32, seed: int = 0,
             device="cpu", kind: str = "normal", p: float = 0.013) -> torch.Tensor:
    """Node features [n, pad_to or d]: N(0,1) or Bernoulli(p) ('binary');
    padding columns are zero."""
    device = torch.device(device)
    if dtype != torch.float32 and n * (pad_to or d) > (1 << 28):
        return _features_chunked(n, d, pad_to, dtype, seed, device, kind, p)
    g = _gen(seed, device)
    if kind == "binary":
        x = (torch.rand(n, d, generator=g, device=device) < p).to(torch.float32)
    else:
        x = torch.randn(n, d, generator=g, device=device, dtype=torch.float32)
    if pad_to is not None and pad_to > d:
        x = torch.nn.functional.pad(x, (0, pad_to - d))
    return x.to(dtype)


def _features_chunked(n, d, pad_to, dtype, seed, device, kind, p, rows: int = 1 << 20):
    """features() for matrices too large to stage in float32: generated in
    row chunks straight into the target dtype."""
    g = _gen(seed, device)
    out = torch.zeros(n, pad_to or d, dtype=dtype, device=device)
    for s in range(0, n, rows):
        e = min(n, s + rows)
        if kind == "binary":
            x = (torch.rand(e - s, d, generator=g, device=device) < p).to(dtype)
        else:
            x = torch.randn(e - s, d, generator=g, device=device, dtype=torch.float32).to(dtype)
        out[s:e, :d] = x
    return out


# ---------------------------------------------------------------------------
# BASELINE.json configurations
# ---------------------------------------------------------------------------
CONFIGS = {
    "c1": dict(kind="chung_lu", n=2708, edges=10556, gamma=2.5, seed=1),
    "c2": dict(kind="chung_lu", n=169343, edges=2_330_000 - 169343, gamma=2.1, seed=2),
    "c3": dict(kind="sbm", n=232965, communities=50, intra=0.8, edges=114_600_000 - 232965, seed=3),
    "c4": dict(kind="chung_lu", n=2449029, edges=123_700_000 - 2449029, gamma=2.0, seed=4,
               max_degree=17000.0),
}


def config_graph(name: str, device="cpu", scale: float = 1.0) -> CSRGraph:
    """Graph of BASELINE config `name` ('c1'..'c4'); `scale` < 1 shrinks node
    and edge counts proportionally (parity tests)."""
    c = CONFIGS[name]
    n = max(32, int(c["n"] * scale))
    e = max(64, int(c["edges"] * scale))
    if c["kind"] == "sbm":
        return sbm(n, c["communities"], c["intra"], e, seed=c["seed"], device=device)
    return chung_lu(n, e, c["gamma"], seed=c["seed"], max_degree=c.get("max_degree"),
                    device=device)


def powerlaw_csr(n: int, num_edges: int, gamma: float = 2.1, max_degree: int = 100_000,
                 seed: int = 5, device="cpu", chunk: int = 1 << 27) -> CSRGraph:
    """Directed power-law graph as CSR, generated directly (no symmetrise or
    dedup pass, so it scales to billions of edges in HBM).

    Out-degrees: the Chung-Lu expectation w_r = c (r+1)^(-1/(gamma-1)) for
    degree rank r, capped at `max_degree` and rescaled to `num_edges`,
    rounded stochastically.  Neighbours: i.i.d. endpoint ranks drawn from
    the continuous inverse CDF of the same power law.  Node ids are a
    seeded permutation of ranks, so hubs are spread over the id range.
    Neighbour lists are in draw order and may repeat a node.  values are
    empty (the sampler derives GCN weights from the degrees)."""
    device = torch.device(device)
    g = _gen(seed, device)
    a = 1.0 / (gamma - 1.0)
    r = torch.arange(n, device=device, dtype=torch.float64)
    w = (r + 1.0).pow(-a)
    w = w * (num_edges / w.sum())
    for _ in range(6):
        w = w.clamp(max=float(max_degree))
        w = w * (num_edges / w.sum())
    w = w.clamp(max=float(max_degree))
    fl = torch.floor(w)
    deg = (fl + (torch.rand(n, generator=g, device=device, dtype=torch.float64) < (w - fl))).to(torch.int64)
    del w, fl, r
    perm = torch.randperm(n, generator=g, device=device)  # rank -> node id
    deg_by_id = torch.empty_like(deg)
    deg_by_id[perm] = deg
    del deg
    indptr = torch.zeros(n + 1, dtype=torch.int64, device=device)
    torch.cumsum(deg_by_id, 0, out=indptr[1:])
    del deg_by_id
    nnz = int(indptr[-1].item())
    indices = torch.empty(nnz, dtype=torch.int32, device=device)
    b = 1.0 - a
    top = float((n + 1.0) ** b - 1.0)
    for s in range(0, nnz, chunk):
        e = min(nnz, s + chunk)
        u = torch.rand(e - s, generator=g, device=device, dtype=torch.float64)
        x = (1.0 + u * top).pow(1.0 / b).sub_(1.0).floor_().clamp_(0, n - 1).to(torch.int64)
        indices[s:e] = perm[x].to(torch.int32)
        del u, x
    return CSRGraph(n, indptr, indices, torch.empty(0, dtype=torch.float32, device=device))


def distinct_seeds(n: int, count: int, seed: int = 42, device="cpu") -> torch.Tensor:
    """`count` distinct node ids drawn uniformly from [0, n) (int64)."""
    device = torch.device(device)
    g = _gen(seed, device)
    have = torch.empty(0, dtype=torch.int64, device=device)
    while have.numel() < count:
        draw = torch.randint(0, n, (2 * count,), generator=g, device=device)
        cat = torch.cat([have, draw])
        u, idx = torch.unique(cat, return_inverse=True)
        # keep first occurrences in draw order
        first = torch.full((u.numel(),), cat.numel(), dtype=torch.int64, device=device)
        first.scatter_reduce_(0, idx, torch.arange(cat.numel(), device=device), reduce="amin")
        have = cat[torch.sort(first).values]
    return have[:count].contiguous()


# c5: mini-batch sampling at web scale
C5 = dict(n=111_000_000, edges=1_600_000_000, gamma=2.1, max_degree=100_000, seed=5,
          batch=1024, fanouts=[15, 10, 5], philox_seed=42, feat=128, classes=172)


def c5_graph(device="cpu", scale: float = 1.0) -> CSRGraph:
    """The c5 CSR (111M nodes, ~1.6B edges, int64 indptr, int32 indices);
    `scale` < 1 shrinks nodes and edges proportionally."""
    n = max(64, int(C5["n"] * scale))
    e = max(256, int(C5["edges"] * scale))
    return powerlaw_csr(n, e, gamma=C5["gamma"], max_degree=C5["max_degree"], seed=C5["seed"],
                        device=device)
