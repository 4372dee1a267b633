"""Full-graph training epoch and evaluation (helper/engine.py:22-83, 646-667).

Same steps as the reference: forward over the whole graph, cross-entropy (or
BCE for multi-label) on the training rows, backward, clip_grad_norm_(1.0),
optimizer step, loss.item().  The SpMMs inside run on the gfx950 kernels.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def compute_loss_and_metrics(logits, labels):
    """(loss, correct_count tensor, num_samples) (engine.py:22-41)."""
    if labels.dim() > 1:
        loss = F.binary_cross_entropy_with_logits(logits, labels)
        correct = ((logits > 0).float() == labels).sum()
        return loss, correct, labels.numel()
    loss = F.cross_entropy(logits, labels)
    correct = (logits.argmax(dim=1) == labels).sum()
    return loss, correct, labels.size(0)


def loss_and_metrics_rows(logits, rows, labels, check_rows: bool = True):
    """compute_loss_and_metrics(logits[rows].float(), labels) with the
    single-label cross-entropy on the fused kernel (no gather, no cast) when
    rows are strictly ascending (train_idx from a mask is; checked once per
    tensor, or not at all with check_rows=False, which then takes the torch
    path for any rows given); the reference's torch ops otherwise.  rows
    None = the first labels.numel() rows."""
    from ..layers.fused import cross_entropy_rows, cross_entropy_supported, rows_distinct
    if (FUSED_LOSS and labels.dim() == 1 and cross_entropy_supported(logits, labels)
            and (rows is None or (check_rows and rows.dtype == torch.int64 and rows.is_cuda
                                  and rows.dim() == 1 and rows_distinct(rows)))):
        loss, counts = cross_entropy_rows(logits, rows, labels)
        return loss, counts[0], labels.numel()
    sel = logits[rows] if rows is not None else logits[: labels.shape[0]]
    return compute_loss_and_metrics(sel.float(), labels)


# Cross-entropy on the fused kernel where it applies; False restores the
# reference's torch ops.
FUSED_LOSS = True


def train_epoch_full(model, graphs_for_model, features: torch.Tensor, labels: torch.Tensor,
                     train_idx: torch.Tensor, optimizer: torch.optim.Optimizer, device,
                     timer=None, sync: bool = True):
    """One full-graph training step (engine.py:44-83).  Returns (loss, acc);
    with sync=False the loss and accuracy stay on the device (no host sync)."""
    model.train()
    if timer is not None:
        timer.reset()
    if features.device != device:
        features = features.to(device)
    optimizer.zero_grad()
    logits = model(graphs_for_model, features)
    loss, correct, n = loss_and_metrics_rows(logits, train_idx, labels[train_idx])
    acc = correct / n if n > 0 else 0.0
    loss.backward()
    torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=1.0)
    optimizer.step()
    if not sync:
        return loss.detach(), acc
    return loss.item(), acc


@torch.no_grad()
def evaluate(model, bcsr_full, features: torch.Tensor, labels: torch.Tensor,
             eval_idx: torch.Tensor, device):
    """Accuracy of a full-graph inference on eval_idx (engine.py:646-667)."""
    model.eval()
    logits = model.inference(bcsr_full, features)
    _, correct, n = compute_loss_and_metrics(logits[eval_idx].float(), labels[eval_idx])
    return (correct / n).item() if n > 0 else 0.0


# ---------------------------------------------------------------------------
# mini-batch training (helper/engine.py:86-256)
# ---------------------------------------------------------------------------
def _adopt(tensors, stream) -> None:
    """Tensors made on the sampling stream are used on `stream`: tell the
    caching allocator, so their memory is not reused before that work ends.
    The allocator tracks storages, so views of one storage (a sampled
    batch's arrays are views of a few compact buffers) are recorded once."""
    seen = set()
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            key = t.untyped_storage().data_ptr()
            if key not in seen:
                seen.add(key)
                t.record_stream(stream)


def _graph_tensors(g):
    out = [g.window_offset, g.original_col_indices, g.values_condensed]
    cached = getattr(g, "_cache", {}).get("T")
    if cached is not None:  # a transpose built on the sampling stream
        AT = cached[1]
        out += [AT.window_offset, AT.original_col_indices, AT.values_condensed]
    for name in ("active_windows", "active_masks", "src_nodes", "dst_nodes"):
        t = getattr(g, name, None)
        if t is not None:
            out.append(t)
    return out


_SAMPLING_STREAMS = {}


def _sampling_stream(device) -> torch.cuda.Stream:
    """The producer's stream, one per device for the life of the process
    (default priority).  The caching allocator keeps freed blocks per
    stream, so a new stream per epoch would allocate fresh device memory
    every epoch; reusing one keeps the producer's pool warm."""
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    s = _SAMPLING_STREAMS.get(key)
    if s is None:
        s = torch.cuda.Stream(torch.device("cuda", key))
        _SAMPLING_STREAMS[key] = s
    return s


def _transpose_needs(model, features: torch.Tensor):
    """Per layer, whether its backward uses the block's A^T (the first
    layer's input is the feature matrix; later inputs carry gradients)."""
    out = []
    for l, layer in enumerate(getattr(model, "layers", [])):
        x_grad = l > 0 or features.requires_grad
        f = getattr(layer, "needs_transpose", None)
        out.append(True if f is None else bool(f(x_grad)))
    return out


def _sample_batch(sampler, graph, seeds, features, device, needs_t=None):
    """(subgraphs, batch_features or None, rows of the seeds in the logits).

    NeighborSampler: graph is a CSR (row_ptr, col_idx); blocks come back
    destination-first, the input features are gathered for
    blocks[0].src_nodes and the seeds are the first rows of the output.
    BCSRSampler: graph is the full BCSRGraph; the model reads the full
    feature matrix by global column id and the seed rows are located through
    the last layer's active windows (engine.py:170-181)."""
    from ..sampler import NeighborSampler
    if isinstance(sampler, NeighborSampler):
        want = None
        if torch.is_grad_enabled():
            # the backward's A^T, for the layers whose backward runs it: built
            # by the sampler's own call (no further sync), on the sampling
            # stream, off the training critical path
            want = [needs_t is None or l >= len(needs_t) or bool(needs_t[l]) for l in range(len(sampler.fanouts))]
        blocks = sampler.sample_layers(graph.row_ptr, graph.col_idx, seeds, transposes=want)
        if want is not None:
            for l, b in enumerate(blocks):
                if want[l]:
                    b.transpose()  # found in the block's cache (built here when the sampler did not)
        inp = blocks[0].src_nodes
        if features.is_cuda and features.dim() == 2 and (features.shape[1] <= 1 or features.stride(1) == 1):
            from ..core import ops
            feats = ops.gather_rows(features, inp)
        elif features.is_cuda:
            feats = features.index_select(0, inp)
        else:  # host-resident features: gather on the host, copy over
            feats = features.index_select(0, inp.cpu()).pin_memory().to(device, non_blocking=True)
        return blocks, feats, None
    subgraphs = sampler.sample_layers(graph, seeds)
    feats = None
    if not features.is_cuda:  # UVA-style mode of engine.py:128-141
        g0 = subgraphs[0]
        inp = g0.original_col_indices
        feats = features[inp.cpu().clamp(min=0).long()].to(device, non_blocking=True)
        g0.original_col_indices = torch.arange(inp.numel(), device=device, dtype=torch.int32)
        g0.is_local_input = True
    return subgraphs, feats, None


def _sorted_on(seeds: torch.Tensor, device) -> torch.Tensor:
    """The batch's seeds in ascending order, on `device`.  A host batch is
    sorted before its copy (1,024 ids: microseconds on the host, against a
    sort launch and its kernel on the device)."""
    if seeds.is_cuda:
        return torch.sort(seeds).values
    return torch.sort(seeds).values.to(device, non_blocking=True)


def _seed_rows(sampler, subgraphs, seeds, logits, tile_rows):
    from ..sampler import NeighborSampler
    if isinstance(sampler, NeighborSampler):
        return None  # the seeds are the first rows of the output
    act = subgraphs[-1].active_windows.long()
    sw = torch.div(seeds, tile_rows, rounding_mode="floor")
    sa, perm = torch.sort(act)
    wi = perm[torch.searchsorted(sa, sw)]
    rows = wi * tile_rows + seeds % tile_rows
    return torch.clamp(rows, max=logits.shape[0] - 1)


def train_epoch_node_sampling(model, graphs_for_model, features: torch.Tensor,
                              labels: torch.Tensor, train_idx: torch.Tensor,
                              optimizer: torch.optim.Optimizer, device, sampler,
                              batch_size: int = 1024, tile_rows: int = 16, timer=None,
                              pipeline: bool = True, max_batches: int = 0, graphed=None):
    """One epoch of mini-batch training (engine.py:86-256).  Returns
    (average loss, accuracy).

    pipeline=True: a producer thread samples (and gathers features) on its
    own stream, one batch ahead of the training loop on the current stream
    (engine.py:112-203).  Streams keep the default priority.
    `sampler` is a BCSRSampler (window top-K, the reference's) with the full
    BCSRGraph, or a NeighborSampler (Philox fanout) with the CSR graph
    (an object with row_ptr / col_idx).  max_batches > 0 stops early.
    graphed: a GraphedBlockStep over the same model and optimizer, which
    replays each batch's step from a HIP graph captured per bucket of batch
    shapes (NeighborSampler blocks only); the timer then records the whole
    step under "Step"."""
    import queue
    import threading
    from ..data import WindowWiseDataLoader
    from .timer import EpochTimer

    model.train()
    timer = timer or EpochTimer()
    timer.reset()
    total_loss = torch.zeros(1, device=device)
    total_correct = torch.zeros(1, device=device)
    total_samples = 0
    num_batches = 0
    graph = graphs_for_model[0] if isinstance(graphs_for_model, list) else graphs_for_model
    loader = WindowWiseDataLoader(train_idx.cpu(), batch_size=batch_size, tile_rows=tile_rows)
    main = torch.cuda.current_stream(device)
    needs_t = _transpose_needs(model, features)

    if graphed is not None:
        from ..sampler import NeighborSampler
        if not isinstance(sampler, NeighborSampler):
            raise ValueError("graphed steps take the node-wise sampler's blocks (NeighborSampler)")

    def step(seeds, subgraphs, feats):
        nonlocal total_samples, num_batches
        if graphed is not None:
            loss, correct = graphed(subgraphs, feats, labels[seeds])
            timer.record("Step")
            with torch.no_grad():
                total_loss.add_(loss)
                total_correct.add_(correct)
            total_samples += seeds.numel()
            num_batches += 1
            timer.end_batch()
            return
        optimizer.zero_grad()
        logits = model(subgraphs, feats if feats is not None else features)
        timer.record("Fwd")
        rows = _seed_rows(sampler, subgraphs, seeds, logits, tile_rows)
        loss, correct, n = loss_and_metrics_rows(logits, rows, labels[seeds], check_rows=False)
        loss.backward()
        timer.record("Bwd")
        torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=1.0)
        optimizer.step()
        timer.record("Step")
        with torch.no_grad():
            total_loss.add_(loss.detach())
            total_correct.add_(correct)
        total_samples += n
        num_batches += 1
        timer.end_batch()

    if pipeline:
        side = _sampling_stream(device)
        q: "queue.Queue" = queue.Queue(maxsize=1)
        failure = []

        def producer():
            try:
                with torch.cuda.stream(side):
                    for b, seeds in enumerate(loader):
                        if max_batches and b >= max_batches:
                            break
                        seeds = _sorted_on(seeds, device)
                        subgraphs, feats, _ = _sample_batch(sampler, graph, seeds, features, device, needs_t)
                        ev = torch.cuda.Event()
                        ev.record(side)
                        q.put((seeds, subgraphs, feats, ev))
            except BaseException as e:  # surfaced in the training thread
                failure.append(e)
            finally:
                q.put(None)

        worker = threading.Thread(target=producer, daemon=True)
        worker.start()
        while True:
            timer.start_batch()
            item = q.get()
            timer.record("Data")
            if item is None:
                break
            seeds, subgraphs, feats, ev = item
            main.wait_event(ev)
            _adopt([t for g in subgraphs for t in _graph_tensors(g)] + [seeds, feats], main)
            timer.record("Sample")
            step(seeds, subgraphs, feats)
        worker.join()
        if failure:
            raise failure[0]
    else:
        for b, seeds in enumerate(loader):
            if max_batches and b >= max_batches:
                break
            timer.start_batch()
            seeds = _sorted_on(seeds, device)
            timer.record("Data")
            subgraphs, feats, _ = _sample_batch(sampler, graph, seeds, features, device, needs_t)
            timer.record("Sample")
            step(seeds, subgraphs, feats)

    if num_batches == 0:
        return 0.0, 0.0
    return total_loss.item() / num_batches, total_correct.item() / max(total_samples, 1)
