"""WindowWiseDataLoader (data/data_loader.py:39-115): the vectorised batch
search yields the same batches as walking the shuffled windows one at a
time, as the reference's loop does."""
import pytest
import torch

from graph_rws_amd.data import WindowWiseDataLoader


def _walk(loader, gen_seed):
    """The reference's loop over windows (data_loader.py:87-110), on the
    loader's own window table and the same permutation."""
    g = torch.Generator()
    g.manual_seed(gen_seed)
    perm = torch.randperm(loader.num_windows, generator=g)
    out, batch, n = [], [], 0
    for w in perm.tolist():
        s, c = loader.window_info[w]
        batch.append(loader.sorted_train_idx[s:s + c])
        n += c
        if n >= loader.batch_size:
            out.append(torch.cat(batch))
            batch, n = [], 0
    if not loader.drop_last and batch:
        out.append(torch.cat(batch))
    return out


@pytest.mark.parametrize("n,span,bs", [(5000, 40000, 64), (3000, 3000, 1), (777, 100000, 1024),
                                       (50, 800, 10000), (4096, 4096 * 16, 1024), (10, 100, 3)])
@pytest.mark.parametrize("drop_last", [False, True])
def test_batches_equal_window_walk(n, span, bs, drop_last):
    g0 = torch.Generator()
    g0.manual_seed(n + bs)
    idx = torch.randperm(span, generator=g0)[:n]
    g = torch.Generator()
    g.manual_seed(7)
    loader = WindowWiseDataLoader(idx, batch_size=bs, drop_last=drop_last, generator=g)
    got = list(loader)
    want = _walk(loader, 7)
    assert len(got) == len(want)
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    # every training node once, unless the last partial batch was dropped
    if not drop_last:
        assert torch.equal(torch.sort(torch.cat(got)).values, torch.sort(idx).values)


def test_empty_train_set():
    loader = WindowWiseDataLoader(torch.empty(0, dtype=torch.int64), batch_size=8)
    assert list(loader) == []
