"""grws_probe_row_gather (measurement only): the kernel bench.py times for
the random row-gather ceiling reads exactly the rows it is given.

Each wave folds (XOR) every 32-bit word it loaded into one word; the wave
w of nw takes the 8-row groups 2w, 2w+1, 2w+2nw, 2w+2nw+1, ...  The host
restates that assignment with numpy over the same table and indices: the
words agree only if every listed row's first segments * 128 bytes were
read, and an index outside the table reads zeros.  The argument checks
are exercised without a launch.
"""
import numpy as np
import pytest
import torch

from graph_rws_amd.core import _lib as L

pytestmark = pytest.mark.gpu


def _expected(table_u32, rows, pitch_words, seg_words, idx, blocks):
    nw = 4 * blocks
    groups = idx.size // 8
    out = np.zeros(nw, np.uint32)
    for w in range(nw):
        acc = np.uint32(0)
        q = 2 * w
        while q < groups:
            for gq in (q, q + 1):
                if gq >= groups:
                    continue
                for r in idx[8 * gq:8 * gq + 8]:
                    if 0 <= r < rows:
                        acc ^= np.bitwise_xor.reduce(table_u32[r * pitch_words:r * pitch_words + seg_words])
            q += 2 * nw
        out[w] = acc
    return out


@pytest.mark.parametrize("segments,blocks", [(5, 2), (1, 3), (10, 1)])
def test_probe_reads_the_listed_rows(cuda_device, segments, blocks):
    print(f"case probe_row_gather segments={segments} blocks={blocks}", flush=True)
    rng = np.random.default_rng(segments + 7 * blocks)
    rows, pitch = 97, 1280
    table = rng.integers(0, 2 ** 32, size=rows * pitch // 4, dtype=np.uint64).astype(np.uint32)
    n_idx = 8 * 41
    idx = rng.integers(0, rows, size=n_idx).astype(np.int32)
    idx[5] = rows          # past the table: zeros
    idx[17] = -3           # negative: zeros
    t = torch.from_numpy(table.view(np.int32)).to(cuda_device)
    ix = torch.from_numpy(idx).to(cuda_device)
    out = torch.full((4 * blocks,), -1, dtype=torch.int32, device=cuda_device)
    L.call("grws_probe_row_gather", L.ptr(t), rows, pitch, segments, L.ptr(ix), n_idx, L.ptr(out), blocks,
           L.stream_of(cuda_device))
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    want = _expected(table, rows, pitch // 4, segments * 32, idx, blocks)
    np.testing.assert_array_equal(got, want)


def test_probe_rejects_bad_arguments(cuda_device):
    t = torch.zeros(1024, dtype=torch.int32, device=cuda_device)
    ix = torch.zeros(8, dtype=torch.int32, device=cuda_device)
    out = torch.zeros(4, dtype=torch.int32, device=cuda_device)
    s = L.stream_of(cuda_device)
    lib = L.load()
    bad = [
        (L.ptr(t), 4, 1024, 3, L.ptr(ix), 8, L.ptr(out), 1),     # segments not 1, 5 or 10
        (L.ptr(t), 4, 512, 5, L.ptr(ix), 8, L.ptr(out), 1),      # 640 bytes past a 512-byte pitch
        (L.ptr(t), 4, 1024, 1, L.ptr(ix), 7, L.ptr(out), 1),     # n_idx not a multiple of 8
        (L.ptr(t), 4, 1024, 1, L.ptr(ix), 8, L.ptr(out), 0),     # no blocks
        (L.ptr(t), 4, 1000, 1, L.ptr(ix), 8, L.ptr(out), 1),     # pitch not a multiple of 16
        (None, 4, 1024, 1, L.ptr(ix), 8, L.ptr(out), 1),         # null table
    ]
    for args in bad:
        assert lib.grws_probe_row_gather(*args, s) != 0, args
