"""grws_gather_rows (ops.gather_rows): the mini-batch producer's feature
gather.  Bit-exact against torch's index_select for every unit width the
kernel picks (16, 8, 4, 2 and 1 bytes: row length, pitches and base
addresses decide), int64 and int32 indices, repeated indices, a strided
source and an empty index; an index outside the source gives a zero row and
raises the error flag, and nothing else writes the flag.  Also the batch
copy of the graphed mini-batch step (ops.copy_and_fill)."""
import pytest
import torch

from graph_rws_amd.core import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,dtype,idx_dtype,n", [
    (1000, 128, torch.float16, torch.int64, 5000),   # 256-byte rows: 16-byte units
    (500, 50, torch.float32, torch.int32, 777),      # 200 bytes: 8-byte units
    (300, 3, torch.float32, torch.int64, 64),        # 12 bytes: 4-byte units
    (301, 3, torch.float16, torch.int32, 129),       # 6 bytes: 2-byte units
    (257, 3, torch.uint8, torch.int64, 1000),        # 3 bytes: 1-byte units
    (1_000_000, 128, torch.float16, torch.int64, 250_000),
])
def test_gather_rows_matches_index_select(cuda_device, rows, cols, dtype, idx_dtype, n):
    print(f"case gather {rows}x{cols} {dtype} idx {idx_dtype} n={n}", flush=True)
    g = torch.Generator(device=cuda_device)
    g.manual_seed(rows + n)
    if dtype == torch.uint8:
        src = torch.randint(0, 256, (rows, cols), generator=g, device=cuda_device, dtype=torch.uint8)
    else:
        src = torch.randn(rows, cols, generator=g, device=cuda_device).to(dtype)
    idx = torch.randint(0, rows, (n,), generator=g, device=cuda_device).to(idx_dtype)
    err = torch.zeros(1, dtype=torch.int32, device=cuda_device)
    out = ops.gather_rows(src, idx, err=err)
    ref = src.index_select(0, idx.long())
    assert torch.equal(out.view(torch.uint8) if dtype != torch.uint8 else out,
                       ref.view(torch.uint8) if dtype != torch.uint8 else ref)
    assert int(err.item()) == 0


def test_gather_rows_strided_source_and_output(cuda_device):
    """Rows of a column slice (pitch 256 B, 200 B read) into a wider output."""
    print("case gather strided", flush=True)
    big = torch.randn(4000, 128, device=cuda_device).half()
    src = big[:, 8:108]
    idx = torch.randint(0, 4000, (3000,), device=cuda_device)
    outbig = torch.full((3000, 120), 7.0, device=cuda_device).half()
    out = outbig[:, 4:104]
    ops.gather_rows(src, idx, out=out)
    assert torch.equal(out, src.index_select(0, idx))
    assert (outbig[:, :4] == 7).all() and (outbig[:, 104:] == 7).all()  # nothing outside the rows written


def test_gather_rows_out_of_range_and_empty(cuda_device):
    print("case gather out of range / empty", flush=True)
    src = torch.randn(100, 64, device=cuda_device).half()
    idx = torch.tensor([0, -1, 99, 100, 5, 1 << 40], device=cuda_device)
    err = torch.zeros(1, dtype=torch.int32, device=cuda_device)
    out = ops.gather_rows(src, idx, err=err)
    assert int(err.item()) == 1
    for i, j in enumerate(idx.tolist()):
        if 0 <= j < 100:
            assert torch.equal(out[i], src[j])
        else:
            assert (out[i] == 0).all()
    # in-range call: the flag is left as the caller set it
    err.fill_(5)
    ops.gather_rows(src, idx[[0, 2, 4]], err=err)
    assert int(err.item()) == 5
    empty = ops.gather_rows(src, torch.empty(0, dtype=torch.int64, device=cuda_device))
    assert empty.shape == (0, 64)


def test_copy_and_fill_ranges(cuda_device):
    """ops.copy_and_fill (grws_copy_ranges, grws_fill_ranges_i64), the
    graphed mini-batch step's batch copy: 40 copies (more than one launch's
    32 ranges) of byte sizes with and without a 16-byte tail, empty ranges,
    and int64 fills, bit-exact against the sources and the fill values;
    nothing outside the ranges is written."""
    print("case copy_and_fill 40 ranges", flush=True)
    g = torch.Generator(device=cuda_device)
    g.manual_seed(40)
    copies, expect = [], []
    for i in range(40):
        nbytes = [0, 1, 15, 16, 17, 4096, 12345][i % 7] + 16 * i
        src = torch.randint(0, 256, (nbytes,), generator=g, device=cuda_device, dtype=torch.uint8)
        buf = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=cuda_device)
        copies.append((buf[:nbytes], src))
        expect.append((buf, src, nbytes))
    fills, fbufs = [], []
    for i, n in enumerate([0, 1, 7, 1000, 33]):
        buf = torch.full((n + 8,), -7, dtype=torch.int64, device=cuda_device)
        fills.append((buf[:n], i * 1000 - 3))
        fbufs.append((buf, n, i * 1000 - 3))
    assert ops.copy_and_fill(copies, fills)
    torch.cuda.synchronize()
    for buf, src, n in expect:
        assert torch.equal(buf[:n], src)
        assert bool((buf[n:] == 0xA5).all()), "a copy wrote past its range"
    for buf, n, v in fbufs:
        assert bool((buf[:n] == v).all())
        assert bool((buf[n:] == -7).all()), "a fill wrote past its range"


def test_copy_and_fill_refuses_unsuitable_operands(cuda_device):
    """Host tensors, a misaligned start, unequal sizes, a non-int64 fill and
    operands on two devices are refused (False, nothing done); empty lists
    are a no-op."""
    x = torch.zeros(64, dtype=torch.uint8, device=cuda_device)
    y = torch.ones(64, dtype=torch.uint8, device=cuda_device)
    assert ops.copy_and_fill([], [])
    assert not ops.copy_and_fill([(x, torch.ones(64, dtype=torch.uint8))], [])
    assert not ops.copy_and_fill([(x[1:33], y[:32])], [])
    assert not ops.copy_and_fill([(x[:32], y[:16])], [])
    assert not ops.copy_and_fill([], [(torch.zeros(4, dtype=torch.int32, device=cuda_device), 1)])
    assert not ops.copy_and_fill([(x, y)], [(torch.zeros(4, dtype=torch.int64), 1)])
    torch.cuda.synchronize()
    assert bool((x == 0).all())
