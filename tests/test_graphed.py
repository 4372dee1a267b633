"""GraphedFullStep host-side checks (no device work)."""
import pytest
import torch

from graph_rws_amd.helper import GraphedFullStep


def test_graphed_step_refuses_host_stepping_optimizer():
    """The captured step needs an optimizer that steps on the device
    (capturable=True); the check comes before any device work."""
    p = torch.nn.Parameter(torch.zeros(3))
    opt = torch.optim.Adam([p], lr=0.1)
    with pytest.raises(ValueError, match="capturable"):
        GraphedFullStep(None, None, None, None, None, opt, "cpu")


def test_block_step_refuses_host_stepping_optimizer():
    from graph_rws_amd.helper import GraphedBlockStep
    p = torch.nn.Parameter(torch.zeros(3))
    with pytest.raises(ValueError, match="capturable"):
        GraphedBlockStep(torch.nn.Linear(2, 2), torch.optim.Adam([p], lr=0.1), "cpu")


def test_block_step_refuses_batch_norm():
    """Padding rows would enter a batch norm's statistics."""
    from graph_rws_amd.helper import GraphedBlockStep
    m = torch.nn.Sequential(torch.nn.Linear(2, 2), torch.nn.BatchNorm1d(2))
    with pytest.raises(ValueError, match="batch normalisation"):
        GraphedBlockStep(m, torch.optim.Adam(m.parameters(), lr=0.1, capturable=True), "cpu")


def test_bucket_rows():
    """Buckets are multiples of 16 rows, at least the size asked for, at
    most max(255 rows, 1/8) above it, and monotone."""
    from graph_rws_amd.helper import bucket_rows
    prev = 0
    for x in list(range(1, 5000)) + [65_537, 250_664, 1_000_003, 2**24 + 1]:
        b = bucket_rows(x)
        assert b >= x and b % 16 == 0 and b >= prev
        assert b - x <= max(255, x / 8), (x, b)
        prev = b
    assert bucket_rows(1) == 256 and bucket_rows(256) == 256 and bucket_rows(257) == 512
