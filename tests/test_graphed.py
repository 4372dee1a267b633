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
