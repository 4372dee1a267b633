"""The Python entry points hand raw pointers to the library, so a host
tensor, or one on another device, must be refused before any call: every
public op that takes tensors raises a RuntimeError for host inputs (CPU
tier: nothing here touches a GPU)."""
import pytest
import torch

from graph_rws_amd import builder
from graph_rws_amd.core import _lib as L
from graph_rws_amd.core import ops


def test_require_device_rules():
    L.require_device("t", torch.device("cuda", 0))  # nothing to check
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        L.require_device("t", torch.device("cpu"), torch.zeros(2))
    with pytest.raises(RuntimeError, match="every tensor must be on cuda:0"):
        L.require_device("t", torch.device("cuda", 0), None, torch.zeros(2))


@pytest.mark.parametrize("call", [
    lambda: ops.window_seeds(torch.arange(8, dtype=torch.int32), 100),
    lambda: ops.relabel(torch.arange(4), torch.arange(8), 100),
    lambda: ops.build_spmm_plan(torch.zeros(3, dtype=torch.int64), 0, 16, 16),
    lambda: builder.coo_to_csr_device(4, 4, torch.arange(3), torch.arange(3)),
    lambda: builder.csr_to_bcsr_device(2, 2, torch.tensor([0, 1, 2]), torch.tensor([0, 1], dtype=torch.int32),
                                       torch.ones(2)),
    lambda: builder.coo_to_bcsr_device(2, 2, torch.arange(2), torch.arange(2), torch.ones(2)),
    lambda: builder.bcsr_to_coo(torch.zeros(2, dtype=torch.int64), torch.full((16,), -1, dtype=torch.int32),
                                torch.zeros(256), 16, 4),
    lambda: ops.sample_all_layers(torch.zeros(2, dtype=torch.int64), torch.full((8,), -1, dtype=torch.int32),
                                  torch.zeros(128), torch.arange(4), [5], 16),
    lambda: ops.sample_hop(torch.zeros(3, dtype=torch.int64), torch.zeros(0, dtype=torch.int32),
                           torch.arange(2), 5),
], ids=["window_seeds", "relabel", "build_spmm_plan", "coo_to_csr_device", "csr_to_bcsr_device",
        "coo_to_bcsr_device", "bcsr_to_coo", "sample_all_layers", "sample_hop"])
def test_host_tensors_are_refused(call):
    with pytest.raises(RuntimeError):
        call()


def test_gemm_tn_refuses_host_operands():
    a = torch.zeros(16, 8, dtype=torch.float16)
    with pytest.raises(ValueError):
        ops.gemm_tn(a, a)
