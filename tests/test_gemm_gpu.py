"""Weight-gradient kernel C = A^T B (csrc/gemm_tn.hip) against float64 on
the same f16/bf16 inputs.  Bound: |C - C64| <= 1e-4 * (|A|^T |B|) elementwise
(the products are exact in fp32; only the fp32 accumulation rounds)."""
import pytest
import torch

from graph_rws_amd.core.ops import gemm_tn, gemm_tn_supported

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,M,N", [(0, 8, 16), (1, 8, 8), (31, 128, 136), (1000, 136, 256),
                                   (5000, 256, 8), (100003, 128, 256), (300000, 608, 256)])
def test_gemm_tn_matches_float64(cuda_device, dt, K, M, N):
    print(f"case gemm_tn {dt} K={K} M={M} N={N}", flush=True)
    g = torch.Generator(device=cuda_device).manual_seed(K + M + N)
    A = torch.randn(K, M, generator=g, device=cuda_device).to(dt)
    B = torch.randn(K, N, generator=g, device=cuda_device).to(dt)
    C = gemm_tn(A, B)
    assert C.shape == (M, N) and C.dtype == torch.float32
    ref = A.double().t() @ B.double()
    bound = A.double().abs().t() @ B.double().abs()
    assert bool(((C.double() - ref).abs() <= 1e-4 * bound + 1e-30).all())
    assert torch.equal(C, gemm_tn(A, B))  # deterministic


def test_gemm_tn_strided_and_low_precision_output(cuda_device):
    A0 = torch.randn(20000, 200, device=cuda_device).half()
    A = A0[:, 8:136]  # row stride 200, offset 16 bytes
    B = torch.randn(20000, 64, device=cuda_device).half()
    assert gemm_tn_supported(A, B)
    ref = A.double().t() @ B.double()
    for od in (torch.float16, torch.float32):
        C = gemm_tn(A, B, out_dtype=od)
        assert C.dtype == od
        tol = 2e-3 if od == torch.float16 else 1e-4
        bound = A.double().abs().t() @ B.double().abs()
        assert bool(((C.double() - ref).abs() <= tol * bound).all())
    # a misaligned start and ragged widths go through a widened copy; a
    # ragged width over a wider buffer reuses its row padding (NaN there
    # must not reach the result)
    Am = A0[:, 1:129]
    assert gemm_tn_supported(Am, B)
    Cm = gemm_tn(Am, B)
    bm = Am.double().abs().t() @ B.double().abs()
    assert bool(((Cm.double() - Am.double().t() @ B.double()).abs() <= 1e-4 * bm).all())
    Bp = torch.full((20000, 48), float("nan"), device=cuda_device).half()
    Bp[:, :41] = torch.randn(20000, 41, device=cuda_device).half()
    Br = Bp[:, :41]
    Cr = gemm_tn(A, Br)
    assert Cr.shape == (128, 41) and bool(torch.isfinite(Cr).all())
    br = A.double().abs().t() @ Br.double().abs()
    assert bool(((Cr.double() - A.double().t() @ Br.double()).abs() <= 1e-4 * br).all())
    A41 = torch.randn(20000, 41, device=cuda_device).bfloat16()
    B41 = torch.randn(20000, 41, device=cuda_device).bfloat16()
    C41 = gemm_tn(A41, B41)
    b41 = A41.double().abs().t() @ B41.double().abs()
    assert bool(((C41.double() - A41.double().t() @ B41.double()).abs() <= 1e-4 * b41).all())


def test_graphconv_autocast_backward_uses_split_k(cuda_device):
    """A BCSRGraphConv under f16 autocast: the weight gradients (both paths)
    come out of the split-K kernel and match float64 autograd over the same
    f16-quantised operands within 2e-2 of the largest magnitude."""
    from graph_rws_amd import synth
    from graph_rws_amd.data import BCSRGraph
    from graph_rws_amd.layers import BCSRGraphConv
    torch.manual_seed(0)
    g = synth.chung_lu(6000, 60000, 2.2, seed=5)
    G = BCSRGraph.from_csr(g.row_ptr, g.col_idx, g.values, g.num_nodes, g.num_nodes, tile_cols=16,
                           device=cuda_device, values_dtype=torch.float16)
    conv = BCSRGraphConv(64, 32).to(cuda_device)
    X = torch.randn(g.num_nodes, 64, device=cuda_device).half()
    R = torch.randn(g.num_nodes, 32, device=cuda_device)
    with torch.autocast("cuda", dtype=torch.float16):
        out = conv(G, X, features_target=X)
        loss = (out.float() * R).sum()
    loss.backward()
    import scipy.sparse as sps
    vals16 = torch.from_numpy(g.values.numpy()).half().double().numpy()
    A = torch.from_numpy(sps.csr_matrix((vals16, g.col_idx.numpy(), g.row_ptr.numpy()),
                                        shape=(g.num_nodes, g.num_nodes)).toarray())
    Xd = X.double().cpu()
    Wn = conv.weight_neigh.detach().half().double().cpu().requires_grad_(True)
    Ws = conv.weight_self.detach().half().double().cpu().requires_grad_(True)
    ref = A @ (Xd @ Wn) + Xd @ Ws
    (ref * R.double().cpu()).sum().backward()
    for got, want in ((conv.weight_neigh.grad, Wn.grad), (conv.weight_self.grad, Ws.grad)):
        assert got.dtype == torch.float32
        d = float((got.double().cpu() - want).abs().max())
        assert d <= 2e-2 * float(want.abs().max()), d
