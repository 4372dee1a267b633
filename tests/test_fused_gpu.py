"""Fused hidden-layer tail and cross-entropy (csrc/fused.hip) against torch's
own ops on the same inputs.

Tolerances: fp32 statistics either way, so outputs agree to 1e-5 relative
in fp32 and to one rounding step of the output dtype otherwise; gradients
within 1e-4 of the largest magnitude (fp32 chains of different summation
order)."""
import pytest
import torch
import torch.nn.functional as F

from graph_rws_amd.layers.fused import act_norm_dropout, cross_entropy_rows

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 8e-3}


def _close(a, b, tol):
    a, b = a.double(), b.double()
    scale = max(float(b.abs().max()), 1e-30)
    d = float((a - b).abs().max())
    assert d <= tol * scale, f"max |diff| {d:.3e} > {tol:g} * {scale:.3e}"


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [256, 64, 1024, 12, 300])
def test_act_norm_matches_torch(cuda_device, dt, dim):
    print(f"case act_norm {dt} dim={dim}", flush=True)
    torch.manual_seed(dim)
    rows = 3001
    z = (torch.randn(rows, dim, device=cuda_device) * 2 + 0.3).to(dt).requires_grad_(True)
    norm = torch.nn.LayerNorm(dim).to(cuda_device)
    with torch.no_grad():
        norm.weight.uniform_(0.5, 1.5)
        norm.bias.uniform_(-0.5, 0.5)
    out = act_norm_dropout(z, norm, 0.0, relu=True)
    # without autocast the output keeps z's dtype, as F.layer_norm's does
    assert out.dtype == dt and out.shape == (rows, dim)
    zr = z.detach().float().requires_grad_(True)
    wr = norm.weight.detach().clone().requires_grad_(True)
    br = norm.bias.detach().clone().requires_grad_(True)
    ref = F.layer_norm(F.relu(zr), (dim,), wr, br, norm.eps)
    _close(out.float(), ref.to(dt).float(), TOL[dt])
    # the upstream gradient reaches the fused op in the output dtype: give
    # the fp32 reference the same (quantised) values
    R = torch.randn(rows, dim, device=cuda_device).to(dt).float()
    (out * R).sum().backward()
    (ref * R).sum().backward()
    _close(z.grad.float(), zr.grad.to(dt).float(), max(1e-4, TOL[dt]))
    _close(norm.weight.grad, wr.grad, 1e-4)
    _close(norm.bias.grad, br.grad, 1e-4)


def test_act_norm_autocast_output_dtype(cuda_device):
    """Under autocast the output is the autocast dtype, equal to the fp32
    result rounded once (what the next layer's cast of torch's fp32 output
    would give)."""
    z = torch.randn(500, 256, device=cuda_device).bfloat16()
    norm = torch.nn.LayerNorm(256).to(cuda_device)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = act_norm_dropout(z, norm, 0.0, relu=True)
    ref = F.layer_norm(F.relu(z.float()), (256,), norm.weight, norm.bias, norm.eps)
    assert out.dtype == torch.bfloat16
    _close(out.float(), ref.bfloat16().float(), 8e-3)


def test_dropout_mask_statistics_and_backward(cuda_device):
    torch.manual_seed(3)
    rows, dim, p = 4000, 256, 0.5
    z = torch.randn(rows, dim, device=cuda_device, requires_grad=True)
    norm = torch.nn.LayerNorm(dim).to(cuda_device)
    y = act_norm_dropout(z.detach(), norm, 0.0, relu=True)
    torch.manual_seed(11)
    out = act_norm_dropout(z, norm, p, relu=True)
    kept = out != 0
    frac = float(kept.float().mean())
    assert abs(frac - (1 - p)) < 0.01
    _close(out[kept], y[kept] * 2.0, 1e-5)
    # same torch seed -> same mask; another seed -> another mask
    torch.manual_seed(11)
    assert torch.equal(act_norm_dropout(z.detach(), norm, p, relu=True), out.detach())
    torch.manual_seed(12)
    assert not torch.equal(act_norm_dropout(z.detach(), norm, p, relu=True), out.detach())
    R = torch.randn(rows, dim, device=cuda_device)
    (out * R).sum().backward()
    zr = z.detach().clone().requires_grad_(True)
    ref = F.layer_norm(F.relu(zr), (dim,), norm.weight.detach(), norm.bias.detach(), norm.eps) * kept * 2.0
    (ref * R).sum().backward()
    _close(z.grad, zr.grad, 1e-4)


@pytest.mark.parametrize("dim,p", [(300, 0.3), (64, 0.9), (1000, 0.05)])
def test_dropout_mask_is_the_oracle_philox(cuda_device, dim, p):
    """Element (r, c) is kept iff word c%4 of Philox4x32-10 at counter
    (r_lo, r_hi, c/4, 0), key = the 64-bit seed, is >= p * 2^32.  The
    oracle's Philox is pinned against ATen's vectors, so this pins the
    counter layout and threshold of the kernel's mask."""
    import numpy as np
    import oracle
    print(f"case mask dim={dim} p={p}", flush=True)
    rows = 23
    torch.manual_seed(dim)
    z = torch.randn(rows, dim, device=cuda_device)
    norm = torch.nn.LayerNorm(dim).to(cuda_device)
    with torch.no_grad():
        norm.bias.fill_(1.0)  # no output is exactly zero before dropout
    y = act_norm_dropout(z, norm, 0.0, relu=True)
    torch.manual_seed(77)
    seed = int(torch.randint(0, 2 ** 62, (1,)).item())  # the draw the wrapper makes
    torch.manual_seed(77)
    out = act_norm_dropout(z, norm, p, relu=True)
    thr = min(int(float(np.float32(p)) * 2.0 ** 32), 0xFFFFFFFF)  # p reaches the kernel as fp32
    key = [seed & 0xFFFFFFFF, seed >> 32]
    want = np.zeros((rows, dim), bool)
    for r in range(rows):
        for b in range((dim + 3) // 4):
            w = oracle.philox4x32_10([r, 0, b, 0], key)
            for j in range(min(4, dim - 4 * b)):
                want[r, 4 * b + j] = int(w[j]) >= thr
    got = (out != 0).cpu().numpy()
    assert (got == want).all(), f"{int((got != want).sum())} mask elements differ"
    _close(out[out != 0], y[out != 0] / (1.0 - p), 1e-5)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("classes", [7, 47, 172])
def test_cross_entropy_matches_torch(cuda_device, dt, classes):
    print(f"case ce {dt} C={classes}", flush=True)
    torch.manual_seed(classes)
    R = 20000
    logits = (torch.randn(R, classes, device=cuda_device) * 3).to(dt).requires_grad_(True)
    rows = torch.nonzero(torch.rand(R, device=cuda_device) < 0.6).view(-1)
    labels = torch.randint(0, classes, (rows.numel(),), device=cuda_device)
    labels[::17] = -100  # ignore_index
    loss, counts = cross_entropy_rows(logits, rows, labels)
    lr = logits.detach().clone().requires_grad_(True)
    sel = lr[rows].float()
    ref = F.cross_entropy(sel, labels)
    correct = (sel.argmax(1) == labels).sum()
    _close(loss, ref, 1e-5)
    assert int(counts[0]) == int(correct) and int(counts[1]) == int((labels != -100).sum())
    loss.backward()
    ref.backward()
    assert logits.grad.dtype == dt
    _close(logits.grad.float(), lr.grad.float(), 1e-4 if dt == torch.float32 else 1e-2)


def test_cross_entropy_first_rows_and_bad_labels(cuda_device):
    logits = torch.randn(100, 10, device=cuda_device)
    labels = torch.randint(0, 10, (60,), device=cuda_device)
    loss, counts = cross_entropy_rows(logits, None, labels)
    _close(loss, F.cross_entropy(logits[:60], labels), 1e-5)
    labels[3] = 10  # out of range: torch asserts; here the loss is NaN and the flag is set
    loss, counts = cross_entropy_rows(logits, None, labels)
    assert torch.isnan(loss) and int(counts[2]) == 1
