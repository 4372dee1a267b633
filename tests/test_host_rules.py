"""Host-side layout rules of the ops layer (no device work): line-pitched
buffers, the paired-product layout and the rule that decides when the
convolution adds its self term inside the SpMM."""
import torch

from graph_rws_amd.core import ops


def test_line_pitched_empty_rows_start_on_lines():
    for cols, dt in ((41, torch.float16), (47, torch.bfloat16), (7, torch.float32), (64, torch.float16),
                     (172, torch.float16)):
        t = ops.line_pitched_empty(10, cols, dt, "cpu", zero=True)
        esz = t.element_size()
        assert t.shape == (10, cols) and t.stride(1) == 1
        assert (t.stride(0) * esz) % 128 == 0 and t.stride(0) >= cols
        assert t.stride(0) - cols < 128 // esz                 # the smallest such pitch
        assert not bool(t.any())


def test_pair_pitch_puts_each_product_on_whole_lines():
    assert ops.pair_pitch(256, 2) == 512
    assert ops.pair_pitch(47, 2) == 128
    assert ops.pair_pitch(41, 2) == 128
    assert ops.pair_pitch(16, 4) == 64
    assert ops.pair_pitch(172, 2) == 384


def test_mm_pair_line_pitched_matches_two_products():
    torch.manual_seed(0)
    a = torch.randn(50, 24)
    w1, w2 = torch.randn(24, 47), torch.randn(24, 47)
    t1, t2 = ops.mm_pair_line_pitched(a, w1, w2)
    assert t1.shape == (50, 47) and t2.shape == (50, 47)
    assert t1.stride(0) == ops.pair_pitch(47, 4)
    torch.testing.assert_close(t1, a @ w1)
    torch.testing.assert_close(t2, a @ w2)


def test_fuse_self_rule():
    # narrow paired rows always pay; wide ones only within the Infinity Cache
    assert ops.fuse_self_pays(2_449_029, 47, 2)
    assert ops.fuse_self_pays(232_965, 256, 2)
    assert not ops.fuse_self_pays(2_449_029, 256, 2)
    assert ops.fuse_self_pays(2708, 16, 4)
