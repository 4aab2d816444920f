"""CPU tests of the drop-in modules (no GPU): swap semantics, stock-path equality,
state-dict compatibility and fallbacks.  Restates the reference's
tests/test_conv3d.py:24-44 and BASELINE config 1 (the CPU plumbing case)."""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from rdna4_conv3d import Conv3dWmma, ConvTranspose3dWmma, conv3d_wmma, swap_conv3d
from rdna4_conv3d.conv3d_wmma import Conv3dWmmaFn


def test_swap_copies_weights():
    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.c = nn.Conv3d(4, 8, 3, padding=1)

    m = M()
    w = m.c.weight.data.clone()
    n = swap_conv3d(m)
    assert n == 1
    assert isinstance(m.c, Conv3dWmma)
    assert torch.equal(m.c.weight.data, w)


def test_swap_recursive_and_preserving():
    m = nn.Sequential(
        nn.Conv3d(2, 4, 3, padding=1, padding_mode="replicate", bias=False),
        nn.Sequential(nn.Conv3d(4, 4, 1), nn.ReLU(), nn.ConvTranspose3d(4, 2, 2, stride=2)),
    ).to(torch.float64)
    m.eval()
    ref = {k: v.clone() for k, v in m.state_dict().items()}
    assert swap_conv3d(m) == 2
    assert type(m[0]) is Conv3dWmma and type(m[1][0]) is Conv3dWmma
    assert type(m[1][2]) is nn.ConvTranspose3d  # not swapped by default
    assert m[0].padding_mode == "replicate" and m[0].bias is None
    assert m[0].weight.dtype == torch.float64 and not m[0].training
    for k, v in m.state_dict().items():
        assert torch.equal(v, ref[k])
    # opt-in transpose swap (not counted)
    assert swap_conv3d(m, transpose=True) == 0
    assert type(m[1][2]) is ConvTranspose3dWmma


def test_subclass_does_not_swap_again():
    class MyConv(nn.Conv3d):
        pass

    m = nn.Sequential(MyConv(2, 2, 3))
    assert swap_conv3d(m) == 0  # exact-type match, like the reference (conv3d_wmma.py:1416)


def test_plumbing_config_cpu_bitwise_equal():
    """Conv3d(24,24,3,p=1,bias) on [1,24,32,32,32] fp32, CPU fwd+bwd."""
    g = torch.Generator().manual_seed(0)
    torch.manual_seed(1)
    stock = nn.Conv3d(24, 24, 3, padding=1)
    drop = Conv3dWmma(24, 24, 3, padding=1)
    drop.load_state_dict(stock.state_dict())
    x = torch.randn(1, 24, 32, 32, 32, generator=g)
    go = torch.randn(1, 24, 32, 32, 32, generator=torch.Generator().manual_seed(2))
    x1, x2 = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    y1, y2 = stock(x1), drop(x2)
    assert torch.equal(y1, y2)
    y1.backward(go)
    y2.backward(go)
    assert torch.equal(x1.grad, x2.grad)
    assert torch.equal(stock.weight.grad, drop.weight.grad)
    assert torch.equal(stock.bias.grad, drop.bias.grad)


def test_convtranspose_cpu_equals_stock():
    torch.manual_seed(0)
    stock = nn.ConvTranspose3d(6, 3, 2, stride=2)
    drop = ConvTranspose3dWmma(6, 3, 2, stride=2)
    drop.load_state_dict(stock.state_dict())
    x = torch.randn(2, 6, 3, 4, 5)
    assert torch.equal(stock(x), drop(x))
    assert torch.equal(stock(x, output_size=[6, 8, 10]), drop(x, output_size=[6, 8, 10]))


def test_fallbacks_on_cpu():
    torch.manual_seed(0)
    x = torch.randn(1, 4, 8, 8, 8)
    conv = Conv3dWmma(4, 5, 3, stride=2, padding=1)
    torch.testing.assert_close(conv(x), F.conv3d(x, conv.weight, conv.bias, 2, 1), atol=1e-5, rtol=1e-5)
    same = Conv3dWmma(4, 4, 3, padding="same")
    torch.testing.assert_close(same(x), F.conv3d(x, same.weight, same.bias, 1, "same"))
    wg = torch.randn(4, 2, 3, 3, 3)
    assert torch.equal(conv3d_wmma(x, wg, None, 1, 1, 1, 2), F.conv3d(x, wg, None, 1, 1, 1, 2))
    # the Function itself routes CPU tensors to F.conv3d
    w = torch.randn(5, 4, 3, 3, 3)
    assert torch.equal(Conv3dWmmaFn.apply(x, w, None, (1, 1, 1), (1, 1, 1), (1, 1, 1)),
                       F.conv3d(x, w, None, 1, 1, 1))


def test_empty_batch_cpu():
    conv = Conv3dWmma(3, 4, 3, padding=1)
    y = conv(torch.randn(0, 3, 4, 4, 4))
    assert y.shape == (0, 4, 4, 4, 4)


@pytest.mark.parametrize("k,pad", [(3, 0), (3, 2), (1, 1)])
def test_geometries_cpu_match_stock(k, pad):
    torch.manual_seed(k + pad)
    stock = nn.Conv3d(3, 5, k, padding=pad)
    drop = Conv3dWmma(3, 5, k, padding=pad)
    drop.load_state_dict(stock.state_dict())
    x = torch.randn(2, 3, 5, 6, 7)
    assert torch.equal(stock(x), drop(x))


def test_bnrelu_on_cpu_is_batchnorm_then_relu():
    """BatchNormReLU3d (native BatchNorm + ReLU on gfx950) keeps nn.BatchNorm3d's
    parameters, buffers and semantics; on the CPU it is exactly BatchNorm3d + ReLU."""
    import torch.nn.functional as F
    from rdna4_conv3d.fused import BatchNormReLU3d
    torch.manual_seed(0)
    mod = BatchNormReLU3d(6, momentum=None)
    ref = nn.BatchNorm3d(6, momentum=None)
    ref.load_state_dict(mod.state_dict())
    assert set(mod.state_dict()) == set(ref.state_dict())
    x = torch.randn(2, 6, 3, 4, 5)
    for _ in range(2):
        torch.testing.assert_close(mod(x), F.relu(ref(x)), atol=0, rtol=0)
    torch.testing.assert_close(mod.running_var, ref.running_var, atol=0, rtol=0)
    assert int(mod.num_batches_tracked) == 2
    mod.eval()
    ref.eval()
    torch.testing.assert_close(mod(x), F.relu(ref(x)), atol=0, rtol=0)


def test_maxpool_on_cpu_is_maxpool3d():
    """MaxPool3dWmma is nn.MaxPool3d (same module type, state and output) off the
    GPU and for every configuration other than kernel 2 / stride 2."""
    from rdna4_conv3d.fused import MaxPool3dWmma
    x = torch.randn(2, 3, 6, 8, 16, requires_grad=True)
    for args in [(2,), (2, 2), (3, 1, 1), ((2, 2, 1),)]:
        mod, ref = MaxPool3dWmma(*args), nn.MaxPool3d(*args)
        assert isinstance(mod, nn.MaxPool3d)
        assert not mod._native_ok(x)
        torch.testing.assert_close(mod(x), ref(x), atol=0, rtol=0)


def test_forward_cat_on_cpu_is_conv_of_cat():
    """Conv3dWmma.forward_cat(a, b) equals the module applied to torch.cat((a, b), 1)
    wherever the native kernels do not run (here: CPU tensors)."""
    from rdna4_conv3d import Conv3dWmma
    torch.manual_seed(0)
    conv = Conv3dWmma(12, 5, 3, padding=1)
    a, b = torch.randn(2, 8, 4, 5, 6), torch.randn(2, 4, 4, 5, 6)
    torch.testing.assert_close(conv.forward_cat(a, b), conv(torch.cat((a, b), 1)), atol=0, rtol=0)


def test_swap_strided_conv3d_and_cpu_fallback():
    """swap_strided_conv3d replaces exactly the strided nn.Conv3d children
    (weights, padding_mode kept) and leaves stride-1 ones to swap_conv3d; on
    the CPU StridedConv3dWmma is nn.Conv3d, bit for bit."""
    import torch.nn as nn
    from rdna4_conv3d.strided import StridedConv3dWmma, swap_strided_conv3d
    torch.manual_seed(0)
    m = nn.Sequential(nn.Conv3d(2, 4, 3, padding=1), nn.Sequential(nn.Conv3d(4, 8, 3, stride=2, padding=1)),
                      nn.Conv3d(8, 8, 1, stride=(1, 2, 2), padding_mode="zeros"))
    x = torch.randn(1, 2, 6, 8, 8)
    before = m(x)
    assert swap_strided_conv3d(m) == 2
    assert type(m[0]) is nn.Conv3d
    assert type(m[1][0]) is StridedConv3dWmma and type(m[2]) is StridedConv3dWmma
    assert m[1][0].stride == (2, 2, 2) and m[2].stride == (1, 2, 2)
    assert torch.equal(m(x), before)
    assert swap_strided_conv3d(m) == 0
