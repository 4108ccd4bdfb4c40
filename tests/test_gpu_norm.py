"""RMSNorm kernels (ssm_scan.norm, csrc/ssm_norm.hip) against models/common.py:14-16.

The reference expression in float64 (torch autograd for the gradients) on the same float32
values: forward rtol 1e-5 / atol 1e-6, gradients rtol 1e-4 / atol 1e-5 on every element; the
float64 kernels through the same autograd function to 1e-12.  Also: rows with a stride (a
column slice), bitwise-repeatable backward, and the dtypes that keep the torch expression.
"""

import pytest
import torch

from ssm_scan import norm

pytestmark = pytest.mark.gpu


def ref64(x, w, eps):
    x64 = x.detach().double().requires_grad_()
    w64 = w.detach().double().requires_grad_()
    y = x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + eps) * w64
    return x64, w64, y


def close(got, ref, rtol, atol):
    torch.testing.assert_close(got.double(), ref.double(), rtol=rtol, atol=atol)


@pytest.mark.parametrize("shape", [(2, 37, 256), (1, 1, 64), (5, 3, 100), (3, 7, 1000), (4, 9, 1),
                                   (2, 33, 65), (16, 512, 256), (2, 5, 1024)])
def test_forward_and_gradients_match_reference(dev, shape):
    g = torch.Generator().manual_seed(shape[-1] + shape[1])
    x = (torch.randn(shape, generator=g) * 3.0).to(dev).requires_grad_()
    w = (1.0 + 0.5 * torch.randn(shape[-1], generator=g)).to(dev).requires_grad_()
    dy = torch.randn(shape, generator=g).to(dev)
    y = norm.rms_norm(x, w, 1e-5)
    assert y.shape == x.shape and y.dtype == torch.float32
    y.backward(dy)
    x64, w64, y64 = ref64(x, w, 1e-5)
    y64.backward(dy.double())
    close(y.detach(), y64.detach(), 1e-5, 1e-6)
    close(x.grad, x64.grad, 1e-4, 1e-5)
    close(w.grad, w64.grad, 1e-4, 1e-5)


@pytest.mark.parametrize("shape", [(3, 11, 256), (2, 4, 513)])
def test_float64_kernels(dev, shape):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(shape, generator=g, dtype=torch.float64).to(dev).requires_grad_()
    w = torch.randn(shape[-1], generator=g, dtype=torch.float64).to(dev).requires_grad_()
    dy = torch.randn(shape, generator=g, dtype=torch.float64).to(dev)
    y = norm.RMSNormFn.apply(x, w, 1e-6)
    y.backward(dy)
    x64, w64, y64 = ref64(x, w, 1e-6)
    y64.backward(dy)
    for a, b in ((y.detach(), y64.detach()), (x.grad, x64.grad), (w.grad, w64.grad)):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_strided_rows_and_repeatable_backward(dev):
    """x a column slice of a wider tensor (row stride 2C, read in place); two backward passes
    give bitwise equal gradients."""
    g = torch.Generator().manual_seed(3)
    big = torch.randn(4, 100, 512, generator=g).to(dev)
    w = torch.randn(256, generator=g).to(dev).requires_grad_()
    dy = torch.randn(4, 100, 256, generator=g).to(dev)
    grads = []
    for _ in range(2):
        x = big[..., :256].detach().requires_grad_()
        assert x.stride() == (51200, 512, 1)
        y = norm.rms_norm(x, w, 1e-5)
        y.backward(dy)
        grads.append((y.detach(), x.grad.clone(), w.grad.clone()))
        w.grad = None
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    x64, w64, y64 = ref64(big[..., :256], w, 1e-5)
    y64.backward(dy.double())
    close(grads[0][0], y64.detach(), 1e-5, 1e-6)
    close(grads[0][1], x64.grad, 1e-4, 1e-5)
    close(grads[0][2], w64.grad, 1e-4, 1e-5)


def test_other_dtypes_keep_the_reference_expression(dev):
    """bf16 rows with a float32 weight promote to float32 (as the reference's product does);
    float64 rows are normalized in float32 (the reference's x.float())."""
    g = torch.Generator().manual_seed(5)
    w = torch.randn(256, generator=g).to(dev)
    xb = torch.randn(2, 8, 256, generator=g).to(dev, torch.bfloat16)
    yb = norm.rms_norm(xb, w)
    assert yb.dtype == torch.float32
    assert torch.equal(yb, norm.rms_norm_reference(xb, w, 1e-5))
    xd = torch.randn(2, 8, 256, generator=g, dtype=torch.float64).to(dev)
    yd = norm.rms_norm(xd, w.double())
    assert torch.equal(yd, norm.rms_norm_reference(xd, w.double(), 1e-5))


def test_rejects_wide_rows_through_the_abi(dev):
    x = torch.zeros(2, 1025, device=dev)
    w = torch.ones(1025, device=dev)
    with pytest.raises(ValueError, match="dim"):
        norm.RMSNormFn.apply(x, w, 1e-5)
