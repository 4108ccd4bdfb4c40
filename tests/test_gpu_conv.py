"""Causal depthwise conv1d + SiLU (ssm_conv_fwd / ssm_conv_bwd) against the float64 oracle
and torch.nn.functional.conv1d (float64, CPU; gradients by autograd).

Mirrors the conv of models/mamba.py:101-107 incl. its state handling (:104-106): a sequence
processed in pieces with the carried state, and one token at a time, equals the whole
sequence (the reference's decode == forward check, tests/test_models.py:36-48).
Tolerances: float32 rtol 1e-5 / atol 1e-6 (a W-tap dot product); bf16 inputs rtol 2e-2 / atol
1e-5; float64 1e-12.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ssm_scan.conv import causal_conv1d
from oracle import scan_ref as R
from ssm_inputs import np64

pytestmark = pytest.mark.gpu
TOL = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (2e-2, 1e-5), torch.float64: (1e-12, 1e-12)}


def ref_conv(x_bld, w, bias, activation=True):
    """torch float64 CPU reference (autograd-capable): (B, L, D) -> (B, L, D)."""
    W = w.shape[1]
    xc = F.pad(x_bld.transpose(1, 2), (W - 1, 0))
    y = F.conv1d(xc, w.unsqueeze(1), bias, groups=w.shape[0])
    if activation:
        y = F.silu(y)
    return y.transpose(1, 2)


def inputs(B, L, D, W, seed, split_view=True):
    g = torch.Generator().manual_seed(seed)
    if split_view:   # the in_proj(u).chunk(2) view: (B, L, D) with row stride 2D
        xz = torch.randn(B, L, 2 * D, generator=g, dtype=torch.float64)
        x = xz[..., :D]
    else:
        x = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, W, generator=g, dtype=torch.float64) * 0.5
    bias = torch.randn(D, generator=g, dtype=torch.float64) * 0.1
    return x, w, bias


@pytest.mark.parametrize("W", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("L", [1, 3, 64, 65, 200])
def test_forward_matches_oracle(dev, W, L):
    x, w, bias = inputs(2, L, 37, W, seed=W * 100 + L)
    y = causal_conv1d(x.to(dev, torch.float32), w.to(dev, torch.float32), bias.to(dev, torch.float32))
    ry, _ = R.conv1d_causal(np64(x).transpose(0, 2, 1), np64(w), np64(bias))
    rt, at = TOL[torch.float32]
    np.testing.assert_allclose(np64(y), ry.transpose(0, 2, 1), rtol=rt, atol=at)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("activation,with_bias", [(True, True), (False, True), (True, False)])
def test_forward_backward_matches_torch(dev, dtype, activation, with_bias):
    x, w, bias = inputs(3, 150, 64, 4, seed=7)
    if not with_bias:
        bias = None
    xd = x.to(dtype)                      # the reference consumes the same rounded inputs
    leaves = [xd.to(dev).requires_grad_(), w.to(dev, torch.float32 if dtype != torch.float64 else dtype).requires_grad_()]
    bl = None if bias is None else bias.to(dev, leaves[1].dtype).requires_grad_()
    y = causal_conv1d(leaves[0], leaves[1], bl, activation=activation)
    g = torch.Generator().manual_seed(8)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    y.backward(dy.to(dev, dtype))
    rx = xd.double().requires_grad_()
    rw = leaves[1].detach().cpu().double().requires_grad_()
    rb = None if bias is None else bl.detach().cpu().double().requires_grad_()
    ry = ref_conv(rx, rw, rb, activation)
    ry.backward(dy.to(dtype).double())
    rt, at = TOL[dtype]
    scale = max(1.0, float(ry.detach().abs().max()))
    np.testing.assert_allclose(np64(y), ry.detach().numpy(), rtol=rt, atol=at * scale)
    np.testing.assert_allclose(np64(leaves[0].grad), rx.grad.numpy(), rtol=rt, atol=at * scale)
    gs = max(1.0, float(rw.grad.abs().max()))
    np.testing.assert_allclose(np64(leaves[1].grad), rw.grad.numpy(), rtol=rt, atol=at * gs * 10)
    if bias is not None:
        np.testing.assert_allclose(np64(bl.grad), rb.grad.numpy(), rtol=rt, atol=at * gs * 10)


@pytest.mark.parametrize("W,L,D,B", [(1, 33, 37, 2), (3, 70, 100, 3), (8, 31, 64, 1), (5, 97, 130, 2)])
def test_backward_widths_and_ragged_shapes(dev, W, L, D, B):
    """float64 backward across widths, sequence lengths that end inside a 32-step workgroup
    block and channel counts that end inside a 64-channel one (the per-workgroup weight
    partial rows and their fixed-order sum)."""
    x, w, bias = inputs(B, L, D, W, seed=W * 31 + L)
    leaves = [t.to(dev).requires_grad_() for t in (x, w, bias)]
    y = causal_conv1d(*leaves)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(W + L), dtype=torch.float64)
    y.backward(dy.to(dev))
    refs = [t.detach().clone().requires_grad_() for t in (x, w, bias)]
    ref_conv(*refs).backward(dy)
    for a, r, name in zip(leaves, refs, ("dx", "dw", "dbias")):
        np.testing.assert_allclose(np64(a.grad), r.grad.numpy(), rtol=1e-12, atol=1e-12, err_msg=name)


def test_nn_conv1d_weight_and_contiguous_input(dev):
    x, w, bias = inputs(2, 70, 32, 4, seed=3, split_view=False)
    conv = torch.nn.Conv1d(32, 32, 4, groups=32, bias=True).double()
    with torch.no_grad():
        conv.weight.copy_(w.unsqueeze(1))
        conv.bias.copy_(bias)
    y = causal_conv1d(x.to(dev), conv.weight.to(dev), conv.bias.to(dev))
    ry = F.silu(conv(F.pad(x.transpose(1, 2), (3, 0)))).transpose(1, 2)
    np.testing.assert_allclose(np64(y), ry.detach().numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("W", [2, 4, 6])
def test_state_streaming_and_decode_equal_full(dev, W):
    """Pieces with the carried state, and single tokens, reproduce the full sequence."""
    x, w, bias = inputs(2, 67, 48, W, seed=W)
    xd, wd, bd = x.to(dev), w.to(dev), bias.to(dev)
    full = causal_conv1d(xd, wd, bd)
    state = torch.zeros(2, 48, W - 1, dtype=torch.float64, device=dev)
    pieces = [causal_conv1d(xd[:, a:b_], wd, bd, state=state) for a, b_ in ((0, 2), (2, 30), (30, 67))]
    np.testing.assert_allclose(np64(torch.cat(pieces, 1)), np64(full), rtol=1e-12, atol=1e-12)
    ry, rstate = R.conv1d_causal(np64(x).transpose(0, 2, 1), np64(w), np64(bias))
    np.testing.assert_allclose(np64(state), rstate, rtol=0, atol=0)
    state2 = torch.zeros_like(state)
    steps = [causal_conv1d(xd[:, t:t + 1], wd, bd, state=state2) for t in range(67)]
    np.testing.assert_allclose(np64(torch.cat(steps, 1)), np64(full), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np64(state2), rstate, rtol=0, atol=0)


def test_conv_errors(dev):
    x = torch.zeros(1, 4, 8, device=dev)
    with pytest.raises(ValueError):
        causal_conv1d(x, torch.zeros(8, 9, device=dev))           # width 9 > 8
    with pytest.raises(ValueError):
        causal_conv1d(x, torch.zeros(7, 4, device=dev))
    with pytest.raises(RuntimeError):
        causal_conv1d(x.cpu(), torch.zeros(8, 4))


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_forward_backward_match_torch(dev, seed):
    """Seeded random shapes (B 1-4, L 1-599, D 1-299, W 1-8), activation, bias and the split
    in_proj view, float32 against torch float64 autograd: y and dx at the float32 conv bar, the
    weight and bias gradients (sums over B x L tokens) at rtol 1e-4 / atol 1e-5.  A 300-draw
    sweep of the same draws had none outside."""
    rng = np.random.default_rng(seed)
    B, L, D, W = int(rng.integers(1, 5)), int(rng.integers(1, 600)), int(rng.integers(1, 300)), int(rng.integers(1, 9))
    act, with_bias, split = bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    print(f"case seed={seed} B={B} L={L} D={D} W={W} activation={act} bias={with_bias} split={split}", flush=True)
    x, w, bias = inputs(B, L, D, W, seed=seed, split_view=split)
    if not with_bias:
        bias = None
    xg, wg = x.to(dev, torch.float32).requires_grad_(), w.to(dev, torch.float32).requires_grad_()
    bg = None if bias is None else bias.to(dev, torch.float32).requires_grad_()
    y = causal_conv1d(xg, wg, bg, activation=act)
    dy = torch.randn(B, L, D, generator=torch.Generator().manual_seed(seed + 1), dtype=torch.float64)
    (y * dy.to(dev, torch.float32)).sum().backward()
    xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
    br = None if bias is None else bias.clone().requires_grad_()
    (ref_conv(xr, wr, br, activation=act) * dy).sum().backward()
    rt, at = TOL[torch.float32]
    yr = ref_conv(x, w, bias, activation=act)
    np.testing.assert_allclose(np64(y), yr.numpy(), rtol=rt, atol=at, err_msg="y")
    np.testing.assert_allclose(np64(xg.grad), xr.grad.numpy(), rtol=rt, atol=at, err_msg="dx")
    np.testing.assert_allclose(np64(wg.grad), wr.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg="dw")
    if bg is not None:
        np.testing.assert_allclose(np64(bg.grad), br.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg="dbias")
