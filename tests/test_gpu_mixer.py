"""One Mamba layer through the single-node mixer (conv -> x_proj -> fused scan as one autograd
node, ssm_scan.mixer) against the float64 restatement of models/mamba.py:93-126
(oracle/lm_ref.mamba_layer) on identical weights: the output, the input gradient and every
parameter gradient, for each discretization and for shapes whose dt_rank, d_state, d_inner and
conv width are not the defaults or multiples of the kernels' tiles.  The module-by-module path
(taken when the layer records its delta) gives the same gradients.

Tolerances: float32 -- output rtol 1e-4 / atol 1e-5 x max|y|, gradients rtol 1e-3 / atol 1e-4
x max|grad| per parameter (a gradient sums over B x L tokens).
"""

import pytest
import torch

from ssm_scan.block import Mamba
from ssm_scan.mixer import mixer_applies
from oracle import lm_ref

pytestmark = pytest.mark.gpu


def close(a, b, rtol, atol_frac):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    atol = atol_frac * max(b.abs().max().item(), 1e-30)
    assert torch.allclose(a, b, rtol=rtol, atol=atol), (a - b).abs().max().item()


def run_layer(m, u, dy):
    u = u.clone().requires_grad_()
    for p in m.parameters():
        p.grad = None
    y = m(u)
    y.backward(dy)
    return y, u.grad, {k: p.grad.clone() for k, p in m.named_parameters()}


@pytest.mark.parametrize("d_model,d_state,dt_rank,method,B,L,d_conv", [
    (64, 16, None, "zoh", 2, 96, 4),
    (40, 8, 3, "bilinear", 3, 37, 4),
    (48, 16, 5, "euler", 1, 130, 4),
    (56, 12, 4, "zoh", 2, 50, 3),
])
def test_mixer_layer_matches_reference(dev, d_model, d_state, dt_rank, method, B, L, d_conv):
    torch.manual_seed(d_model + L)
    m = Mamba(d_model, d_state=d_state, dt_rank=dt_rank, discretization=method, d_conv=d_conv).to(dev)
    u = torch.randn(B, L, d_model, device=dev)
    dy = torch.randn(B, L, d_model, device=dev)
    assert mixer_applies(m, u, None, False)
    y, du, grads = run_layer(m, u, dy)

    p = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()}
    u64 = u.detach().cpu().double().requires_grad_()
    y64 = lm_ref.mamba_layer(p, "", u64, d_state, m.dt_rank, m.d_conv, method=method)
    y64.backward(dy.cpu().double())
    close(y, y64, 1e-4, 1e-5)
    close(du, u64.grad, 1e-3, 1e-4)
    for k, g in grads.items():
        close(g, p[k].grad, 1e-3, 1e-4)

    m.record_delta = True                     # module-by-module path
    assert not mixer_applies(m, u, None, False)
    y2, du2, grads2 = run_layer(m, u, dy)
    close(y, y2, 1e-5, 1e-6)
    close(du, du2, 1e-4, 1e-5)
    for k in grads:
        close(grads[k], grads2[k], 1e-4, 1e-5)
