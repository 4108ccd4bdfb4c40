"""Seeded synthetic workloads of the BASELINE configs (the counterpart of
benchmarks/bench_scan.py:25-32 make_inputs), shared by bench.py and the tests.

All tensors are drawn on the CPU from torch.Generator().manual_seed(seed) in a fixed order
(the style of benchmarks/bench_scan.py:26-32), so the CPU oracle and the GPU see identical
values; callers move them to the device.
"""

import math

import torch


def baseline_inputs(B, L, D, N, seed=0, gate=False, dtype=torch.float32, with_dy=False):
    """u ~ N(0,1) stored (B, D, L); delta = softplus(0.5 N(0,1) +
    dt_bias) with dt_bias the inverse softplus of dt ~ logU[1e-3, 1e-1] per channel
    (models/mamba.py:40-42); A = -(1..N) broadcast over D (models/mamba.py:61,81); B, C ~ N(0,1)
    stored (B, N, L); D_skip = 1; optional z ~ N(0,1) (B, D, L) and dy ~ N(0,1).
    Returned in the logical layouts (B, L, D) / (B, L, N) as transposed views of the
    channel-major storage.  bf16 variants round u, delta, B, C (and z, dy) to bf16."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, D, L, generator=g)
    dt = torch.exp(torch.rand(D, generator=g) * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3))
    dt = dt.clamp(min=1e-4)
    dt_bias = dt + torch.log(-torch.expm1(-dt))
    delta = torch.nn.functional.softplus(0.5 * torch.randn(B, D, L, generator=g) + dt_bias[None, :, None])
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1)
    Bm = torch.randn(B, N, L, generator=g)
    Cm = torch.randn(B, N, L, generator=g)
    Dskip = torch.ones(D)
    out = dict(u=u, delta=delta, A=A, Bm=Bm, Cm=Cm, D=Dskip)
    if gate:
        out["z"] = torch.randn(B, D, L, generator=g)
    if with_dy:
        out["dy"] = torch.randn(B, D, L, generator=g)
    for k in ("u", "delta", "Bm", "Cm", "z", "dy"):
        if k in out:
            out[k] = out[k].to(dtype).transpose(1, 2)
    return out


def triton_test_inputs(B, L, D, N, h0, seed=0):
    """The distributions of the reference's GPU kernel test (tests/test_triton.py:17-25):
    x ~ N(0,1); delta ~ U[1e-3, 0.301]; A ~ -U[0.05, 4.05]; B, C ~ N(0,1); h0 ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, L, D, generator=g)
    delta = torch.rand(B, L, D, generator=g) * 0.3 + 1e-3
    A = -torch.rand(D, N, generator=g) * 4 - 0.05
    Bm = torch.randn(B, L, N, generator=g)
    Cm = torch.randn(B, L, N, generator=g)
    hz = torch.randn(B, D, N, generator=g) if h0 else None
    return x, delta, A, Bm, Cm, hz
