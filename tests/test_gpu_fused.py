"""Parity of the fused HIP engine (libssmscan.so, ssm_fwd / ssm_bwd) with the float64 oracle.

Tolerances (tests/parity.py): float32 inputs rtol 1e-4 / atol 1e-5 on
every element of the outputs and of every gradient, with no scaling by the tensor's magnitude;
bf16 inputs with a float32 state rtol 2e-2.  Each check prints its count of elements outside
the bar.  Shapes: the reference's own GPU
test shapes (tests/test_triton.py:31), the BASELINE configs 0 and 1, and edge cases (L = 1,
ragged L and D, dstate not a power of two, non-contiguous views, expanded A).
"""

import numpy as np
import pytest
import torch

import ssm_scan
from oracle import c_oracle
from oracle import scan_ref as R
from ssm_inputs import baseline_inputs, np64, triton_test_inputs

pytestmark = pytest.mark.gpu

from parity import ATOL, ATOL_BF16, RTOL, RTOL_BF16, close  # noqa: F401  (the north_star bar)


def run_fused(ins, dev, method, D=None, z=None, bias=None, softplus=False, dout=None, dlast=None):
    """GPU forward + backward through autograd; returns (out, last, grads dict)."""
    x, delta, A, Bm, Cm, h0 = ins
    names = ["dx", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias", "dh0"]
    leaves = [x, delta, A, Bm, Cm, D, z, bias, h0]
    gl = [None if t is None else t.to(dev).requires_grad_() for t in leaves]
    out, last = ssm_scan.selective_scan_fn(gl[0], gl[1], gl[2], gl[3], gl[4], D=gl[5], z=gl[6],
                                           delta_bias=gl[7], delta_softplus=softplus, h0=gl[8],
                                           method=method, return_last_state=True)
    loss = (out * dout.to(dev)).sum()
    if dlast is not None:
        loss = loss + (last * dlast.to(dev)).sum()
    loss.backward()
    grads = {n: t.grad for n, t in zip(names, gl) if t is not None}
    return out.detach(), last.detach(), grads


def oracle(ins, method, D=None, z=None, bias=None, softplus=False, dout=None, dlast=None, use_c=False,
           mag=False):
    x, delta, A, Bm, Cm, h0 = (np64(t) for t in ins)
    raw = delta
    if bias is not None:
        raw = raw + np64(bias)
    d_eff = np.log1p(np.exp(raw)) if softplus else raw
    fwd = c_oracle.fwd if use_c else R.selective_scan_fwd
    out, _, last = fwd(x, d_eff, A, Bm, Cm, h0, method, np64(D), np64(z))
    if use_c:
        g = c_oracle.bwd(x, d_eff, A, Bm, Cm, np64(dout), h0, method, np64(D), np64(z), np64(dlast), mag=mag)
    else:
        g = R.selective_scan_bwd(x, d_eff, A, Bm, Cm, np64(dout), h0, method, np64(D), np64(z), np64(dlast),
                                 mag=mag)
    if softplus or bias is not None:
        dd_raw = g["ddelta"] * (1.0 / (1.0 + np.exp(-raw)) if softplus else 1.0)
        g["ddelta"] = dd_raw
        if mag:
            g["ddelta_mag"] = g["ddelta_mag"] * (1.0 / (1.0 + np.exp(-raw)) if softplus else 1.0)
        if bias is not None:
            g["ddelta_bias"] = dd_raw.sum(axis=(0, 1))
    return out, last, g


GRAD_MAP = {"dx": "dx", "ddelta": "ddelta", "dA": "dA", "dB": "dB", "dC": "dC", "dD": "dD",
            "dz": "dz", "ddelta_bias": "ddelta_bias", "dh0": "dh0"}


def check_all(got, ref, rtol=RTOL, atol=ATOL):
    out, last, grads = got
    rout, rlast, rg = ref
    close(out, rout, rtol, atol, "out")
    close(last, rlast, rtol, atol, "last")
    for k, v in grads.items():
        close(v, rg[GRAD_MAP[k]], rtol, atol, k)


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
@pytest.mark.parametrize("shape", [(2, 1, 32, 16), (2, 37, 50, 16), (3, 130, 96, 8)])
@pytest.mark.parametrize("h0", [False, True])
def test_reference_shapes_match_oracle(dev, method, shape, h0):
    """tests/test_triton.py:28-44 shapes and input distributions; y, last and all 6 grads."""
    ins = triton_test_inputs(*shape, h0)
    g = torch.Generator().manual_seed(1)
    dout = torch.randn(shape[0], shape[1], shape[2], generator=g)
    dlast = torch.randn(shape[0], shape[2], shape[3], generator=g)
    got = run_fused(ins, dev, method, dout=dout, dlast=dlast)
    ref = oracle(ins, method, dout=dout, dlast=dlast)
    check_all(got, ref)


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
def test_gate_skip_bias_softplus_match_oracle(dev, method):
    B, L, D, N = 2, 75, 40, 16
    ins = triton_test_inputs(B, L, D, N, True, seed=3)
    g = torch.Generator().manual_seed(4)
    Dv = torch.randn(D, generator=g)
    z = torch.randn(B, L, D, generator=g)
    bias = torch.randn(D, generator=g) * 0.5 - 3.0
    raw_delta = torch.randn(B, L, D, generator=g) * 0.5
    ins = (ins[0], raw_delta, *ins[2:])
    dout = torch.randn(B, L, D, generator=g)
    got = run_fused(ins, dev, method, D=Dv, z=z, bias=bias, softplus=True, dout=dout)
    ref = oracle(ins, method, D=Dv, z=z, bias=bias, softplus=True, dout=dout)
    check_all(got, ref)


@pytest.mark.parametrize("N", [1, 3, 8, 12, 32, 64])
def test_dstate_padding(dev, N):
    """dstate that is not a padded width (1, 3, 12) or the larger tiles (32, 64)."""
    ins = triton_test_inputs(2, 45, 20, N, True, seed=N)
    g = torch.Generator().manual_seed(N + 1)
    dout = torch.randn(2, 45, 20, generator=g)
    got = run_fused(ins, dev, "zoh", dout=dout)
    ref = oracle(ins, "zoh", dout=dout)
    check_all(got, ref)


def test_config0_forward_matches_c_oracle(dev):
    """B1 L512 D512 N16 fp32, no gate."""
    t = baseline_inputs(1, 512, 512, 16)
    with torch.no_grad():
        y, last = ssm_scan.selective_scan_hip(t["u"].to(dev), t["delta"].to(dev), t["A"].to(dev),
                                              t["Bm"].to(dev), t["Cm"].to(dev))
    ry, _, rlast = c_oracle.fwd(np64(t["u"]), np64(t["delta"]), np64(t["A"]), np64(t["Bm"]), np64(t["Cm"]))
    close(y, ry, name="y")
    close(last, rlast, name="last")


def test_config1_fwd_bwd_matches_c_oracle(dev):
    """B16 L512 D512 N16 fp32 with z gate and D skip; all gradients."""
    t = baseline_inputs(16, 512, 512, 16, gate=True, with_dy=True)
    ins = (t["u"], t["delta"], t["A"], t["Bm"], t["Cm"], None)
    got = run_fused(ins, dev, "zoh", D=t["D"], z=t["z"], dout=t["dy"])
    ref = oracle(ins, "zoh", D=t["D"], z=t["z"], dout=t["dy"], use_c=True)
    check_all(got, ref)   # every element of every tensor within the bar (no exception at c1)


@pytest.mark.parametrize("D", [1536, 5120])
def test_wide_model_matches_oracle(dev, D):
    """The channel widths of the larger Mamba models (d_inner 1536 and 5120): 48 / 160 channel
    tiles whose dB / dC partials the finalize sums; gate, D skip, dt bias + softplus, h0 and
    dlast.  Every element of every output and gradient against the float64 oracle at the bar."""
    B, L, N = 2, 160, 16
    print(f"case B{B} L{L} D{D} N{N}", flush=True)
    g = torch.Generator().manual_seed(D)
    x = torch.randn(B, L, D, generator=g)
    delta = torch.randn(B, L, D, generator=g) * 0.5 - 1.0
    bias = torch.randn(D, generator=g) * 0.5 - 2.0
    A = -(torch.rand(D, N, generator=g) * 4 + 0.05)
    Bm, Cm = torch.randn(B, L, N, generator=g), torch.randn(B, L, N, generator=g)
    h0, Dv, z = torch.randn(B, D, N, generator=g), torch.randn(D, generator=g), torch.randn(B, L, D, generator=g)
    dout, dlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    ins = (x, delta, A, Bm, Cm, h0)
    got = run_fused(ins, dev, "zoh", D=Dv, z=z, bias=bias, softplus=True, dout=dout, dlast=dlast)
    check_all(got, oracle(ins, "zoh", D=Dv, z=z, bias=bias, softplus=True, dout=dout, dlast=dlast))


@pytest.mark.parametrize("B", [300, 65535])
def test_large_batch_matches_oracle(dev, B):
    """Batch rows up to the grid's y limit (65535): one workgroup row per batch row, and the
    finalize summing dA, dD and d_bias over every row in order.  Short rows (L 3, D 8, N 4),
    gate, D skip, bias + softplus, h0 and dlast; every output and gradient at the bar."""
    L, D, N = 3, 8, 4
    print(f"case B{B} L{L} D{D} N{N}", flush=True)
    g = torch.Generator().manual_seed(B)
    ins = (torch.randn(B, L, D, generator=g), torch.randn(B, L, D, generator=g) * 0.5 - 1.0,
           -(torch.rand(D, N, generator=g) * 4 + 0.05), torch.randn(B, L, N, generator=g),
           torch.randn(B, L, N, generator=g), torch.randn(B, D, N, generator=g))
    Dv, z, bias = torch.randn(D, generator=g), torch.randn(B, L, D, generator=g), torch.randn(D, generator=g) * 0.5
    dout, dlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    got = run_fused(ins, dev, "zoh", D=Dv, z=z, bias=bias, softplus=True, dout=dout, dlast=dlast)
    check_all(got, oracle(ins, "zoh", D=Dv, z=z, bias=bias, softplus=True, dout=dout, dlast=dlast))


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
def test_gradcheck_float64(dev, method):
    """tests/test_scan.py:85-88 on the engine: torch.autograd.gradcheck (central differences in
    float64 against the float64 kernels' backward) at B1 L6 D2 N3, with the gate, D skip, dt
    bias + softplus and h0, for the output and the last state."""
    g = torch.Generator().manual_seed(7)
    B, L, D, N = 1, 6, 2, 3
    mk = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64).to(dev).requires_grad_()
    x, delta, Bm, Cm, z, h0 = mk(B, L, D), mk(B, L, D), mk(B, L, N), mk(B, L, N), mk(B, L, D), mk(B, D, N)
    A = (-(torch.rand(D, N, generator=g, dtype=torch.float64) * 2 + 0.1)).to(dev).requires_grad_()
    Dv, bias = mk(D), mk(D)

    def fn(x, delta, A, Bm, Cm, Dv, z, bias, h0):
        return ssm_scan.selective_scan_fn(x, delta, A, Bm, Cm, D=Dv, z=z, delta_bias=bias, delta_softplus=True,
                                          h0=h0, method=method, return_last_state=True)

    assert torch.autograd.gradcheck(fn, (x, delta, A, Bm, Cm, Dv, z, bias, h0), eps=1e-6, atol=1e-6, rtol=1e-4,
                                    nondet_tol=0.0)


def test_backward_is_bitwise_deterministic(dev):
    """tests/test_gpu.py:28-46: two backward passes are torch.equal (always, not only in
    torch's deterministic mode: every reduction here is fixed-order)."""
    x, delta, A, Bm, Cm, _ = triton_test_inputs(3, 300, 96, 16, False)
    ins = [t.to(dev).requires_grad_() for t in (x, delta, A, Bm, Cm)]

    def grads():
        y, _ = ssm_scan.selective_scan_hip(*ins)
        return torch.autograd.grad(y.square().sum(), ins)

    g1, g2 = grads(), grads()
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_layouts_and_strided_views_agree(dev):
    """Time-major, channel-major and strided split views (models/mamba.py:75,101,107) give
    bitwise identical results; A may be an expanded (stride-0) scalar-decay view."""
    B, L, D, N = 2, 70, 48, 16
    x, delta, A, Bm, Cm, h0 = (t.to(dev) for t in triton_test_inputs(B, L, D, N, True, seed=5))
    A_scalar = A[:, :1].expand(D, N)
    ref_y, ref_last = ssm_scan.selective_scan_hip(x, delta, A_scalar.contiguous(), Bm, Cm, h0)
    xc = x.transpose(1, 2).contiguous().transpose(1, 2)          # channel-major storage
    proj = torch.cat([torch.randn(B, L, 5, device=dev), Bm, Cm], -1)  # x_proj-style split
    Bv, Cv = proj[..., 5:5 + N], proj[..., 5 + N:]
    y2, last2 = ssm_scan.selective_scan_hip(xc, delta.transpose(1, 2).contiguous().transpose(1, 2),
                                            A_scalar, Bv, Cv, h0)
    assert torch.equal(ref_y, y2) and torch.equal(ref_last, last2)


def test_bf16_inputs(dev):
    """bf16 u, delta, B, C (state float32): rtol 2e-2 against the oracle on the rounded inputs."""
    t = baseline_inputs(2, 256, 128, 16, dtype=torch.bfloat16)
    ins = [t[k].to(dev) for k in ("u", "delta", "A", "Bm", "Cm")]
    with torch.no_grad():
        y, last = ssm_scan.selective_scan_hip(*ins)
    assert y.dtype == torch.bfloat16 and last.dtype == torch.float32
    ry, _, rlast = c_oracle.fwd(*(np64(v) for v in ins))
    close(y, ry, RTOL_BF16, ATOL_BF16, "y")
    close(last, rlast, RTOL_BF16, ATOL_BF16, "last")


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float16, 4e-3)])
def test_half_precision_inputs_forward_and_backward(dev, dtype, tol):
    """16-bit x, delta, B, C, z (A, D, bias, h0 and the state float32), forward and every
    gradient, against the oracle on the rounded inputs.  The kernels compute in float32, so the
    error is the 16-bit rounding of the outputs and gradients: 8 significand bits for bf16, 11
    for float16 (rtol ~8 units of that rounding, atol 1e-5)."""
    x, delta, A, Bm, Cm, h0 = triton_test_inputs(2, 70, 40, 16, True, seed=21)
    g = torch.Generator().manual_seed(22)
    Dv, bias = torch.randn(40, generator=g), torch.randn(40, generator=g) * 0.5 - 1.0
    z = torch.randn(2, 70, 40, generator=g)
    dout = torch.randn(2, 70, 40, generator=g).to(dtype)
    lo = [t.to(dtype) for t in (x, delta, Bm, Cm, z)]
    ins = (lo[0], lo[1], A, lo[2], lo[3], h0)
    got = run_fused(ins, dev, "zoh", D=Dv, z=lo[4], bias=bias, softplus=True, dout=dout)
    assert got[0].dtype == dtype and got[1].dtype == torch.float32
    assert got[2]["dx"].dtype == dtype and got[2]["dA"].dtype == torch.float32
    ref = oracle(ins, "zoh", D=Dv, z=lo[4], bias=bias, softplus=True, dout=dout)
    check_all(got, ref, rtol=tol, atol=ATOL)


def test_float64_inputs(dev):
    """float64 inputs compute in float64 (promote(dtype, float32)); tight agreement."""
    ins = [t.double() if t is not None else None for t in triton_test_inputs(2, 50, 24, 16, True, seed=8)]
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(2, 50, 24, generator=g, dtype=torch.float64)
    got = run_fused(ins, dev, "zoh", dout=dout)
    ref = oracle(ins, "zoh", dout=dout)
    check_all(got, ref, rtol=1e-9, atol=1e-10)


def test_decode_step_matches_forward(dev):
    """The recurrent step applied L times equals the fused forward (tests/test_gpu.py:49-65)."""
    B, L, D, N = 4, 24, 64, 16
    x, delta, A, Bm, Cm, h0 = (t.to(dev) for t in triton_test_inputs(B, L, D, N, True, seed=11))
    g = torch.Generator().manual_seed(12)
    Dv = torch.randn(D, generator=g).to(dev)
    z = torch.randn(B, L, D, generator=g).to(dev)
    with torch.no_grad():
        out, last = ssm_scan.selective_scan_fn(x, delta, A, Bm, Cm, D=Dv, z=z, h0=h0, return_last_state=True)
        h = h0.clone()
        steps = [ssm_scan.ssm_step(h, x[:, t], delta[:, t], A, Bm[:, t], Cm[:, t], D=Dv, z=z[:, t])
                 for t in range(L)]
    torch.testing.assert_close(torch.stack(steps, 1), out, rtol=RTOL, atol=ATOL)
    torch.testing.assert_close(h, last, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_decode_step_dtypes_bias_softplus(dev, dtype, method):
    """ssm_step with dt bias + softplus, D skip and gate for float32, bf16 (float32 state) and
    float64 inputs against the oracle's step (models/mamba.py:113-118,122-124) on the same
    (rounded) inputs: the state at the float32 bar (float64: 1e-10), the output at the bar of
    its dtype (bf16 output rounding: rtol 2e-2)."""
    g = torch.Generator().manual_seed(21)
    B, D, N = 5, 40, 16
    ct = torch.float64 if dtype == torch.float64 else torch.float32
    mk = lambda *s, dt=dtype: torch.randn(*s, generator=g, dtype=torch.float64).to(dt)
    h = mk(B, D, N, dt=ct)
    x, delta, z = mk(B, D), mk(B, D) * 0.5 - 1.0, mk(B, D)
    A = -(torch.rand(D, N, generator=g, dtype=torch.float64) * 4 + 0.05).to(ct)
    Bm, Cm, Dv, bias = mk(B, N), mk(B, N), mk(D, dt=ct), mk(D, dt=ct) * 0.5
    h_dev = h.to(dev)
    out = ssm_scan.ssm_step(h_dev, x.to(dev), delta.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev), D=Dv.to(dev),
                            z=z.to(dev), delta_bias=bias.to(dev), delta_softplus=True, method=method)
    torch.cuda.synchronize()
    d_eff = np.log1p(np.exp(np64(delta) + np64(bias)))
    ry, rh = R.ssm_step(np64(h), np64(x), d_eff, np64(A), np64(Bm), np64(Cm), method, np64(Dv), np64(z))
    assert out.dtype == dtype and h_dev.dtype == ct
    if dtype == torch.float64:
        close(out, ry, 1e-10, 1e-10, "y")
        close(h_dev, rh, 1e-10, 1e-10, "h")
    else:
        close(h_dev, rh, name="h")
        close(out, ry, *((RTOL_BF16, ATOL_BF16) if dtype == torch.bfloat16 else (RTOL, ATOL)), "y")


def test_cpu_tensors_are_rejected():
    x, delta, A, Bm, Cm, _ = triton_test_inputs(1, 4, 8, 16, False)
    with pytest.raises(RuntimeError, match="GPU"):
        ssm_scan.selective_scan_hip(x, delta, A, Bm, Cm)


@pytest.mark.parametrize("lowrank,L,scalar", [(False, 77, False), (True, 600, False), (True, 64, True)])
def test_A_log_input_equals_A_input(dev, lowrank, L, scalar):
    """A_is_log: the kernels form A = -exp(A_log) (models/mamba.py:81) and return the gradient of
    A_log; equal to passing -exp(A_log) with torch and chaining its gradient, to float32
    rounding (one exp evaluated by the kernel, one by torch).  Covers the low-rank delta, time
    segments (B 1, L 600) and a stride-0 expanded A_log (the scalar-decay mode)."""
    B, D, N, Rk = (1, 64, 16, 8) if L == 600 else (2, 40, 16, 8)
    g = torch.Generator().manual_seed(L)
    x = torch.randn(B, L, D, generator=g).to(dev)
    dt = (torch.randn(B, L, Rk if lowrank else D, generator=g) * 0.5).to(dev)
    W = (torch.randn(D, Rk, generator=g) * 0.3).to(dev) if lowrank else None
    A_log = torch.log(torch.rand(D, 1 if scalar else N, generator=g) * 4 + 0.5).to(dev)
    Bm, Cm = torch.randn(B, L, N, generator=g).to(dev), torch.randn(B, L, N, generator=g).to(dev)
    Dv, z = torch.randn(D, generator=g).to(dev), torch.randn(B, L, D, generator=g).to(dev)
    bias = (torch.rand(D, generator=g) - 3.0).to(dev)
    dout = torch.randn(B, L, D, generator=g).to(dev)
    res = []
    for as_log in (True, False):
        leaf = A_log.clone().requires_grad_()
        A = leaf if as_log else -torch.exp(leaf)
        if scalar:
            A = A.expand(-1, N)
        out = ssm_scan.selective_scan_fn(x, dt, A, Bm, Cm, D=Dv, z=z, delta_bias=bias, delta_softplus=True,
                                         delta_proj=W, A_is_log=as_log)
        (out * dout).sum().backward()
        res.append((out.detach(), leaf.grad))
    torch.testing.assert_close(res[0][0], res[1][0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(res[0][1], res[1][1], rtol=1e-4, atol=1e-5)
