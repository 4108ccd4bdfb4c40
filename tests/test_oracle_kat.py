"""Pins the float64 oracle (oracle/scan_ref.py, oracle/ssm_oracle.c) against known answers.

Mirrors the reference's own checks (tests/test_scan.py:20-142) and adds independent
derivations of every gradient (torch.autograd and finite differences), so that a dropped
term, a wrong sign or a transposed operand in the oracle fails here.
"""

import math

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import scan_ref as R

RNG = np.random.default_rng(0)


def rand_ab(B=2, L=37, D=3, N=4, seed=0):
    g = np.random.default_rng(seed)
    return g.random((B, L, D, N)) * 0.9 + 0.05, g.standard_normal((B, L, D, N))


def scalar_bruteforce_scan(a, b, h0):
    """Pure-Python scalar loops (tests/test_scan.py:20-31 style)."""
    out = np.zeros_like(b)
    for i in range(a.shape[0]):
        for d in range(a.shape[2]):
            for n in range(a.shape[3]):
                h = float(h0[i, d, n])
                for t in range(a.shape[1]):
                    h = float(a[i, t, d, n]) * h + float(b[i, t, d, n])
                    out[i, t, d, n] = h
    return out


# --------------------------------------------------------------------------- scans

def test_sequential_matches_scalar_bruteforce():
    a, b = rand_ab(L=25)
    h0 = RNG.standard_normal((2, 3, 4))
    np.testing.assert_allclose(R.scan_sequential(a, b, h0), scalar_bruteforce_scan(a, b, h0), rtol=1e-12)


@pytest.mark.parametrize("L", [1, 2, 7, 16, 37, 64, 100])
@pytest.mark.parametrize("name", list(R.SCANS))
@pytest.mark.parametrize("with_h0", [False, True])
def test_scans_match_sequential(name, L, with_h0):
    a, b = rand_ab(L=L, seed=L)
    h0 = RNG.standard_normal((2, 3, 4)) if with_h0 else None
    np.testing.assert_allclose(R.SCANS[name](a, b, h0), R.scan_sequential(a, b, h0), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("chunk", [1, 3, 8, 64])
def test_chunked_any_chunk_size(chunk):
    a, b = rand_ab(L=50)
    np.testing.assert_allclose(R.scan_chunked(a, b, None, chunk), R.scan_sequential(a, b), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("name", ["hillis_steele", "blelloch", "chunked"])
def test_scans_long_sequence_extreme_decays(name):
    g = np.random.default_rng(1)
    a = g.random((1, 2048, 2, 3))
    a[..., 0, :] = 1 - 1e-4 * g.random((1, 2048, 3))
    a[..., 1, :] = 1e-6 * g.random((1, 2048, 3))
    b = g.standard_normal((1, 2048, 2, 3))
    out = R.SCANS[name](a, b)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, R.scan_sequential(a, b), rtol=1e-9, atol=1e-9)


def test_scan_is_linear_in_b_and_h0():
    a, b = rand_ab(L=30, seed=3)
    b2 = RNG.standard_normal(b.shape)
    h0, h02 = RNG.standard_normal((2, 3, 4)), RNG.standard_normal((2, 3, 4))
    lhs = R.scan_sequential(a, 2.0 * b - b2, 2.0 * h0 - h02)
    rhs = 2.0 * R.scan_sequential(a, b, h0) - R.scan_sequential(a, b2, h02)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-11, atol=1e-11)


# --------------------------------------------------------------------------- discretization

def test_diagonal_zoh_matches_dense_matrix_exponential():
    D, N = 3, 5
    A = -RNG.random((D, N)) * 3 - 0.1
    Bv = RNG.standard_normal(N)
    delta = RNG.random(D) * 0.7
    x = RNG.standard_normal(D)
    a, b = R.discretize(delta.reshape(1, 1, D), A, Bv.reshape(1, 1, N), x.reshape(1, 1, D), "zoh")
    for d in range(D):
        Ad, Bd = R.zoh_matrix(np.diag(A[d]), Bv[:, None], float(delta[d]))
        np.testing.assert_allclose(a[0, 0, d], np.diagonal(Ad), rtol=1e-12)
        np.testing.assert_allclose(b[0, 0, d], Bd[:, 0] * x[d], rtol=1e-10, atol=1e-14)


def test_zoh_is_exact_for_piecewise_constant_input():
    """RK4 over one step of dh/dt = A h + B u must equal the dense ZOH (tests/test_scan.py:104-116)."""
    A = np.array([[-1.0, 0.5], [-0.3, -2.0]])
    B = np.array([[1.0], [0.5]])
    h = np.array([[0.2], [-0.4]])
    u, delta, steps = 0.7, 0.3, 2000
    f = lambda s: A @ s + B * u
    s, dt = h.copy(), delta / steps
    for _ in range(steps):
        k1 = f(s); k2 = f(s + dt / 2 * k1); k3 = f(s + dt / 2 * k2); k4 = f(s + dt * k3)
        s = s + dt / 6 * (k1 + 2 * k2 + 2 * k3 + k4)
    Ad, Bd = R.zoh_matrix(A, B, delta)
    np.testing.assert_allclose(Ad @ h + Bd * u, s, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("method", ["euler", "bilinear"])
def test_discretizations_converge_to_zoh(method):
    A = -RNG.random((4, 3)) - 0.5
    x, Bm = RNG.standard_normal((1, 1, 4)), RNG.standard_normal((1, 1, 3))
    errs = []
    for dt in (1e-1, 1e-2, 1e-3):
        delta = np.full((1, 1, 4), dt)
        za, zb = R.discretize(delta, A, Bm, x, "zoh")
        ma, mb = R.discretize(delta, A, Bm, x, method)
        errs.append(np.abs(za - ma).max() + np.abs(zb - mb).max())
    assert errs[0] > errs[1] > errs[2] and errs[2] < 1e-5


def test_bilinear_is_pade_of_exp():
    """Tustin a = (1 + z/2)/(1 - z/2) agrees with exp(z) to O(z^3) (third-order term z^3/12)."""
    z = -np.array([1e-2, 2e-2, 4e-2])
    a, _ = R.discretize(z.reshape(1, 1, 3), np.ones((3, 1)), np.ones((1, 1, 1)), np.ones((1, 1, 3)), "bilinear")
    err = a[0, 0, :, 0] - np.exp(z)
    np.testing.assert_allclose(err, z ** 3 / 12.0, rtol=2e-1)


def test_unknown_method_raises():
    with pytest.raises(ValueError):
        R.discretize(np.ones((1, 1, 1)), -np.ones((1, 1)), np.ones((1, 1, 1)), np.ones((1, 1, 1)), "rk4")


# --------------------------------------------------------------------------- selective scan fwd

def sel_inputs(B=2, L=9, D=3, N=4, seed=0, h0=True, gate=True):
    g = np.random.default_rng(seed)
    x = g.standard_normal((B, L, D))
    delta = g.random((B, L, D)) * 0.5 + 0.01
    A = -g.random((D, N)) * 2 - 0.1
    Bm = g.standard_normal((B, L, N))
    Cm = g.standard_normal((B, L, N))
    hz = g.standard_normal((B, D, N)) if h0 else None
    Dv = g.standard_normal(D) if gate else None
    z = g.standard_normal((B, L, D)) if gate else None
    return x, delta, A, Bm, Cm, hz, Dv, z


def scalar_selective_scan(x, delta, A, Bm, Cm, h0, method, Dv, z):
    Bsz, L, D = x.shape
    N = A.shape[1]
    out = np.zeros((Bsz, L, D))
    last = np.zeros((Bsz, D, N))
    for b in range(Bsz):
        for d in range(D):
            h = [float(h0[b, d, n]) if h0 is not None else 0.0 for n in range(N)]
            for t in range(L):
                y = 0.0
                for n in range(N):
                    zt = float(delta[b, t, d]) * float(A[d, n])
                    bx = float(Bm[b, t, n]) * float(x[b, t, d])
                    if method == "zoh":
                        a, bb = math.exp(zt), math.expm1(zt) / float(A[d, n]) * bx
                    elif method == "euler":
                        a, bb = math.exp(zt), float(delta[b, t, d]) * bx
                    else:
                        a = (1 + zt / 2) / (1 - zt / 2)
                        bb = float(delta[b, t, d]) / (1 - zt / 2) * bx
                    h[n] = a * h[n] + bb
                    y += float(Cm[b, t, n]) * h[n]
                o = y + (float(Dv[d]) * float(x[b, t, d]) if Dv is not None else 0.0)
                if z is not None:
                    zz = float(z[b, t, d])
                    o *= zz / (1 + math.exp(-zz))
                out[b, t, d] = o
            last[b, d] = h
    return out, last


@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
@pytest.mark.parametrize("h0,gate", [(False, False), (True, True), (True, False)])
def test_forward_matches_scalar_bruteforce(method, h0, gate):
    x, delta, A, Bm, Cm, hz, Dv, z = sel_inputs(h0=h0, gate=gate)
    out, _, last = R.selective_scan_fwd(x, delta, A, Bm, Cm, hz, method, Dv, z)
    out_s, last_s = scalar_selective_scan(x, delta, A, Bm, Cm, hz, method, Dv, z)
    np.testing.assert_allclose(out, out_s, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(last, last_s, rtol=1e-12, atol=1e-13)


# --------------------------------------------------------------------------- selective scan bwd

def torch_textbook(x, delta, A, Bm, Cm, h0, method, Dv, z):
    """Independent torch restatement of the textbook loop; gradients come from autograd."""
    Bsz, L, D = x.shape
    h = torch.zeros(Bsz, D, A.shape[1], dtype=x.dtype) if h0 is None else h0
    ys = []
    for t in range(L):
        zt = delta[:, t, :, None] * A
        bx = x[:, t, :, None] * Bm[:, t, None, :]
        if method == "zoh":
            a, b = torch.exp(zt), torch.expm1(zt) / A * bx
        elif method == "euler":
            a, b = torch.exp(zt), delta[:, t, :, None] * bx
        else:
            a = (1 + zt / 2) / (1 - zt / 2)
            b = delta[:, t, :, None] / (1 - zt / 2) * bx
        h = a * h + b
        ys.append((h * Cm[:, t, None, :]).sum(-1))
    out = torch.stack(ys, 1)
    if Dv is not None:
        out = out + x * Dv
    if z is not None:
        out = out * torch.nn.functional.silu(z)
    return out, h


@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
@pytest.mark.parametrize("h0,gate,dlast", [(False, False, False), (True, True, True), (False, True, False),
                                           (True, False, True)])
def test_backward_matches_torch_autograd(method, h0, gate, dlast):
    ins = sel_inputs(B=2, L=11, D=3, N=5, seed=7, h0=h0, gate=gate)
    g = np.random.default_rng(11)
    dout = g.standard_normal(ins[0].shape)
    dl = g.standard_normal((2, 3, 5)) if dlast else None
    ours = R.selective_scan_bwd(*ins[:5], dout, ins[5], method, ins[6], ins[7], dl)
    tt = [None if v is None else torch.tensor(v, requires_grad=True) for v in ins]
    out, last = torch_textbook(*tt[:6], method, tt[6], tt[7])
    loss = (out * torch.tensor(dout)).sum()
    if dl is not None:
        loss = loss + (last * torch.tensor(dl)).sum()
    loss.backward()
    names = ["dx", "ddelta", "dA", "dB", "dC", "dh0", "dD", "dz"]
    for name, t in zip(names, tt):
        if t is None:
            assert name not in ours
            continue
        np.testing.assert_allclose(ours[name], t.grad.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)


def test_zoh_small_z_series_branch_is_accurate():
    """dA through the |z| < 1e-3 series branch agrees with autograd (tiny delta)."""
    x, delta, A, Bm, Cm, hz, Dv, z = sel_inputs(B=1, L=8, D=2, N=3, seed=5, h0=True, gate=False)
    delta = delta * 1e-4
    dout = np.random.default_rng(2).standard_normal(x.shape)
    ours = R.selective_scan_bwd(x, delta, A, Bm, Cm, dout, hz, "zoh")
    tt = [torch.tensor(v, requires_grad=True) for v in (x, delta, A, Bm, Cm, hz)]
    out, _ = torch_textbook(*tt, "zoh", None, None)
    (out * torch.tensor(dout)).sum().backward()
    np.testing.assert_allclose(ours["dA"], tt[2].grad.numpy(), rtol=1e-9)


@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
def test_backward_matches_finite_differences(method):
    """Central differences, B1 L6 D2 N3 (tests/test_scan.py:85-88 shape)."""
    ins = list(sel_inputs(B=1, L=6, D=2, N=3, seed=3, h0=True, gate=True))
    g = np.random.default_rng(4)
    dout = g.standard_normal(ins[0].shape)
    dl = g.standard_normal((1, 2, 3))

    def loss(v):
        out, _, last = R.selective_scan_fwd(*v[:6], method, v[6], v[7])
        return float((out * dout).sum() + (last * dl).sum())

    grads = R.selective_scan_bwd(*ins[:5], dout, ins[5], method, ins[6], ins[7], dl)
    names = ["dx", "ddelta", "dA", "dB", "dC", "dh0", "dD", "dz"]
    eps = 1e-6
    for k, name in enumerate(names):
        num = np.zeros_like(ins[k])
        for idx in np.ndindex(ins[k].shape):
            p = [v.copy() if v is not None else None for v in ins]
            m = [v.copy() if v is not None else None for v in ins]
            p[k][idx] += eps
            m[k][idx] -= eps
            num[idx] = (loss(p) - loss(m)) / (2 * eps)
        np.testing.assert_allclose(grads[name], num, rtol=1e-6, atol=1e-7, err_msg=name)


# --------------------------------------------------------------------------- decode step, conv

@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
def test_decode_steps_equal_full_forward(method):
    x, delta, A, Bm, Cm, hz, Dv, z = sel_inputs(B=2, L=12, D=3, N=4, seed=9)
    out, _, last = R.selective_scan_fwd(x, delta, A, Bm, Cm, hz, method, Dv, z)
    h = hz.copy()
    for t in range(12):
        o, h = R.ssm_step(h, x[:, t], delta[:, t], A, Bm[:, t], Cm[:, t], method, Dv, z[:, t])
        np.testing.assert_allclose(o, out[:, t], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(h, last, rtol=1e-12)


def test_conv1d_matches_torch_and_streams():
    g = np.random.default_rng(6)
    x = g.standard_normal((2, 5, 17))
    w = g.standard_normal((5, 4))
    bias = g.standard_normal(5)
    y, _ = R.conv1d_causal(x, w, bias)
    ref = torch.nn.functional.conv1d(torch.nn.functional.pad(torch.tensor(x), (3, 0)),
                                     torch.tensor(w)[:, None, :], torch.tensor(bias), groups=5)
    np.testing.assert_allclose(y, torch.nn.functional.silu(ref).numpy(), rtol=1e-12, atol=1e-13)
    y1, st = R.conv1d_causal(x[..., :9], w, bias)
    y2, _ = R.conv1d_causal(x[..., 9:], w, bias, state=st)
    np.testing.assert_allclose(np.concatenate([y1, y2], -1), y, rtol=1e-12, atol=1e-13)


# --------------------------------------------------------------------------- C oracle

@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
@pytest.mark.parametrize("h0,gate", [(False, False), (True, True)])
def test_c_oracle_matches_numpy_oracle(method, h0, gate):
    ins = sel_inputs(B=3, L=40, D=7, N=6, seed=21, h0=h0, gate=gate)
    g = np.random.default_rng(22)
    dout = g.standard_normal(ins[0].shape)
    dl = g.standard_normal((3, 7, 6))
    o1, y1, l1 = R.selective_scan_fwd(*ins[:6], method, ins[6], ins[7])
    o2, y2, l2 = c_oracle.fwd(*ins[:6], method, ins[6], ins[7])
    for a, b in ((o1, o2), (y1, y2), (l1, l2)):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-13)
    g1 = R.selective_scan_bwd(*ins[:5], dout, ins[5], method, ins[6], ins[7], dl)
    g2 = c_oracle.bwd(*ins[:5], dout, ins[5], method, ins[6], ins[7], dl)
    assert set(g1) == set(g2)
    for k in g1:
        np.testing.assert_allclose(g2[k], g1[k], rtol=1e-11, atol=1e-12, err_msg=k)


@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
def test_term_magnitudes_bound_values_and_add_over_rows(method):
    """The term magnitudes that scale the float32 cancellation bound of the GPU tests:
    the ddelta, dA, dB and dC magnitudes equal the C oracle's (its own scalar loop), every magnitude bounds its value,
    an element of one term has magnitude |value|, and dA_mag adds over batch rows (so it is a
    sum of |terms|, not |sum|)."""
    ins = sel_inputs(B=3, L=40, D=7, N=6, seed=23, h0=True, gate=True)
    g = np.random.default_rng(24)
    dout, dl = g.standard_normal(ins[0].shape), g.standard_normal((3, 7, 6))
    gm = R.selective_scan_bwd(*ins[:5], dout, ins[5], method, ins[6], ins[7], dl, mag=True)
    gc = c_oracle.bwd(*ins[:5], dout, ins[5], method, ins[6], ins[7], dl, mag=True)
    np.testing.assert_allclose(gm["ddelta_mag"], gc["ddelta_mag"], rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(gm["dA_mag"], gc["dA_mag"], rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(gm["dB_mag"], gc["dB_mag"], rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(gm["dC_mag"], gc["dC_mag"], rtol=1e-11, atol=1e-12)
    for k in ("ddelta", "dA", "dB", "dC"):
        assert np.all(gm[k + "_mag"] >= np.abs(gm[k]) * (1 - 1e-12)), k
        assert np.any(gm[k + "_mag"] > 1.5 * np.abs(gm[k])), k   # terms do cancel here
    x, delta, A, Bm, Cm, hz, Dv, z = ins
    rows = [R.selective_scan_bwd(x[b:b + 1], delta[b:b + 1], A, Bm[b:b + 1], Cm[b:b + 1], dout[b:b + 1],
                                 hz[b:b + 1], method, Dv, z[b:b + 1], dl[b:b + 1], mag=True) for b in range(3)]
    np.testing.assert_allclose(sum(r["dA_mag"] for r in rows), gm["dA_mag"], rtol=1e-12)
    one = sel_inputs(B=1, L=1, D=5, N=1, seed=25, h0=True, gate=False)
    g1 = R.selective_scan_bwd(*one[:5], g.standard_normal((1, 1, 5)), one[5], method, one[6], one[7],
                              g.standard_normal((1, 5, 1)), mag=True)
    for k in ("ddelta", "dA"):
        np.testing.assert_allclose(g1[k + "_mag"], np.abs(g1[k]), rtol=1e-14, err_msg=k)


# --------------------------------------------------------------------------- scan / discretize VJPs

@pytest.mark.parametrize("with_h0", [False, True])
def test_scan_vjp_matches_torch_autograd(with_h0):
    a, b = rand_ab(B=2, L=13, D=2, N=3, seed=5)
    g = np.random.default_rng(6)
    h0 = g.standard_normal((2, 2, 3)) if with_h0 else None
    dh = g.standard_normal(b.shape)
    h = R.scan_sequential(a, b, h0)
    da, db, dh0 = R.scan_vjp(a, h0, h, dh)
    ta, tb = torch.tensor(a, requires_grad=True), torch.tensor(b, requires_grad=True)
    th0 = torch.tensor(h0, requires_grad=True) if with_h0 else None
    hh = torch.zeros_like(tb[:, 0]) if th0 is None else th0
    outs = []
    for t in range(a.shape[1]):
        hh = ta[:, t] * hh + tb[:, t]
        outs.append(hh)
    (torch.stack(outs, 1) * torch.tensor(dh)).sum().backward()
    np.testing.assert_allclose(da, ta.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-12, atol=1e-12)
    if with_h0:
        np.testing.assert_allclose(dh0, th0.grad.numpy(), rtol=1e-12, atol=1e-12)
    else:
        assert dh0 is None


@pytest.mark.parametrize("method", R.DISCRETIZATIONS)
@pytest.mark.parametrize("tiny", [False, True])
def test_discretize_vjp_matches_torch_autograd(method, tiny):
    g = np.random.default_rng(9)
    B, L, D, N = 2, 5, 3, 4
    delta = g.random((B, L, D)) * (1e-5 if tiny else 0.8) + (1e-6 if tiny else 0.01)
    A = -g.random((D, N)) * 3 - 0.1
    Bm, x = g.standard_normal((B, L, N)), g.standard_normal((B, L, D))
    ga, gb = g.standard_normal((B, L, D, N)), g.standard_normal((B, L, D, N))
    ours = R.discretize_vjp(delta, A, Bm, x, ga, gb, method)
    tt = [torch.tensor(v, requires_grad=True) for v in (delta, A, Bm, x)]
    dA_ = tt[0].unsqueeze(-1) * tt[1]
    Bx = tt[3].unsqueeze(-1) * tt[2].unsqueeze(2)
    if method == "zoh":
        a, b = torch.exp(dA_), torch.expm1(dA_) / tt[1] * Bx
    elif method == "euler":
        a, b = torch.exp(dA_), tt[0].unsqueeze(-1) * Bx
    else:
        a = (1 + dA_ / 2) / (1 - dA_ / 2)
        b = tt[0].unsqueeze(-1) / (1 - dA_ / 2) * Bx
    ((a * torch.tensor(ga)).sum() + (b * torch.tensor(gb)).sum()).backward()
    for got, t in zip(ours, tt):
        np.testing.assert_allclose(got, t.grad.numpy(), rtol=1e-9, atol=1e-12)


# --------------------------------------------------------------------------- LM restatement

@pytest.mark.parametrize("W", [4, 2, 1])
def test_lm_ref_layer_composes_pinned_oracle_pieces(W):
    """oracle/lm_ref.mamba_layer equals in_proj -> conv1d_causal -> selective_scan_fwd (D skip,
    SiLU gate) -> out_proj built from the pinned numpy oracle; its decode path (state carried
    one token at a time) equals its full-sequence path, also at conv width 1 (an empty conv
    state that stays empty)."""
    from oracle import lm_ref
    g = torch.Generator().manual_seed(0)
    dm, D, N, R_ = 8, 16, 4, 2
    p = {"m.in_proj.weight": torch.randn(2 * D, dm, generator=g, dtype=torch.float64) * 0.3,
         "m.conv.weight": torch.randn(D, 1, W, generator=g, dtype=torch.float64) * 0.5,
         "m.conv.bias": torch.randn(D, generator=g, dtype=torch.float64) * 0.1,
         "m.x_proj.weight": torch.randn(R_ + 2 * N, D, generator=g, dtype=torch.float64) * 0.3,
         "m.dt_proj.weight": torch.randn(D, R_, generator=g, dtype=torch.float64) * 0.3,
         "m.dt_proj.bias": torch.randn(D, generator=g, dtype=torch.float64) * 0.3 - 2.0,
         "m.A_log": torch.log(torch.arange(1, N + 1, dtype=torch.float64).repeat(D, 1)),
         "m.D": torch.randn(D, generator=g, dtype=torch.float64),
         "m.out_proj.weight": torch.randn(dm, D, generator=g, dtype=torch.float64) * 0.3}
    u = torch.randn(2, 11, dm, generator=g, dtype=torch.float64)
    out = lm_ref.mamba_layer(p, "m.", u, N, R_, W)
    # the same layer from the numpy oracle pieces
    xz = u.numpy() @ p["m.in_proj.weight"].numpy().T
    x, z = xz[..., :D], xz[..., D:]
    xc, _ = R.conv1d_causal(x.transpose(0, 2, 1), p["m.conv.weight"].numpy()[:, 0], p["m.conv.bias"].numpy())
    xc = xc.transpose(0, 2, 1)
    proj = xc @ p["m.x_proj.weight"].numpy().T
    dt, Bm, Cm = proj[..., :R_], proj[..., R_:R_ + N], proj[..., R_ + N:]
    delta = np.log1p(np.exp(dt @ p["m.dt_proj.weight"].numpy().T + p["m.dt_proj.bias"].numpy()))
    A = -np.exp(p["m.A_log"].numpy())
    o, _, _ = R.selective_scan_fwd(xc, delta, A, Bm, Cm, None, "zoh", p["m.D"].numpy(), z)
    ref = o @ p["m.out_proj.weight"].numpy().T
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-11, atol=1e-12)
    state = {"conv": torch.zeros(2, D, W - 1, dtype=torch.float64), "ssm": torch.zeros(2, D, N, dtype=torch.float64)}
    steps = torch.cat([lm_ref.mamba_layer(p, "m.", u[:, t:t + 1], N, R_, W, state=state) for t in range(11)], 1)
    np.testing.assert_allclose(steps.numpy(), out.numpy(), rtol=1e-11, atol=1e-12)
    assert state["conv"].shape == (2, D, W - 1)


@pytest.mark.parametrize("shape,eps", [((3, 7, 256), 1e-5), ((2, 5, 1000), 1e-6), ((4, 1), 1e-5), ((6, 64), 1e-3)])
def test_lm_ref_rmsnorm_matches_torch_rms_norm(shape, eps):
    """oracle/lm_ref.rmsnorm (models/common.py:14-16) against torch.nn.functional.rms_norm, an
    independent library implementation of the same normalisation, in float64."""
    from oracle import lm_ref
    g = torch.Generator().manual_seed(shape[-1])
    x = torch.randn(shape, generator=g, dtype=torch.float64) * 3.0
    w = 1.0 + 0.5 * torch.randn(shape[-1], generator=g, dtype=torch.float64)
    ref = torch.nn.functional.rms_norm(x, (shape[-1],), w, eps)
    torch.testing.assert_close(lm_ref.rmsnorm(x, w, eps), ref, rtol=1e-13, atol=1e-13)
    # a plausible slip (eps outside the root, or a sum instead of the mean) fails this check
    assert not torch.allclose(x / (x.pow(2).mean(-1, keepdim=True).sqrt() + eps) * w, ref, rtol=1e-13, atol=0) or eps < 1e-12


@pytest.mark.parametrize("ragged", [False, True])
def test_cpu_baseline_restatement_matches_oracle(monkeypatch, ragged):
    """oracle/cpu_chunked (the torch-CPU restatement timed as bench.py's cpu_baseline) against
    the numpy oracle in float64: the output (y + D x) * silu(z) and all seven gradients of one
    fwd + bwd, to 1e-10.  Channel tiles of 3 (d_block forced below D, models/scan.py:185-190)
    and, ragged, a length that is not a multiple of the chunk (padding of scan_chunked)."""
    from oracle import cpu_chunked
    monkeypatch.setattr(cpu_chunked, "_blocks", lambda B, L, D, N: [(i, min(i + 3, D)) for i in range(0, D, 3)])
    B, L, D, N = 2, 37 if ragged else 32, 8, 4
    g = torch.Generator().manual_seed(71)
    x = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    delta = torch.rand(B, L, D, generator=g, dtype=torch.float64) * 0.3 + 1e-3
    A = -torch.rand(D, N, generator=g, dtype=torch.float64) * 4 - 0.05
    Bm, Cm = (torch.randn(B, L, N, generator=g, dtype=torch.float64) for _ in range(2))
    Dv = torch.randn(D, generator=g, dtype=torch.float64)
    z, dy = (torch.randn(B, L, D, generator=g, dtype=torch.float64) for _ in range(2))
    f = [t.numpy() for t in (x, delta, A, Bm, Cm)]
    out, y, _ = R.selective_scan_fwd(*f, None, "zoh", Dv.numpy(), z.numpy())
    np.testing.assert_allclose(cpu_chunked.fwd(x, delta, A, Bm, Cm).numpy(), y, rtol=1e-10, atol=1e-12)
    ref = R.selective_scan_bwd(*f, dy.numpy(), None, "zoh", Dv.numpy(), z.numpy())
    got = cpu_chunked.fwd_bwd(x, delta, A, Bm, Cm, Dv, z, dy)
    for name, gv in zip(("dx", "ddelta", "dA", "dB", "dC", "dD", "dz"), got):
        np.testing.assert_allclose(gv.numpy(), ref[name], rtol=1e-10, atol=1e-12, err_msg=name)
    # a planted slip (a dropped D skip in the restatement's output) is caught by this check
    bad = (torch.from_numpy(y) * torch.nn.functional.silu(z)).numpy()
    assert not np.allclose(bad, out, rtol=1e-10, atol=1e-12)
