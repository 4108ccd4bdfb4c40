"""Seeded random configurations of the fused scan (forward + every gradient) against the
float64 oracle: shapes, methods, optional operands and storage layouts drawn together, so
combinations that the targeted tests do not list are still covered.

Each case prints its configuration before running (it names the case if it fails).
Tolerances as the fused tests: rtol 1e-4 / atol 1e-5 on every element, float32 (tests/parity.py).
"""

import numpy as np
import pytest
import torch

import ssm_scan
from oracle import scan_ref as R
from ssm_inputs import np64
import parity

pytestmark = pytest.mark.gpu

METHODS = ("zoh", "euler", "bilinear")


def close(got, ref, name):
    parity.close(got, ref, name=name)   # rtol 1e-4 / atol 1e-5 on every element


def draw(seed):
    rng = np.random.default_rng(seed)
    cfg = dict(B=int(rng.integers(1, 4)), L=int(rng.choice([1, 2, 15, 16, 17, 63, 200, 333])),
               D=int(rng.integers(1, 71)), N=int(rng.choice([1, 2, 5, 8, 16, 24, 32, 64])),
               method=METHODS[int(rng.integers(0, 3))], gate=bool(rng.integers(0, 2)),
               skip=bool(rng.integers(0, 2)), softplus=bool(rng.integers(0, 2)), h0=bool(rng.integers(0, 2)),
               dlast=bool(rng.integers(0, 2)), channel_major=bool(rng.integers(0, 2)),
               bc_split=bool(rng.integers(0, 2)))
    return cfg


def build(cfg, seed):
    g = torch.Generator().manual_seed(seed)
    B, L, D, N = cfg["B"], cfg["L"], cfg["D"], cfg["N"]
    x = torch.randn(B, L, D, generator=g)
    if cfg["softplus"]:
        delta = torch.randn(B, L, D, generator=g) * 0.5 - 1.0
        bias = torch.randn(D, generator=g) * 0.5 - 2.0
    else:
        delta = torch.rand(B, L, D, generator=g) * 0.3 + 1e-3
        bias = None
    A = -(torch.rand(D, N, generator=g) * 4 + 0.05)
    proj = torch.randn(B, L, 3 + 2 * N, generator=g)
    Dv = torch.randn(D, generator=g) if cfg["skip"] else None
    z = torch.randn(B, L, D, generator=g) if cfg["gate"] else None
    h0 = torch.randn(B, D, N, generator=g) if cfg["h0"] else None
    dout = torch.randn(B, L, D, generator=g)
    dlast = torch.randn(B, D, N, generator=g) if cfg["dlast"] else None
    return x, delta, A, proj, Dv, z, bias, h0, dout, dlast


def oracle(x, delta, A, proj, Dv, z, bias, h0, dout, dlast, N, method, softplus, mag=False):
    x, delta, A, proj = np64(x), np64(delta), np64(A), np64(proj)
    Bm, Cm = proj[..., 3:3 + N], proj[..., 3 + N:]
    raw = delta + (np64(bias) if bias is not None else 0.0)
    d_eff = np.log1p(np.exp(raw)) if softplus else raw
    D_, z_, h0_ = (None if t is None else np64(t) for t in (Dv, z, h0))
    out, _, last = R.selective_scan_fwd(x, d_eff, A, Bm, Cm, h0_, method, D_, z_)
    gr = R.selective_scan_bwd(x, d_eff, A, Bm, Cm, np64(dout), h0_, method, D_, z_,
                              None if dlast is None else np64(dlast), mag=mag)
    if softplus:
        gr["ddelta"] = gr["ddelta"] / (1.0 + np.exp(-raw))
        if mag:
            gr["ddelta_mag"] = gr["ddelta_mag"] / (1.0 + np.exp(-raw))
    if bias is not None:
        gr["ddelta_bias"] = gr["ddelta"].sum(axis=(0, 1))
    return out, last, gr


@pytest.mark.parametrize("seed", [s for s in range(25) if s != 13])
def test_random_configuration_matches_oracle(dev, seed):
    run_case(dev, seed)


# Seeds of a 400-configuration sweep of draw() where one or two elements of dA
# (summed over batch and time) or of ddelta (summed over the states) sit outside the bar:
# small values left by terms whose magnitudes add up to 24-304, an error of 0.2-1.6e-6 of
# that magnitude.  Every other gradient element of these cases is held to the bar.
CANCELLING_SEEDS = (13, 74, 82, 153, 159, 208, 229, 249, 360)


@pytest.mark.parametrize("seed", CANCELLING_SEEDS)
def test_random_configuration_cancellation_within_float32_resolution(dev, seed):
    """dA and ddelta elements outside the bar are within float32 resolution (2^-16) of the sum
    of their terms' magnitudes, at most 2 per tensor; all else at the bar."""
    run_case(dev, seed, cancel_allow=2)


# A wider sweep, 2,000 draws (seeds 2000-3999): 17 draws with one or two such elements and one,
# seed 3086 (N = 64, bilinear, B2 L333: 64-term state sums), with four ddelta elements at
# 0.07-0.37e-6 of their terms' magnitudes (100-200); none outside the rule otherwise.
WIDE_SWEEP_CANCELLING = tuple((s, 2) for s in (2008, 2077, 2215, 2555, 2572, 2724, 2752, 2798, 2812, 2897, 3045,
                                              3556, 3562, 3599, 3769, 3926, 3961)) + ((3086, 4),)


@pytest.mark.parametrize("seed,allow", WIDE_SWEEP_CANCELLING)
def test_random_configuration_wide_sweep_cancellation(dev, seed, allow):
    """The wide sweep's draws that need the cancellation rule, each at its own count."""
    run_case(dev, seed, cancel_allow=allow)


def run_case(dev, seed, cancel_allow=None):
    cfg = draw(seed)
    print(f"case seed={seed} {cfg}", flush=True)
    x, delta, A, proj, Dv, z, bias, h0, dout, dlast = build(cfg, 1000 + seed)
    N = cfg["N"]

    def to_dev(t):
        if t is None:
            return None
        t = t.to(dev)
        if cfg["channel_major"] and t.dim() == 3 and t.shape[-1] == cfg["D"]:
            t = t.transpose(1, 2).contiguous().transpose(1, 2)   # (B, D, L) storage
        return t.requires_grad_()

    leaves = [to_dev(t) for t in (x, delta, A, proj, Dv, z, bias, h0)]
    xg, dg, Ag, pg, Dg, zg, bg, hg = leaves
    if cfg["bc_split"]:
        Bm, Cm = pg[..., 3:3 + N], pg[..., 3 + N:]          # strided views of an x_proj-like output
    else:
        Bm, Cm = pg[..., 3:3 + N].contiguous(), pg[..., 3 + N:].contiguous()
    out, last = ssm_scan.selective_scan_fn(xg, dg, Ag, Bm, Cm, D=Dg, z=zg, delta_bias=bg,
                                           delta_softplus=cfg["softplus"], h0=hg, method=cfg["method"],
                                           return_last_state=True)
    loss = (out * dout.to(dev)).sum()
    if dlast is not None:
        loss = loss + (last * dlast.to(dev)).sum()
    loss.backward()
    rout, rlast, rg = oracle(x, delta, A, proj, Dv, z, bias, h0, dout, dlast, N, cfg["method"], cfg["softplus"],
                             mag=cancel_allow is not None)
    close(out, rout, "out")
    close(last, rlast, "last")
    close(xg.grad, rg["dx"], "dx")
    if cancel_allow is None:
        close(dg.grad, rg["ddelta"], "ddelta")
        close(Ag.grad, rg["dA"], "dA")
    else:
        parity.close_or_cancelled(dg.grad, rg["ddelta"], rg["ddelta_mag"], "ddelta", allow=cancel_allow)
        parity.close_or_cancelled(Ag.grad, rg["dA"], rg["dA_mag"], "dA", allow=cancel_allow)
    close(pg.grad[..., 3:3 + N], rg["dB"], "dB")
    close(pg.grad[..., 3 + N:], rg["dC"], "dC")
    assert float(pg.grad[..., :3].abs().max()) == 0.0
    if Dg is not None:
        close(Dg.grad, rg["dD"], "dD")
    if zg is not None:
        close(zg.grad, rg["dz"], "dz")
    if bg is not None:
        close(bg.grad, rg["ddelta_bias"], "ddelta_bias")
    if hg is not None:
        close(hg.grad, rg["dh0"], "dh0")


@pytest.mark.parametrize("seed", range(12))
def test_random_lowrank_configuration_matches_oracle(dev, seed):
    """The dt_proj projection fused into delta staging (delta_proj, rank 1..16, dstate <= 16):
    random shapes, methods, gate/skip/h0 and layouts; every gradient including d(dt) and dW."""
    run_lowrank(dev, seed)


# A 1,000-draw sweep of the low-rank draws (seeds 100-1099) found 3 with one element of dA (a sum
# over batch and time) or dW (a sum over the tokens) outside the bar, all bilinear at L = 257:
# errors of 1.6e-8 - 4.1e-7 of their terms' magnitudes.  Seed 320 was a fourth under an earlier
# time-segment plan (another order of the segment sums) and stays here as a check at the rule.
LOWRANK_CANCELLING = (268, 320, 780, 1094)


@pytest.mark.parametrize("seed", LOWRANK_CANCELLING)
def test_random_lowrank_cancellation_within_float32_resolution(dev, seed):
    """dA and dW elements outside the bar lie within float32 resolution (2^-16) of the sum of
    their terms' magnitudes, at most 1 per tensor; every other output and gradient at the bar."""
    run_lowrank(dev, seed, cancel_allow=1)


def run_lowrank(dev, seed, cancel_allow=None):
    rng = np.random.default_rng(500 + seed)
    B, L, D = int(rng.integers(1, 4)), int(rng.choice([1, 16, 17, 100, 257])), int(rng.integers(1, 70))
    N, Rk = int(rng.choice([1, 4, 8, 13, 16])), int(rng.integers(1, 17))
    method = METHODS[int(rng.integers(0, 3))]
    gate, skip, h0f, cm = (bool(rng.integers(0, 2)) for _ in range(4))
    print(f"case seed={seed} B={B} L={L} D={D} N={N} R={Rk} {method} gate={gate} skip={skip} "
          f"h0={h0f} channel_major={cm}", flush=True)
    g = torch.Generator().manual_seed(2000 + seed)
    x = torch.randn(B, L, D, generator=g)
    proj = torch.randn(B, L, Rk + 2 * N, generator=g)
    W = torch.randn(D, Rk, generator=g) * (0.5 / Rk ** 0.5)
    A = -(torch.rand(D, N, generator=g) * 4 + 0.05)
    bias = torch.rand(D, generator=g) * 2.0 - 4.0
    Dv = torch.randn(D, generator=g) if skip else None
    z = torch.randn(B, L, D, generator=g) if gate else None
    h0 = torch.randn(B, D, N, generator=g) if h0f else None
    dout = torch.randn(B, L, D, generator=g)

    def to_dev(t):
        if t is None:
            return None
        t = t.to(dev)
        if cm and t.dim() == 3 and t.shape[-1] == D:
            t = t.transpose(1, 2).contiguous().transpose(1, 2)
        return t.requires_grad_()

    xg, pg, Wg, Ag, bg, Dg, zg, hg = (to_dev(t) for t in (x, proj, W, A, bias, Dv, z, h0))
    dt, Bm, Cm = pg[..., :Rk], pg[..., Rk:Rk + N], pg[..., Rk + N:]
    out = ssm_scan.selective_scan_fn(xg, dt, Ag, Bm, Cm, D=Dg, z=zg, delta_bias=bg, delta_softplus=True,
                                     h0=hg, method=method, delta_proj=Wg)
    (out * dout.to(dev)).sum().backward()

    xd, pd, Wd = np64(x), np64(proj), np64(W)
    dtd, Bd, Cd = pd[..., :Rk], pd[..., Rk:Rk + N], pd[..., Rk + N:]
    raw = dtd @ Wd.T + np64(bias)
    d_eff = np.log1p(np.exp(raw))
    D_, z_, h0_ = (None if t is None else np64(t) for t in (Dv, z, h0))
    rout, _, _ = R.selective_scan_fwd(xd, d_eff, np64(A), Bd, Cd, h0_, method, D_, z_)
    gr = R.selective_scan_bwd(xd, d_eff, np64(A), Bd, Cd, np64(dout), h0_, method, D_, z_, None,
                              mag=cancel_allow is not None)
    sig = 1.0 / (1.0 + np.exp(-raw))
    draw_ = gr["ddelta"] * sig
    dW = draw_.reshape(-1, D).T @ dtd.reshape(-1, Rk)
    close(out, rout, "out")
    close(xg.grad, gr["dx"], "dx")
    close(pg.grad, np.concatenate([draw_ @ Wd, gr["dB"], gr["dC"]], -1), "dproj")
    if cancel_allow is None:
        close(Ag.grad, gr["dA"], "dA")
        close(Wg.grad, dW, "dW")
    else:
        # dW's terms are (d raw)_t dt_t over the tokens, each d raw bounded by its own magnitude
        dW_mag = (gr["ddelta_mag"] * sig).reshape(-1, D).T @ np.abs(dtd.reshape(-1, Rk))
        parity.close_or_cancelled(Ag.grad, gr["dA"], gr["dA_mag"], "dA", allow=cancel_allow)
        parity.close_or_cancelled(Wg.grad, dW, dW_mag, "dW", allow=cancel_allow)
    close(bg.grad, draw_.sum(axis=(0, 1)), "dbias")
    if Dg is not None:
        close(Dg.grad, gr["dD"], "dD")
    if zg is not None:
        close(zg.grad, gr["dz"], "dz")
    if hg is not None:
        close(hg.grad, gr["dh0"], "dh0")


# Draws with elements of dA (seeds 12, 16: 2 and 1 elements) or d_bias (seed 48, found by a
# 400-draw sweep of seeds 0-399: 1.75e-8 of its terms' magnitude, a sum over 281 steps) outside
# the bar; every such element of the sweep lay within the cancellation rule.
SEGMENT_CANCELLING = (12, 16, 48)


@pytest.mark.parametrize("seed", [s for s in range(24) if s not in SEGMENT_CANCELLING])
def test_random_forced_segments_match_oracle(dev, seed):
    """Random shapes, methods and options with the sequence forced into 2 .. all-chunk time
    segments (summary passes, carries and segment-local walks in both directions), every output
    and gradient at the bar."""
    run_segments(dev, seed)


@pytest.mark.parametrize("seed", SEGMENT_CANCELLING)
def test_random_forced_segments_cancellation(dev, seed):
    """dA, ddelta and d_bias elements outside the bar lie within float32 resolution (2^-16) of the
    sum of their terms' magnitudes, at most 2 per tensor; all else at the bar."""
    run_segments(dev, seed, cancel_allow=2)


def run_segments(dev, seed, cancel_allow=None):
    from ssm_inputs import triton_test_inputs
    from test_gpu_fused import oracle as fused_oracle
    from test_gpu_long import run_seg
    rng = np.random.default_rng(seed)
    B, L, D = int(rng.integers(1, 3)), int(rng.integers(17, 700)), int(rng.integers(1, 70))
    N = int(rng.choice([1, 4, 16, 24, 32, 64]))
    method = METHODS[int(rng.integers(0, 3))]
    segments = int(rng.integers(2, max(3, (L + 15) // 16 + 1)))
    gate, skip, soft = (bool(rng.integers(0, 2)) for _ in range(3))
    print(f"case seed={seed} B={B} L={L} D={D} N={N} {method} segments={segments} gate={gate} skip={skip} "
          f"softplus={soft}", flush=True)
    ins = triton_test_inputs(B, L, D, N, True, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    Dv = torch.randn(D, generator=g) if skip else None
    z = torch.randn(B, L, D, generator=g) if gate else None
    bias = (torch.randn(D, generator=g) * 0.5 - 1.0) if soft else None
    dout, dlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    out, last, grads = run_seg(ins, dev, method, segments, D=Dv, z=z, bias=bias, softplus=soft, dout=dout, dlast=dlast)
    rout, rlast, rg = fused_oracle(ins, method, D=Dv, z=z, bias=bias, softplus=soft, dout=dout, dlast=dlast,
                                   mag=cancel_allow is not None)
    close(out, rout, "out")
    close(last, rlast, "last")
    mags = {} if cancel_allow is None else {"dA": rg["dA_mag"], "ddelta": rg["ddelta_mag"],
                                            "ddelta_bias": rg["ddelta_mag"].sum(axis=(0, 1))}
    for k, v in grads.items():
        if k in mags:
            parity.close_or_cancelled(v, rg[k], mags[k], k, allow=cancel_allow)
        else:
            close(v, rg[k], k)


@pytest.mark.parametrize("seed", range(24))
def test_random_bf16_configuration_matches_oracle(dev, seed):
    """Random draws (as above) with bf16 x, delta, B, C (an x_proj-like bf16 tensor), z and dout,
    float32 A, D, bias, h0 and state: every output and gradient against the float64 oracle on
    the rounded inputs at the bf16 bar (rtol 2e-2 / atol 1e-5).  A 600-draw sweep (seeds 0-599)
    had no element outside it beyond dA / ddelta within the cancellation rule."""
    cfg = draw(seed)
    print(f"case seed={seed} {cfg}", flush=True)
    x, delta, A, proj, Dv, z, bias, h0, dout, dlast = build(cfg, 1000 + seed)
    N = cfg["N"]
    bf = torch.bfloat16

    def rounded(t):
        return None if t is None else t.to(bf).float()

    x, delta, proj, z, dout = rounded(x), rounded(delta), rounded(proj), rounded(z), rounded(dout)

    def to_dev(t, cast):
        if t is None:
            return None
        t = t.to(dev)
        if cast:
            t = t.to(bf)
        if cfg["channel_major"] and t.dim() == 3 and t.shape[-1] == cfg["D"]:
            t = t.transpose(1, 2).contiguous().transpose(1, 2)
        return t.requires_grad_()

    xg, dg, pg, zg = (to_dev(t, True) for t in (x, delta, proj, z))
    Ag, Dg, bg, hg = (to_dev(t, False) for t in (A, Dv, bias, h0))
    if cfg["bc_split"]:
        Bm, Cm = pg[..., 3:3 + N], pg[..., 3 + N:]
    else:
        Bm, Cm = pg[..., 3:3 + N].contiguous(), pg[..., 3 + N:].contiguous()
    out, last = ssm_scan.selective_scan_fn(xg, dg, Ag, Bm, Cm, D=Dg, z=zg, delta_bias=bg,
                                           delta_softplus=cfg["softplus"], h0=hg, method=cfg["method"],
                                           return_last_state=True)
    loss = (out.float() * dout.to(dev)).sum()
    if dlast is not None:
        loss = loss + (last * dlast.to(dev)).sum()
    loss.backward()
    rout, rlast, rg = oracle(x, delta, A, proj, Dv, z, bias, h0, dout, dlast, N, cfg["method"], cfg["softplus"])

    def c(got, ref, name):
        parity.close(got, ref, parity.RTOL_BF16, parity.ATOL_BF16, name)

    assert out.dtype == bf and xg.grad.dtype == bf and pg.grad.dtype == bf
    c(out, rout, "out")
    c(last, rlast, "last")
    c(xg.grad, rg["dx"], "dx")
    c(dg.grad, rg["ddelta"], "ddelta")
    c(Ag.grad, rg["dA"], "dA")
    c(pg.grad[..., 3:3 + N], rg["dB"], "dB")
    c(pg.grad[..., 3 + N:], rg["dC"], "dC")
    for got, key in ((Dg, "dD"), (zg, "dz"), (bg, "ddelta_bias"), (hg, "dh0")):
        if got is not None:
            c(got.grad, rg[key], key)


def large_draw(seed):
    """Larger shapes (B <= 3, L 512-5000, D 96-1000, N 16-64; at most 60 M elements), automatic
    time segments and channel tiles, every method and option."""
    rng = np.random.default_rng(9000 + seed)
    B = int(rng.integers(1, 4))
    L, D = int(rng.choice([700, 1500, 4096, 5000])), int(rng.choice([96, 256, 512, 1000]))
    N = int(rng.choice([16, 16, 32, 64]))
    method = METHODS[int(rng.integers(0, 3))]
    gate, skip, soft = (bool(rng.integers(0, 2)) for _ in range(3))
    while B * L * D * N > 60_000_000:
        L //= 2
    return B, L, D, N, method, gate, skip, soft


def run_large(dev, seed, use_c, rule=False):
    """One large_draw case against the oracle.  With `rule`, dA, dB, dC, ddelta and ddelta_bias
    (sums that can cancel) are held to the cancellation rule: every element outside the bar within
    float32 resolution of its terms' magnitudes, at most max(8, size / 50,000) of them per tensor."""
    from ssm_inputs import triton_test_inputs
    from test_gpu_fused import GRAD_MAP, oracle as fused_oracle
    from test_gpu_long import run_seg
    B, L, D, N, method, gate, skip, soft = large_draw(seed)
    print(f"case seed={seed} B={B} L={L} D={D} N={N} {method} gate={gate} skip={skip} softplus={soft}", flush=True)
    ins = triton_test_inputs(B, L, D, N, True, seed=seed)
    g = torch.Generator().manual_seed(seed + 5)
    Dv = torch.randn(D, generator=g) if skip else None
    z = torch.randn(B, L, D, generator=g) if gate else None
    bias = (torch.randn(D, generator=g) * 0.5 - 1.0) if soft else None
    dout, dlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    out, last, grads = run_seg(ins, dev, method, None, D=Dv, z=z, bias=bias, softplus=soft, dout=dout, dlast=dlast)
    rout, rlast, rg = fused_oracle(ins, method, D=Dv, z=z, bias=bias, softplus=soft, dout=dout, dlast=dlast,
                                   use_c=use_c, mag=rule)
    close(out, rout, "out")
    close(last, rlast, "last")
    mags = {"dA": rg["dA_mag"], "dB": rg["dB_mag"], "dC": rg["dC_mag"], "ddelta": rg["ddelta_mag"],
            "ddelta_bias": rg["ddelta_mag"].sum(axis=(0, 1))} if rule else {}
    for k, v in grads.items():
        if k in mags:
            parity.close_or_cancelled(v, rg[k], mags[k], k, allow=max(8, v.numel() // 50_000))
        else:
            close(v, rg[GRAD_MAP[k]], k)


# A 40-draw sweep of large_draw (seeds 0-39) against the C oracle: these 10 draws have every
# element of every output and gradient at the bar.  In the other 30 every element outside it is
# a dA, dB, dC, ddelta or ddelta_bias sum within the cancellation rule (1 to 37 per tensor of up to
# 3.75 M elements, at most 3.4e-6 of the terms' magnitudes).  Which draws sit at the bar depends
# on the time-segment plan, which sets the order of the segment sums.
LARGE_AT_BAR = (2, 5, 16, 17, 18, 22, 24, 26, 35, 37)


@pytest.mark.parametrize("seed", LARGE_AT_BAR)
def test_random_large_shapes_match_c_oracle(dev, seed):
    run_large(dev, seed, use_c=True)


@pytest.mark.parametrize("seed", [s for s in range(40) if s not in LARGE_AT_BAR])
def test_random_large_shapes_within_cancellation_rule(dev, seed):
    run_large(dev, seed, use_c=True, rule=True)
