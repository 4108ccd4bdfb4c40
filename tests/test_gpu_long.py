"""Long sequences (time segments in the forward and the backward) against the float64 oracle.

When B x D alone cannot fill the GPU the fused forward splits time into segments (summary
pass, carry over segment summaries, main pass) -- the structure of scan_chunked
(models/scan.py:142-165) lifted to segments.  Checked here:
  * forced segment counts (incl. ragged last segments) at small shapes, forward and the
    backward that consumes the segmented forward's saved chunk states, all methods;
  * the automatic choice at B1 D64 L8192, and forward and backward planned apart (B6 L512
    D512: the forward unsegmented, the backward in 8 segments);
  * BASELINE config 2 at its largest length, B1 L131072 D512 N16, float32 and bf16
    (rtol 1e-4 / atol 1e-5 float32; rtol 2e-2 / atol 1e-5 bf16), against the C fp64 oracle;
  * the backward at B1 L65536 D512 N16 (gate + D skip), walked in time segments, and with bf16
    inputs at B1 L16384;
  * forced segments with 16-bit inputs, and with a strided (non-uniform) layout.
"""

import pytest
import torch

import ssm_scan
from oracle import c_oracle
from ssm_inputs import baseline_inputs, np64, triton_test_inputs
from parity import close_or_cancelled
from test_gpu_fused import ATOL, ATOL_BF16, RTOL, RTOL_BF16, check_all, close, oracle

pytestmark = pytest.mark.gpu


def run_seg(ins, dev, method, segments, D=None, z=None, bias=None, softplus=False, dout=None, dlast=None):
    x, delta, A, Bm, Cm, h0 = ins
    names = ["dx", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias", "dh0"]
    gl = [None if t is None else t.to(dev).requires_grad_() for t in (x, delta, A, Bm, Cm, D, z, bias, h0)]
    out, last = ssm_scan.selective_scan_fn(gl[0], gl[1], gl[2], gl[3], gl[4], D=gl[5], z=gl[6],
                                           delta_bias=gl[7], delta_softplus=softplus, h0=gl[8],
                                           method=method, return_last_state=True, segments=segments)
    loss = (out * dout.to(dev)).sum()
    if dlast is not None:
        loss = loss + (last * dlast.to(dev)).sum()
    loss.backward()
    return out.detach(), last.detach(), {n: t.grad for n, t in zip(names, gl) if t is not None}


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
@pytest.mark.parametrize("segments", [2, 3, 5])
def test_forced_segments_match_oracle(dev, method, segments):
    B, L, D, N = 2, 100, 40, 16             # 7 chunks of 16 steps: ragged last segment
    ins = triton_test_inputs(B, L, D, N, True, seed=segments)
    g = torch.Generator().manual_seed(segments + 1)
    dout = torch.randn(B, L, D, generator=g)
    dlast = torch.randn(B, D, N, generator=g)
    got = run_seg(ins, dev, method, segments, dout=dout, dlast=dlast)
    ref = oracle(ins, method, dout=dout, dlast=dlast)
    check_all(got, ref)


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
@pytest.mark.parametrize("segments", [1, 9, 13, 21, 63])
def test_forced_segment_counts_past_the_fold(dev, method, segments):
    """B2 L1000 = 63 chunks in 9, 13, 21 and 63 time segments (7, 5, 3 and 1 chunks each), and
    unsegmented (1) on the same draws: past the 8 segments the forward's main pass folds itself,
    so both passes run their carry kernels, which read the segment summaries 16 at a time -- one
    partial group (13), a full group and a partial one (21), three full groups and a partial
    one (63), and 9.  Every output and gradient against the float64 oracle at the bar, except
    that ddelta (a sum over the 16 states) and dA (over batch and time) may hold up to 2
    elements outside it, each within float32 resolution of the sum of its terms' magnitudes
    (the cancellation rule of tests/parity.py)."""
    B, L, D, N = 2, 1000, 40, 16
    ins = triton_test_inputs(B, L, D, N, True, seed=113)     # one draw for every segment count
    g = torch.Generator().manual_seed(213)
    dout = torch.randn(B, L, D, generator=g)
    dlast = torch.randn(B, D, N, generator=g)
    out, last, grads = run_seg(ins, dev, method, segments, dout=dout, dlast=dlast)
    rout, rlast, rg = oracle(ins, method, dout=dout, dlast=dlast, mag=True)
    close(out, rout, name="out")
    close(last, rlast, name="last")
    for k, v in grads.items():
        if k == "ddelta":
            close_or_cancelled(v, rg[k], rg["ddelta_mag"], k, allow=2)
        elif k == "dA":
            close_or_cancelled(v, rg[k], rg["dA_mag"], k, allow=2)
        else:
            close(v, rg[k], name=k)


def test_forced_segments_with_gate_bias_softplus(dev):
    B, L, D, N = 2, 150, 24, 8
    ins = triton_test_inputs(B, L, D, N, True, seed=21)
    g = torch.Generator().manual_seed(22)
    Dv, z = torch.randn(D, generator=g), torch.randn(B, L, D, generator=g)
    bias = torch.randn(D, generator=g) * 0.5 - 3.0
    ins = (ins[0], torch.randn(B, L, D, generator=g) * 0.5, *ins[2:])
    dout = torch.randn(B, L, D, generator=g)
    got = run_seg(ins, dev, "zoh", 4, D=Dv, z=z, bias=bias, softplus=True, dout=dout)
    ref = oracle(ins, "zoh", D=Dv, z=z, bias=bias, softplus=True, dout=dout)
    check_all(got, ref)


def test_automatic_segments_long_sequence(dev):
    t = baseline_inputs(1, 8192, 64, 16)
    ins = [t[k].to(dev) for k in ("u", "delta", "A", "Bm", "Cm")]
    h0 = torch.randn(1, 64, 16, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        y, last = ssm_scan.selective_scan_hip(*ins, h0=h0.to(dev))
    ry, _, rlast = c_oracle.fwd(*(np64(v) for v in ins), np64(h0))
    close(y, ry, name="y")
    close(last, rlast, name="last")


def test_forward_and_backward_plan_their_segments_apart(dev):
    """B6 L512 D512 N16 with the gate and D skip: 768 wavefronts, so the automatic plan runs
    the forward in one segment and the backward in 8 (it restarts from the forward's saved
    chunk states, which do not depend on the forward's segments).  Every output and gradient
    against the C float64 oracle at the bar; dA, dB, dC and ddelta under the cancellation rule
    (at most 2 elements per tensor, each within float32 resolution of its terms' magnitudes)."""
    t = baseline_inputs(6, 512, 512, 16, gate=True, with_dy=True)
    ins = (t["u"], t["delta"], t["A"], t["Bm"], t["Cm"], None)
    out, last, grads = run_seg(ins, dev, "zoh", None, D=t["D"], z=t["z"], dout=t["dy"])
    rout, rlast, rg = oracle(ins, "zoh", D=t["D"], z=t["z"], dout=t["dy"], use_c=True, mag=True)
    close(out, rout, name="out")
    close(last, rlast, name="last")
    for k, v in grads.items():
        if k in ("dA", "dB", "dC", "ddelta"):
            close_or_cancelled(v, rg[k], rg[k + "_mag"], k, allow=2)
        else:
            close(v, rg[k], name=k)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_longest_forward_matches_c_oracle(dev, dtype):
    """BASELINE config 2 at L = 131072 (B1 D512 N16), forward only."""
    t = baseline_inputs(1, 131072, 512, 16, dtype=dtype)
    ins = [t[k].to(dev) for k in ("u", "delta", "A", "Bm", "Cm")]
    with torch.no_grad():
        y, last = ssm_scan.selective_scan_hip(*ins)
    torch.cuda.synchronize()
    assert y.dtype == dtype and last.dtype == torch.float32
    ry, _, rlast = c_oracle.fwd(*(np64(v) for v in ins))
    rtol, atol = (RTOL, ATOL) if dtype == torch.float32 else (RTOL_BF16, ATOL_BF16)
    close(y, ry, rtol, atol, "y")
    close(last, rlast, rtol, atol, "last")


def test_long_sequence_backward_matches_c_oracle(dev):
    """The reference's long-sequence fwd+bwd benchmark shape (benchmarks/bench_scan.py:35-66:
    B1 D512 N16, here at L = 65536) with the z gate and D skip: one batch row of 512 channels
    leaves the GPU short of work, so both passes walk automatic time segments (the backward from
    the adjoints its summary and carry passes hand them).  Every gradient against the C float64
    oracle; ddelta and dA under the cancellation rule."""
    L = 65536
    t = baseline_inputs(1, L, 512, 16, gate=True, with_dy=True)
    ins = (t["u"], t["delta"], t["A"], t["Bm"], t["Cm"], None)
    got = run_seg(ins, dev, "zoh", 0, D=t["D"], z=t["z"], dout=t["dy"])
    torch.cuda.synchronize()
    ref = oracle(ins, "zoh", D=t["D"], z=t["z"], dout=t["dy"], use_c=True, mag=True)
    out, last, grads = got
    rout, rlast, rg = ref
    close(out, rout, name="out")
    for k, v in grads.items():
        if k not in ("ddelta", "dA"):
            close(v, rg[k], name=k)
    # ddelta_t = sum over the 16 states of float32 terms that can cancel: an element may sit
    # outside the bar only where its error is within float32 resolution (2^-16, a few ulps of
    # each term) of the sum of the terms' magnitudes, and at most 1 ppm of elements may.
    close_or_cancelled(grads["ddelta"], rg["ddelta"], rg["ddelta_mag"], "ddelta",
                       allow=rg["ddelta"].size // 1_000_000)
    # dA = a sum over the 65,536 steps (in segment partials): the same rule, at most 2 of 8,192
    close_or_cancelled(grads["dA"], rg["dA"], rg["dA_mag"], "dA", allow=2)


def test_long_sequence_bf16_backward_matches_c_oracle(dev):
    """bf16 x, delta, B, C, z and dout (A, D and the state float32) at B1 L16384 D512 N16 with the
    gate and D skip: both passes walk automatic time segments.  Outputs and every gradient
    against the C float64 oracle on the bf16-rounded inputs at the bf16 bar (rtol 2e-2 /
    atol 1e-5): the kernels compute in float32, the 16-bit outputs and gradients carry their
    rounding (tests/test_gpu.py:68-77 of the reference trains at this length under bf16)."""
    L = 16384
    t = baseline_inputs(1, L, 512, 16, gate=True, with_dy=True)
    bf = torch.bfloat16
    ins = (t["u"].to(bf), t["delta"].to(bf), t["A"], t["Bm"].to(bf), t["Cm"].to(bf), None)
    z, dout = t["z"].to(bf), t["dy"].to(bf)
    got = run_seg(ins, dev, "zoh", 0, D=t["D"], z=z, dout=dout)
    torch.cuda.synchronize()
    assert got[0].dtype == bf and got[2]["dx"].dtype == bf and got[2]["dA"].dtype == torch.float32
    ref = oracle(ins, "zoh", D=t["D"], z=z, dout=dout, use_c=True)
    check_all(got, ref, rtol=RTOL_BF16, atol=ATOL_BF16)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float16, 4e-3)])
def test_forced_segments_half_precision(dev, dtype, tol):
    """16-bit x, delta, B, C, z with both passes in 4 time segments (gate, D skip, bias +
    softplus, h0 and a gradient on the last state), against the oracle on the rounded inputs at
    the 16-bit rounding of the outputs (as the unsegmented half-precision test)."""
    B, L, D, N = 2, 150, 40, 16
    x, delta, A, Bm, Cm, h0 = triton_test_inputs(B, L, D, N, True, seed=31)
    g = torch.Generator().manual_seed(32)
    Dv, bias = torch.randn(D, generator=g), torch.randn(D, generator=g) * 0.5 - 1.0
    z = torch.randn(B, L, D, generator=g)
    dout = torch.randn(B, L, D, generator=g).to(dtype)
    dlast = torch.randn(B, D, N, generator=g)
    lo = [t.to(dtype) for t in (x, delta, Bm, Cm, z)]
    ins = (lo[0], lo[1], A, lo[2], lo[3], h0)
    got = run_seg(ins, dev, "zoh", 4, D=Dv, z=lo[4], bias=bias, softplus=True, dout=dout, dlast=dlast)
    ref = oracle(ins, "zoh", D=Dv, z=lo[4], bias=bias, softplus=True, dout=dout, dlast=dlast)
    check_all(got, ref, rtol=tol, atol=ATOL)


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
def test_forced_segments_strided_layout(dev, method):
    """x and z as the two halves of one (B, L, 2D) buffer (row stride 2D, the in_proj split of
    models/mamba.py:100) while delta is contiguous: not a uniform layout, so both passes take the
    strided-address path, here in 3 time segments; every output and gradient at the bar."""
    B, L, D, N = 2, 120, 32, 16
    x, delta, A, Bm, Cm, h0 = triton_test_inputs(B, L, D, N, True, seed=41)
    g = torch.Generator().manual_seed(42)
    z = torch.randn(B, L, D, generator=g)
    Dv = torch.randn(D, generator=g)
    dout = torch.randn(B, L, D, generator=g)
    xz = torch.cat([x, z], -1).to(dev).requires_grad_()
    xg, zg = xz[..., :D], xz[..., D:]
    assert xg.stride() == (L * 2 * D, 2 * D, 1)
    leaves = [t.to(dev).requires_grad_() for t in (delta, A, Bm, Cm, Dv, h0)]
    dg, Ag, Bg, Cg, Dg, hg = leaves
    out, last = ssm_scan.selective_scan_fn(xg, dg, Ag, Bg, Cg, D=Dg, z=zg, h0=hg, method=method,
                                           return_last_state=True, segments=3)
    (out * dout.to(dev)).sum().backward()
    rout, rlast, rg = oracle((x, delta, A, Bm, Cm, h0), method, D=Dv, z=z, dout=dout)
    close(out, rout, name="out")
    close(last, rlast, name="last")
    close(xz.grad[..., :D], rg["dx"], name="dx")
    close(xz.grad[..., D:], rg["dz"], name="dz")
    for name, t in zip(("ddelta", "dA", "dB", "dC", "dD", "dh0"), leaves):
        close(t.grad, rg[name], name=name)
