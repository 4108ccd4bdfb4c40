"""The fused forward's whole-chunk iterations against the float64 oracle.

With a uniform layout, N equal to the padded state count and every channel of a wavefront real
(D a multiple of the workgroup's channels), the forward runs the chunks that lie wholly inside
the sequence through a copy of its loop body without range selects, and the rest (a segment's
first iteration, the ragged last chunk, the pipeline's drain) through the ranged body.  These
shapes put both kinds in one launch: ragged sequence ends, time segments whose first chunk is
odd or even, 32 states, 16-bit inputs, a channel-major (B, D, L) storage, and the low-rank
delta projection -- every output and gradient at the bar of the path's dtype, with the
cancellation rule of tests/parity.py for ddelta and dA (up to 2 elements per tensor within
float32 resolution of the sum of their terms' magnitudes).
"""

import pytest
import torch

from ssm_inputs import triton_test_inputs
from parity import close_or_cancelled
from test_gpu_fused import ATOL, ATOL_BF16, RTOL, RTOL_BF16, close, oracle
from test_gpu_long import run_seg

pytestmark = pytest.mark.gpu


def check(got, ref, rtol=RTOL, atol=ATOL):
    out, last, grads = got
    rout, rlast, rg = ref
    close(out, rout, rtol, atol, "out")
    close(last, rlast, rtol, atol, "last")
    for k, v in grads.items():
        if k in ("ddelta", "dA"):
            close_or_cancelled(v, rg[k], rg[k + "_mag"], k, allow=2, rtol=rtol, atol=atol)
        else:
            close(v, rg[k], rtol, atol, k)


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
@pytest.mark.parametrize("segments", [1, 3, 13])
def test_whole_chunks_with_ragged_end_and_segments(dev, method, segments):
    """B2 L1000 D48 N16: 62 whole chunks and a ragged one of 8 steps, unsegmented and in 3 and 13
    time segments (segments of 21 and 5 chunks: first chunks of both parities), with the gate,
    D skip, delta bias + softplus, h0 and a gradient on the last state."""
    B, L, D, N = 2, 1000, 48, 16
    ins = triton_test_inputs(B, L, D, N, True, seed=301)
    g = torch.Generator().manual_seed(302)
    Dv, z = torch.randn(D, generator=g), torch.randn(B, L, D, generator=g)
    bias = torch.randn(D, generator=g) * 0.5 - 1.0
    dout, dlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    got = run_seg(ins, dev, method, segments, D=Dv, z=z, bias=bias, softplus=True, dout=dout, dlast=dlast)
    ref = oracle(ins, method, D=Dv, z=z, bias=bias, softplus=True, dout=dout, dlast=dlast, mag=True)
    check(got, ref)


def test_whole_chunks_with_32_states(dev):
    """N = 32 (two channels per wavefront), L = 200 (12 whole chunks and 8 steps)."""
    B, L, D, N = 1, 200, 32, 32
    ins = triton_test_inputs(B, L, D, N, True, seed=311)
    g = torch.Generator().manual_seed(312)
    dout, dlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    got = run_seg(ins, dev, "zoh", 0, dout=dout, dlast=dlast)
    check(got, oracle(ins, "zoh", dout=dout, dlast=dlast, mag=True))


def test_whole_chunks_bf16(dev):
    """bf16 x, delta, B, C, z and dout at B2 L260 D64 N16, against the oracle on the rounded
    inputs at the bf16 bar."""
    B, L, D, N = 2, 260, 64, 16
    x, delta, A, Bm, Cm, h0 = triton_test_inputs(B, L, D, N, True, seed=321)
    g = torch.Generator().manual_seed(322)
    bf = torch.bfloat16
    z = torch.randn(B, L, D, generator=g).to(bf)
    Dv = torch.randn(D, generator=g)
    dout = torch.randn(B, L, D, generator=g).to(bf)
    ins = (x.to(bf), delta.to(bf), A, Bm.to(bf), Cm.to(bf), h0)
    got = run_seg(ins, dev, "zoh", 2, D=Dv, z=z, dout=dout)
    check(got, oracle(ins, "zoh", D=Dv, z=z, dout=dout, mag=True), rtol=RTOL_BF16, atol=ATOL_BF16)


def test_whole_chunks_channel_major(dev):
    """x, delta, z and dout as transposed views of (B, D, L) storage (the conv output's layout,
    models/mamba.py:101-107): a uniform layout with unit stride along time."""
    B, L, D, N = 2, 200, 32, 16
    x, delta, A, Bm, Cm, h0 = triton_test_inputs(B, L, D, N, True, seed=331)
    g = torch.Generator().manual_seed(332)
    z = torch.randn(B, L, D, generator=g)
    dout = torch.randn(B, L, D, generator=g)

    def cm(t):  # the same values in (B, D, L) storage, seen as (B, L, D)
        return t.transpose(1, 2).contiguous().transpose(1, 2)

    ins_cm = (cm(x), cm(delta), A, Bm, Cm, h0)
    assert ins_cm[0].stride() == (L * D, 1, L)
    got = run_seg(ins_cm, dev, "zoh", 0, z=cm(z), dout=dout)
    check(got, oracle((x, delta, A, Bm, Cm, h0), "zoh", z=z, dout=dout, mag=True))


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
def test_whole_chunks_low_rank_delta(dev, method):
    """The low-rank delta path (dt_proj applied while staging; dt, B and C as split views of an
    x_proj-like output) with whole chunks, a ragged end and 3 time segments: B2 L100 D48 N16,
    rank 16, every output and gradient against the float64 oracle at the bar."""
    from test_gpu_lowrank import make, oracle as lr_oracle, run as lr_run
    B, L, D, N, Rk = 2, 100, 48, 16, 16
    ins = make(B, L, D, N, Rk, seed=341)
    out, last, grads = lr_run(dev, *ins, Rk, N, method, segments=3)
    rout, rlast, rg = lr_oracle(*ins, Rk, N, method)
    close(out, rout, name="out")
    close(last, rlast, name="last")
    for k, v in grads.items():
        close(v, rg[k], name=k)
