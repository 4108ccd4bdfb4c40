"""ssm_fwd_noalloc: the forward with its long-sequence workspace in the library's fixed device
array instead of a caller buffer.  Called through the C ABI and checked bitwise against
ssm_fwd with a caller workspace (same kernels), and against the float64 C oracle at the float32
bar (rtol 1e-4 / atol 1e-5), on two calls in a row whose second input is smaller (the array
keeps the first call's contents).  The size rejection is host logic and runs on the CPU.
"""

import ctypes

import pytest
import torch

from oracle import c_oracle
from parity import close
from ssm_inputs import np64, triton_test_inputs
from ssm_scan import _abi, hip_scan

SCRATCH_BYTES = 8 * 1024 * 1024   # SSM_FWD_NOALLOC_SCRATCH_BYTES


def _args(x, delta, A, Bm, Cm, D, z, h0, out, last, method, segments):
    a = _abi.FwdArgs()
    hip_scan._fill_common(a, x, delta, A, Bm, Cm, D, z, None, False, h0, method, x.dtype)
    a.out, a.last = _abi.view(out), _abi.view(last)
    a.segments = segments
    return a


def test_noalloc_rejects_a_workspace_beyond_the_scratch():
    """B1 L16384 D512 N16 with 128 segments needs 3 x 128 x 512 x 16 x 4 B = 12 MiB > 8 MiB:
    SSM_ESPACE before any device call; ssm_fwd_workspace_bytes states the size."""
    B, L, D, N = 1, 16384, 512, 16
    x, Bm, A = torch.zeros(B, L, D), torch.zeros(B, L, N), torch.zeros(D, N)
    a = _args(x, x, A, Bm, Bm, None, None, None, x, None, hip_scan.METHODS["zoh"], 128)
    lib = _abi.lib()
    need = lib.ssm_fwd_workspace_bytes(ctypes.byref(a))
    assert need > SCRATCH_BYTES
    rc = lib.ssm_fwd_noalloc(ctypes.byref(a), None)
    assert rc == _abi.ESPACE
    msg = lib.ssm_last_error().decode()
    assert "fixed scratch" in msg and str(need) in msg


CASES = [  # (B, L, D, N, segments, method, gate): the second call is smaller than the first
    (1, 8192, 256, 16, 16, "zoh", True),
    (2, 1000, 64, 16, 5, "bilinear", False),
]


def _case(dev, B, L, D, N, segments, method, gate):
    x, delta, A, Bm, Cm, h0 = triton_test_inputs(B, L, D, N, True, seed=L)
    g = torch.Generator().manual_seed(L + 1)
    Dv = torch.randn(D, generator=g)
    z = torch.randn(B, L, D, generator=g) if gate else None
    host = (x, delta, A, Bm, Cm, Dv, z, h0)
    return host, [None if t is None else t.to(dev) for t in host]


def _call(lib, dev, ins, B, L, D, N, method, segments, entry):
    out = torch.empty(B, L, D, device=dev)
    last = torch.empty(B, D, N, device=dev)
    a = _args(*ins, out, last, hip_scan.METHODS[method], segments)
    need = lib.ssm_fwd_workspace_bytes(ctypes.byref(a))
    assert 0 < need <= SCRATCH_BYTES
    stream = _abi.stream_handle(dev)
    if entry == "ssm_fwd":
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
        _abi.check(lib.ssm_fwd(ctypes.byref(a), stream), entry)
    else:
        # nothing may be allocated: neither by torch's caching allocator nor on the device at all
        torch.cuda.synchronize()
        before, free_before = torch.cuda.memory_allocated(dev), torch.cuda.mem_get_info(dev)[0]
        _abi.check(lib.ssm_fwd_noalloc(ctypes.byref(a), stream), entry)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before
        assert torch.cuda.mem_get_info(dev)[0] == free_before
    torch.cuda.synchronize()
    return out, last


@pytest.mark.gpu
def test_noalloc_forward_equals_ssm_fwd_on_consecutive_calls(dev):
    lib = _abi.lib()
    # warm-up: the first call on a device looks the scratch array's address up, and a kernel's
    # first launch may load its code; the calls measured below are not the first ones
    for B, L, D, N, segments, method, gate in CASES:
        _, ins = _case(dev, B, L, D, N, segments, method, gate)
        _abi.check(lib.ssm_fwd_noalloc(ctypes.byref(_args(*ins, torch.empty(B, L, D, device=dev),
                                                          torch.empty(B, D, N, device=dev),
                                                          hip_scan.METHODS[method], segments)),
                                       _abi.stream_handle(dev)), "warm-up")
        torch.cuda.synchronize()
    for B, L, D, N, segments, method, gate in CASES:
        print(f"case B{B} L{L} D{D} N{N} segments {segments} {method} gate {gate}", flush=True)
        host, ins = _case(dev, B, L, D, N, segments, method, gate)
        o1, l1 = _call(lib, dev, ins, B, L, D, N, method, segments, "ssm_fwd")
        o2, l2 = _call(lib, dev, ins, B, L, D, N, method, segments, "ssm_fwd_noalloc")
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
        x, delta, A, Bm, Cm, Dv, z, h0 = host
        rout, _, rlast = c_oracle.fwd(*(np64(t) for t in (x, delta, A, Bm, Cm, h0)), method=method,
                                      D=np64(Dv), z=np64(z))
        close(o2, rout, name="out")
        close(l2, rlast, name="last")


@pytest.mark.gpu
def test_noalloc_lowers_an_automatic_plan_to_the_scratch(dev):
    """B3 L65536 D512 N16: the automatic plan's 32 segments need 9 MiB of workspace; with
    segments = 0 ssm_fwd_noalloc runs the most that fit 8 MiB, (8 MiB / 3 - 255) // (3 x 512 x
    16 x 4 B) = 28, and equals ssm_fwd forced to 28 segments bitwise (forced counts are
    checked against the oracle elsewhere); no allocation."""
    lib = _abi.lib()
    B, L, D, N = 3, 65536, 512, 16
    print(f"case B{B} L{L} D{D} N{N} automatic segments", flush=True)
    _, ins = _case(dev, B, L, D, N, 0, "zoh", False)
    out = torch.empty(B, L, D, device=dev)
    a = _args(*ins, out, torch.empty(B, D, N, device=dev), hip_scan.METHODS["zoh"], 0)
    assert lib.ssm_fwd_workspace_bytes(ctypes.byref(a)) > SCRATCH_BYTES
    fit = (SCRATCH_BYTES // 3 - 255) // (B * D * N * 4)
    assert fit == 28
    o1, l1 = _call(lib, dev, ins, B, L, D, N, "zoh", fit, "ssm_fwd")
    o2 = torch.empty(B, L, D, device=dev)
    l2 = torch.empty(B, D, N, device=dev)
    torch.cuda.synchronize()
    before, free_before = torch.cuda.memory_allocated(dev), torch.cuda.mem_get_info(dev)[0]
    a = _args(*ins, o2, l2, hip_scan.METHODS["zoh"], 0)
    _abi.check(lib.ssm_fwd_noalloc(ctypes.byref(a), _abi.stream_handle(dev)), "ssm_fwd_noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(dev) == before
    assert torch.cuda.mem_get_info(dev)[0] == free_before
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
