"""CPU-tier checks of the C ABI and the host logic (no device calls).

* libssmscan.so loads and exports every function include/ssm_scan.h declares;
* the ctypes structs have the C layout (compiled with gcc against the header);
* the integer plans equal the oracle's restatement of the reference over exhaustive ranges
  and the committed golden table (bit-exact);
* argument validation returns the reference's error classes.
"""

import ctypes
import json
import os
import random
import re
import subprocess

import pytest
import torch

from oracle import scan_ref as R
from ssm_scan import _abi, hip_scan, plan
import ssm_scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ssm_scan.h")
GOLDEN = os.path.join(ROOT, "tests", "golden", "plans.json")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\s*\*?\s*(ssm_[a-z0-9_]+)\s*\(", src, flags=re.M)))


def test_library_exports_every_declared_function():
    lib = _abi.lib()
    names = header_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_abi.EXPORTED)
    assert lib.ssm_abi_version() == _abi.ABI_VERSION


def test_ctypes_layout_matches_c_header(tmp_path):
    structs = {"ssm_tensor": _abi.Tensor, "ssm_fwd_args": _abi.FwdArgs, "ssm_bwd_args": _abi.BwdArgs,
               "ssm_step_args": _abi.StepArgs, "ssm_decode_args": _abi.DecodeArgs, "ssm_lscan_args": _abi.LscanArgs,
               "ssm_decode_block": _abi.DecodeBlock, "ssm_decode_stack_args": _abi.DecodeStackArgs,
               "ssm_lscan_bwd_args": _abi.LscanBwdArgs,
               "ssm_disc_args": _abi.DiscArgs, "ssm_conv_args": _abi.ConvArgs, "ssm_norm_args": _abi.NormArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    (tmp_path / "l.c").write_text("\n".join(lines))
    subprocess.run(["gcc", str(tmp_path / "l.c"), "-o", str(tmp_path / "l")], check=True)
    out = subprocess.run([str(tmp_path / "l")], check=True, capture_output=True, text=True).stdout
    for line in out.splitlines():
        cname, field, val = line.split()
        py = structs[cname]
        got = ctypes.sizeof(py) if field == "size" else getattr(py, field).offset
        assert got == int(val), line


def test_default_chunk_exact():
    for L in list(range(0, 70000)) + [2 ** k + d for k in range(17, 45) for d in (-1, 0, 1)]:
        assert plan.default_chunk(L) == R.default_chunk(L), L


def test_blocks_block_d_bwd_tile_exact():
    rng = random.Random(0)
    for _ in range(3000):
        B, L, D, N = rng.randint(1, 64), rng.randint(1, 1 << 17), rng.randint(1, 2048), rng.choice([1, 3, 8, 16, 64])
        db = rng.choice([None, 0, 1, 2, 7, 24, 128, 4096])
        assert plan.blocks((B, L, D), N, db) == R.blocks((B, L, D), N, db)
        assert plan.block_d(B, D) == R.block_d(B, D)
        bd = R.block_d(B, D)
        assert plan.bwd_tile(B, L, N, bd) == R.bwd_tile(B, L, N, bd)


def test_resolve_scan_exact():
    for scan in R.SCAN_NAMES:
        for on_gpu in (False, True):
            for method in ("zoh", "euler", "bilinear", "rk4"):
                for N in range(0, 70):
                    for eng in (False, True):
                        assert plan.resolve_scan(scan, on_gpu, method, N, eng) == \
                            R.resolve_scan(scan, on_gpu, method, N, eng)
    with pytest.raises(KeyError):
        plan.resolve_scan("parallel", True, "zoh", 16)


def test_plans_match_committed_golden_table():
    table = json.load(open(GOLDEN))
    for row in table["default_chunk"]:
        assert plan.default_chunk(row[0]) == row[1]
    for row in table["blocks"]:
        assert [list(b) for b in plan.blocks(row[0], row[1], row[2])] == row[3]
    for row in table["block_d"]:
        assert plan.block_d(*row[0]) == row[1]
    for row in table["bwd_tile"]:
        assert plan.bwd_tile(*row[0]) == row[1]
    for row in table["resolve_scan"]:
        assert plan.resolve_scan(*row[0]) == row[1]


def _fwd_args(B=2, L=8, D=4, N=16, method=0, dtype=0, drop=(), empty=False):
    new = torch.empty if empty else torch.zeros
    x = new(B, L, D)
    A = new(D, N)
    Bm = new(B, L, N)
    a = _abi.FwdArgs()
    a.batch, a.seqlen, a.dim, a.dstate, a.method, a.dtype = B, L, D, N, method, dtype
    for name, t in (("x", x), ("delta", x), ("A", A), ("Bm", Bm), ("Cm", Bm), ("out", x)):
        if name not in drop:
            setattr(a, name, _abi.view(t))
    a._keep = (x, A, Bm)
    return a


@pytest.mark.parametrize("kw,exc", [
    (dict(method=3), ValueError), (dict(dtype=7), ValueError), (dict(L=0), ValueError),
    (dict(B=0), ValueError), (dict(N=65), ValueError), (dict(drop=("Cm",)), ValueError),
    (dict(drop=("out",)), ValueError)])
def test_forward_validation_errors(kw, exc):
    a = _fwd_args(**kw)
    rc = _abi.lib().ssm_fwd_check(ctypes.byref(a))
    with pytest.raises(exc):
        _abi.check(rc, "ssm_fwd")


def test_forward_validation_accepts_and_sizes():
    a = _fwd_args(B=16, L=512, D=512, N=16)
    lib = _abi.lib()
    assert lib.ssm_fwd_check(ctypes.byref(a)) == 0
    # chunk-boundary states: B * ceil(L/16) * D * 16 float32
    assert lib.ssm_fwd_saved_bytes(ctypes.byref(a)) == 16 * 32 * 512 * 16 * 4


def _bwd_args(B, L, D, N, segments):
    x = torch.empty(B, L, D)
    A = torch.empty(D, N)
    Bm = torch.empty(B, L, N)
    b = _abi.BwdArgs()
    b.batch, b.seqlen, b.dim, b.dstate, b.segments = B, L, D, N, segments
    for name, t in (("x", x), ("delta", x), ("A", A), ("Bm", Bm), ("Cm", Bm), ("dout", x), ("dx", x),
                    ("ddelta", x), ("dA", A), ("dBm", Bm), ("dCm", Bm)):
        setattr(b, name, _abi.view(t))
    b._keep = (x, A, Bm)
    return b


# (B, L, forward segments, backward segments) chosen automatically at D512 N16 float32 (128
# wavefronts per batch row, 16-step chunks) by the library's cost model of resident rounds on
# 1,024 SIMDs (3 forward / 2 backward wavefronts per SIMD), with walks of at most 128 chunks
# preferred for one to three rows; the counts are the segments the plan actually walks
# (ceil(chunks / ceil(chunks / n))).
AUTO_PLANS = [(1, 512, 8, 8), (2, 512, 8, 8), (4, 512, 4, 4), (6, 512, 1, 8), (8, 512, 1, 2), (12, 512, 1, 1),
              (16, 512, 1, 1), (1, 4096, 16, 16), (1, 16384, 24, 16), (1, 65536, 48, 32), (1, 131072, 72, 64),
              (3, 16384, 8, 16), (5, 8192, 9, 16), (5, 65536, 24, 16), (2, 4096, 8, 8), (8, 4096, 3, 2), (4, 1024, 4, 4)]


@pytest.mark.parametrize("B,L,nf,nb", AUTO_PLANS)
def test_automatic_time_segments(B, L, nf, nb):
    """The automatic plan equals the forced count (workspace sizes depend on the count)."""
    lib = _abi.lib()
    sizes = {}
    other_f, other_b = (nf // 2 if nf > 1 else 2), (nb // 2 if nb > 1 else 2)
    for seg in (0, nf, other_f):
        a = _fwd_args(B=B, L=L, D=512, N=16, empty=True)
        a.segments = seg
        sizes[seg] = lib.ssm_fwd_workspace_bytes(ctypes.byref(a))
    assert sizes[0] == sizes[nf] != sizes[other_f]
    assert (sizes[0] == 0) == (nf == 1)
    sizes = {seg: lib.ssm_bwd_workspace_bytes(ctypes.byref(_bwd_args(B, L, 512, 16, seg))) for seg in (0, nb, other_b)}
    assert sizes[0] == sizes[nb] != sizes[other_b]


def test_backward_requires_gradient_buffers():
    b = _abi.BwdArgs()
    x = torch.zeros(2, 8, 4)
    A = torch.zeros(4, 16)
    Bm = torch.zeros(2, 8, 16)
    b.batch, b.seqlen, b.dim, b.dstate = 2, 8, 4, 16
    for name, t in (("x", x), ("delta", x), ("A", A), ("Bm", Bm), ("Cm", Bm), ("dout", x), ("dx", x),
                    ("ddelta", x), ("dA", A), ("dBm", Bm), ("dCm", Bm)):
        setattr(b, name, _abi.view(t))
    lib = _abi.lib()
    assert lib.ssm_bwd_check(ctypes.byref(b)) == 0
    b.Dskip = _abi.view(torch.zeros(4))
    with pytest.raises(ValueError, match="dD"):
        _abi.check(lib.ssm_bwd_check(ctypes.byref(b)), "ssm_bwd")
    b.dD = _abi.view(torch.zeros(4))
    assert lib.ssm_bwd_check(ctypes.byref(b)) == 0
    assert lib.ssm_bwd_workspace_bytes(ctypes.byref(b)) > 0


def test_python_api_rejects_cpu_tensors_and_bad_arguments():
    x = torch.zeros(1, 4, 8)
    A = -torch.ones(8, 16)
    Bm = torch.zeros(1, 4, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        ssm_scan.selective_scan_hip(x, x, A, Bm, Bm)
    with pytest.raises(ValueError):
        ssm_scan.selective_scan_hip(x, x, A, Bm, Bm, method="rk4")
    with pytest.raises(ValueError, match="power of two"):
        ssm_scan.selective_scan_hip(x, x, -torch.ones(8, 3), Bm[..., :3], Bm[..., :3])


def test_dense_layout_helper():
    t = torch.zeros(2, 5, 7)
    assert hip_scan.is_dense(t) and hip_scan.is_dense(t.transpose(1, 2))
    assert not hip_scan.is_dense(torch.zeros(2, 5, 14)[..., :7])
    assert not hip_scan.is_dense(torch.zeros(7, 1).expand(7, 4))
    out = hip_scan.empty_like_layout(torch.zeros(2, 7, 5).transpose(1, 2), torch.bfloat16)
    assert out.stride() == (35, 1, 5) and out.dtype == torch.bfloat16
    assert hip_scan.empty_like_layout(torch.zeros(2, 5, 14)[..., :7], torch.float32).is_contiguous()


@pytest.mark.parametrize("rank,with_proj,ok", [(0, False, True), (16, True, True), (1, True, True),
                                                (17, True, False), (-1, True, False), (4, False, False)])
def test_lowrank_delta_validation(rank, with_proj, ok):
    """delta_rank 0 (off) or 1..16 with a (D, R) delta_proj; anything else is rejected."""
    a = _fwd_args(B=2, L=8, D=4, N=16)
    W = torch.zeros(4, max(rank, 1))
    low = torch.zeros(2, 8, max(rank, 1))
    a.delta = _abi.view(low)
    if with_proj:
        a.delta_proj = _abi.view(W)
    a.delta_rank = rank
    a._keep2 = (W, low)
    rc = _abi.lib().ssm_fwd_check(ctypes.byref(a))
    if ok:
        assert rc == 0
    else:
        with pytest.raises(ValueError):
            _abi.check(rc, "ssm_fwd")


def test_lowrank_delta_needs_small_dstate():
    a = _fwd_args(B=2, L=8, D=4, N=32)
    W, low = torch.zeros(4, 8), torch.zeros(2, 8, 8)
    a.delta, a.delta_proj, a.delta_rank = _abi.view(low), _abi.view(W), 8
    a._keep2 = (W, low)
    with pytest.raises(ValueError):
        _abi.check(_abi.lib().ssm_fwd_check(ctypes.byref(a)), "ssm_fwd")


@pytest.mark.parametrize("field,value", [("dstate", 65), ("width", 9), ("method", 3), ("batch", 0), ("dt_rank", 300),
                                         ("conv_state_dtype", 2), ("conv_state_dtype", 3)])
def test_decode_layer_validation(field, value):
    """ssm_decode_check rejects out-of-range layer shapes before any launch."""
    a = _abi.DecodeArgs()
    a.batch, a.dim, a.dstate, a.width, a.dt_rank, a.d_model, a.method = 2, 64, 16, 4, 4, 32, 0
    for name in ("u", "xz", "conv_w", "conv_b", "conv_state", "x_proj_wt", "dt_proj_w", "dt_bias", "A_log",
                 "Dskip", "ssm_state", "y"):
        setattr(a, name, 16)   # non-null placeholders: the check never dereferences them
    assert _abi.lib().ssm_decode_check(ctypes.byref(a)) == 0
    setattr(a, field, value)
    with pytest.raises(ValueError):
        _abi.check(_abi.lib().ssm_decode_check(ctypes.byref(a)), "ssm_decode_step")


def _stack_args(n_blocks=2):
    a = _abi.DecodeStackArgs()
    a.batch, a.dim, a.dstate, a.width, a.dt_rank, a.d_model, a.method = 64, 512, 16, 4, 16, 256, 0
    blocks = (_abi.DecodeBlock * n_blocks)()
    for k in blocks:
        for name, _ in _abi.DecodeBlock._fields_[:11]:
            setattr(k, name, 16)   # non-null placeholders: the check never dereferences them
        k.eps = 1e-5
    a.n_blocks, a.blocks, a.u = n_blocks, blocks, 16
    a.workspace = 16
    a.workspace_bytes = _abi.lib().ssm_decode_stack_workspace_bytes(ctypes.byref(a))
    a._keep = blocks
    return a


def test_decode_stack_workspace_layout():
    """Workspace of the stack step: two residual-stream buffers, the out_proj partial sums over
    64-channel tiles, the conv output and gate, the x_proj partial sums over 32-channel tiles,
    each region rounded up to 256 bytes, then the 256-byte region of the status word (bad token
    ids), whose offset ssm_decode_stack_status_offset reports."""
    a = _stack_args()
    r = lambda v: -(-v // 256) * 256
    B, dm, D, P = 64, 256, 512, 16 + 32
    want = 2 * r(B * dm * 4) + r(B * (D // 64) * dm * 4) + 2 * r(B * D * 4) + r(B * (D // 32) * P * 4)
    assert a.workspace_bytes == want + 256
    assert _abi.lib().ssm_decode_stack_status_offset(ctypes.byref(a)) == want
    assert _abi.lib().ssm_decode_stack_check(ctypes.byref(a)) == 0
    a.batch = 0
    assert _abi.lib().ssm_decode_stack_status_offset(ctypes.byref(a)) == -1


@pytest.mark.parametrize("field,value", [("d_model", 513), ("dim", 1025), ("dstate", 12), ("dt_rank", 24),
                                         ("width", 5), ("method", 3), ("batch", 0), ("n_blocks", 0),
                                         ("conv_state_dtype", 2), ("workspace_bytes", 1024), ("workspace", None),
                                         ("u", None), ("batch", 1 << 20), ("d_model", 250), ("u", 8)])
def test_decode_stack_validation(field, value):
    """ssm_decode_stack_check rejects shapes past the stack kernels' limits, a missing or short
    workspace and offsets past 32 bits before any launch."""
    a = _stack_args()
    setattr(a, field, value)
    with pytest.raises((ValueError, MemoryError)):
        _abi.check(_abi.lib().ssm_decode_stack_check(ctypes.byref(a)), "ssm_decode_stack")


@pytest.mark.parametrize("shape", [dict(), dict(d_model=128, d_state=8), dict(d_model=512), dict(d_model=520),
                                   dict(d_model=250), dict(d_state=12), dict(d_state=32), dict(d_conv=5),
                                   dict(d_conv=1), dict(d_model=384), dict(d_model=256, expand=3)])
def test_decoder_path_choice_agrees_with_the_library(shape):
    """FastDecoder takes the stack path exactly for the shapes ssm_decode_stack_check accepts
    (the Python limits and the C ones describe the same kernels)."""
    from ssm_scan.block import MambaLM
    from ssm_scan.decode import FastDecoder
    model = MambaLM(n_layers=1, **shape)
    m = model.blocks[0].mixer
    a = _stack_args(n_blocks=1)
    a.batch, a.dim, a.dstate, a.width, a.dt_rank = 8, m.d_inner, m.d_state, m.d_conv, m.dt_rank
    a.d_model = model.blocks[0].norm1.weight.numel()
    a.workspace_bytes = _abi.lib().ssm_decode_stack_workspace_bytes(ctypes.byref(a))
    accepted = _abi.lib().ssm_decode_stack_check(ctypes.byref(a)) == 0
    assert (FastDecoder(model).path == "stack") == accepted, (shape, _abi.lib().ssm_last_error())


@pytest.mark.parametrize("change", ["tokens_without_embed", "head_without_logits", "no_vocab", "huge_vocab"])
def test_decode_stack_ends_validation(change):
    """The optional ends of the token step: tokens need the embedding table, a head needs a
    logits buffer, and either needs a vocabulary whose offsets fit 32 bits."""
    a = _stack_args()
    a.tokens, a.embed, a.head_w4, a.logits, a.vocab = 16, 16, 16, 16, 256
    assert _abi.lib().ssm_decode_stack_check(ctypes.byref(a)) == 0
    if change == "tokens_without_embed":
        a.embed = None
    elif change == "head_without_logits":
        a.logits = None
    elif change == "no_vocab":
        a.vocab = 0
    else:
        a.vocab = 1 << 22
    with pytest.raises(ValueError):
        _abi.check(_abi.lib().ssm_decode_stack_check(ctypes.byref(a)), "ssm_decode_stack")


@pytest.mark.parametrize("name", [f for f, _ in _abi.DecodeBlock._fields_[:11]])
def test_decode_stack_block_tensors_required(name):
    """Every block tensor is required, the conv state except at conv width 1 (an empty state)."""
    a = _stack_args()
    setattr(a.blocks[1], name, None)
    with pytest.raises(ValueError):
        _abi.check(_abi.lib().ssm_decode_stack_check(ctypes.byref(a)), "ssm_decode_stack")
    if name == "conv_state":
        a.width = 1
        a.workspace_bytes = _abi.lib().ssm_decode_stack_workspace_bytes(ctypes.byref(a))
        assert _abi.lib().ssm_decode_stack_check(ctypes.byref(a)) == 0


def test_linear_scan_grid_limit():
    """One lane per recurrence (per chunk for the chunked algorithm) in a 1-D grid: 2^31 lanes
    or more is rejected before any launch."""
    t = torch.zeros(2, 8, 4)
    a = _abi.LscanArgs()
    a.batch, a.seqlen, a.width, a.algo, a.dtype = 2, 8, 4, 1, 0
    for name in ("a", "b", "h"):
        setattr(a, name, _abi.view(t))
    lib = _abi.lib()
    assert lib.ssm_lscan_check(ctypes.byref(a)) == 0
    a.batch, a.width = 4, 1 << 29
    with pytest.raises(ValueError, match="too large"):
        _abi.check(lib.ssm_lscan_check(ctypes.byref(a)), "ssm_lscan")
    a.batch, a.width, a.seqlen, a.chunk = 1, 1 << 20, 1 << 12, 1
    assert lib.ssm_lscan_check(ctypes.byref(a)) == 0      # sequential: 2^20 lanes
    a.algo = 4                                            # chunked, chunk 1: 2^32 lanes
    with pytest.raises(ValueError, match="too large"):
        _abi.check(lib.ssm_lscan_check(ctypes.byref(a)), "ssm_lscan")


def _norm_args(rows=4, dim=256, dtype=0):
    x = torch.zeros(rows, dim)
    a = _abi.NormArgs()
    a.rows, a.dim, a.dtype, a.eps = rows, dim, dtype, 1e-5
    a.x, a.weight = _abi.view(x), _abi.view(torch.ones(dim))
    a.rstd = x.data_ptr()
    a._keep = x
    return a


@pytest.mark.parametrize("change,ok", [({}, True), ({"dim": 1024}, True), ({"dim": 1025}, False),
                                       ({"dim": 0}, False), ({"rows": 0}, False), ({"dtype": 1}, False),
                                       ({"dtype": 3}, True), ({"eps": -1.0}, False)])
def test_norm_validation(change, ok):
    """RMSNorm rows of 1..1024 float32/float64 elements; other shapes and dtypes are rejected on
    the host."""
    a = _norm_args(**{k: v for k, v in change.items() if k in ("rows", "dim", "dtype")})
    if "eps" in change:
        a.eps = change["eps"]
    rc = _abi.lib().ssm_norm_check(ctypes.byref(a))
    if ok:
        assert rc == 0
    else:
        with pytest.raises(ValueError):
            _abi.check(rc, "ssm_norm")


def test_norm_needs_unit_column_stride_and_rstd():
    lib = _abi.lib()
    a = _norm_args()
    a.x.stride[1] = 2
    with pytest.raises(ValueError, match="unit column stride"):
        _abi.check(lib.ssm_norm_check(ctypes.byref(a)), "ssm_norm")
    a = _norm_args()
    a.rstd = None
    with pytest.raises(ValueError, match="rstd"):
        _abi.check(lib.ssm_norm_check(ctypes.byref(a)), "ssm_norm")
    a = _norm_args(rows=1000, dim=256)
    # backward partials: one (dim,) row per workgroup of 4 wavefronts x 8 rows
    assert lib.ssm_norm_workspace_bytes(ctypes.byref(a)) == ((1000 + 31) // 32) * 256 * 4


def test_disc_lane_offsets_validated():
    """The discretization kernels address a lane's channel (state) inside a row with a 31-bit
    element offset: an inner stride whose span over the channels (states) reaches 2^31 is
    rejected on the host; channel-major and time-major layouts of ordinary sizes pass."""
    t = torch.zeros(2, 8, 4)
    a = _abi.DiscArgs()
    a.batch, a.seqlen, a.dim, a.dstate, a.method, a.dtype = 2, 8, 4, 4, 0, 0
    a.delta, a.x, a.Bm, a.A = _abi.view(t), _abi.view(t.transpose(1, 2).contiguous().transpose(1, 2)), \
        _abi.view(t), _abi.view(torch.zeros(4, 4))
    lib = _abi.lib()
    assert lib.ssm_disc_check(ctypes.byref(a)) == 0
    a.x.stride[2] = (1 << 31) // 3 + 1                     # span 3 * stride >= 2^31
    with pytest.raises(ValueError, match="inner stride"):
        _abi.check(lib.ssm_disc_check(ctypes.byref(a)), "ssm_disc")
    a.x.stride[2] = 1
    a.Bm.stride[2] = -1
    with pytest.raises(ValueError, match="inner stride"):
        _abi.check(lib.ssm_disc_check(ctypes.byref(a)), "ssm_disc")
