"""The committed golden vectors (tests/golden/vectors.npz, written by tests/golden/make_vectors.py):
seeded float32 inputs and the float64 oracle's outputs for the fused scan (three
discretizations, with and without gate / D skip / h0 / dlast, and at 16 states), the linear scan
and its VJP, discretize and its VJP, the causal conv with a carried state, and the decode step.

CPU: the generator still draws the stored inputs bit for bit, and the oracle still computes the
stored outputs from them (a change to either shows here).  GPU: every HIP entry point on the
stored inputs against the stored outputs, at the float32 bar (rtol 1e-4 / atol 1e-5,
tests/parity.py)."""

import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_vectors as MV  # noqa: E402
import parity  # noqa: E402

CASES = MV.load()
SCAN_CASES = sorted(n for n in CASES if n.startswith("scan/"))


def test_vectors_hold_every_case_and_the_seeded_inputs():
    fresh = MV.make_inputs()
    assert set(fresh) == set(CASES)
    for name, inp in fresh.items():
        stored = CASES[name][0]
        assert set(inp) == set(stored), name
        for k, v in inp.items():
            assert stored[k].dtype == np.float32 and np.array_equal(stored[k], v), (name, k)


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_the_committed_outputs(name):
    inp, out = CASES[name]
    got = MV.compute(name, inp)
    assert set(got) == set(out), name
    for k, v in got.items():
        np.testing.assert_allclose(v, out[k], rtol=1e-10, atol=1e-13, err_msg=f"{name} {k}")


def close(got, ref, name):
    parity.close(got, ref, name=name)   # rtol 1e-4 / atol 1e-5 on every element


def _t(a, dev, grad=False):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.requires_grad_() if grad else t


@pytest.mark.gpu
@pytest.mark.parametrize("name", SCAN_CASES)
def test_fused_scan_matches_vectors(dev, name):
    import ssm_scan
    inp, ref = CASES[name]
    print(f"case {name} shape {inp['x'].shape} N {inp['A'].shape[1]}", flush=True)
    leaves = {k: _t(v, dev, grad=True) for k, v in inp.items() if k not in ("dout", "dlast")}
    out, last = ssm_scan.selective_scan_fn(leaves["x"], leaves["delta"], leaves["A"], leaves["Bm"], leaves["Cm"],
                                           D=leaves.get("D"), z=leaves.get("z"), h0=leaves.get("h0"),
                                           method=name.split("/")[1], return_last_state=True)
    loss = (out * _t(inp["dout"], dev)).sum()
    if "dlast" in inp:
        loss = loss + (last * _t(inp["dlast"], dev)).sum()
    loss.backward()
    close(out, ref["out"], "out")
    close(last, ref["last"], "last")
    for g, leaf in (("dx", "x"), ("ddelta", "delta"), ("dA", "A"), ("dB", "Bm"), ("dC", "Cm"), ("dD", "D"),
                    ("dz", "z"), ("dh0", "h0")):
        if leaf in leaves:
            close(leaves[leaf].grad, ref[g], g)


@pytest.mark.gpu
@pytest.mark.parametrize("algo", ["sequential", "hillis_steele", "blelloch", "chunked"])
def test_linear_scans_match_vectors(dev, algo):
    from ssm_scan import scan as S
    inp, ref = CASES["lscan"]
    a, b, h0 = (_t(inp[k], dev, grad=True) for k in ("a", "b", "h0"))
    h = S.SCANS[algo](a, b, h0)
    (h * _t(inp["dh"], dev)).sum().backward()
    close(h, ref["h"], "h")
    close(a.grad, ref["da"], "da")
    close(b.grad, ref["db"], "db")
    close(h0.grad, ref["dh0"], "dh0")


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
def test_discretize_matches_vectors(dev, method):
    from ssm_scan.scan import discretize
    inp, ref = CASES[f"disc/{method}"]
    delta, A, Bm, x = (_t(inp[k], dev, grad=True) for k in ("delta", "A", "Bm", "x"))
    a, b = discretize(delta, A, Bm, x, method)
    ((a * _t(inp["ga"], dev)).sum() + (b * _t(inp["gb"], dev)).sum()).backward()
    close(a, ref["a"], "a")
    close(b, ref["b"], "b")
    for g, leaf in (("ddelta", delta), ("dA", A), ("dBm", Bm), ("dx", x)):
        close(leaf.grad, ref[g], g)


@pytest.mark.gpu
def test_conv_with_state_matches_vectors(dev):
    from ssm_scan.conv import causal_conv1d
    inp, ref = CASES["conv"]
    state = _t(inp["state"], dev).clone()
    with torch.no_grad():
        y = causal_conv1d(_t(inp["x"], dev), _t(inp["w"], dev), _t(inp["bias"], dev), state=state)
    close(y, ref["y"], "y")
    close(state, ref["state"], "state")


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
def test_decode_step_matches_vectors(dev, method):
    from ssm_scan.step import ssm_step
    inp, ref = CASES[f"step/{method}"]
    t = {k: _t(v, dev) for k, v in inp.items()}
    h = t["h"].clone()
    y = ssm_step(h, t["x"], t["delta"], t["A"], t["Bm"], t["Cm"], D=t["D"], z=t["z"], method=method)
    close(y, ref["y"], "y")
    close(h, ref["h"], "h")
