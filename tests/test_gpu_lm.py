"""The Mamba LM of models/lm.py (10 Mamba layers, d_model 256, BASELINE config 3's architecture)
with the scan path on the engine's kernels, against the float64 torch restatement of the
reference model (oracle/lm_ref.py) on identical weights: logits, loss and every parameter
gradient; and the recurrent decode path (prefill + one token at a time) against the full
forward (tests/test_models.py:36-48 of the reference).

Tolerances: float32 through 10 layers -- logits rtol 1e-4 / atol 1e-5 x max|logit|,
gradients rtol 1e-3 / atol 1e-4 x max|grad| per parameter.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ssm_scan.block import MambaLM
from oracle import lm_ref
from ssm_inputs import np64

pytestmark = pytest.mark.gpu


def build(seed=0, n_layers=10):
    torch.manual_seed(seed)
    return MambaLM(n_layers=n_layers)


def ref_params(model):
    return {k: v.detach().cpu().double().requires_grad_() for k, v in model.state_dict().items()}


def test_lm_forward_backward_matches_reference(dev):
    model = build(0).to(dev)
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, 256, (2, 48), generator=g)
    tgt = torch.randint(0, 256, (2, 48), generator=g)
    logits = model(idx.to(dev))
    loss = F.cross_entropy(logits.reshape(-1, 256), tgt.to(dev).reshape(-1))
    loss.backward()
    p = ref_params(model)
    rlogits = lm_ref.lm_forward(p, idx, n_layers=10)
    rloss = F.cross_entropy(rlogits.reshape(-1, 256), tgt.reshape(-1))
    rloss.backward()
    scale = float(rlogits.detach().abs().max())
    np.testing.assert_allclose(np64(logits), rlogits.detach().numpy(), rtol=1e-4, atol=1e-5 * scale)
    assert abs(loss.item() - rloss.item()) < 1e-5 * rloss.item()
    named = dict(model.named_parameters())
    assert len(named) == len([k for k in p if k != "head.weight"])
    for name, prm in named.items():
        ref = p[name].grad.numpy()
        gs = max(float(np.abs(ref).max()), 1e-12)
        np.testing.assert_allclose(np64(prm.grad), ref, rtol=1e-3, atol=1e-4 * gs, err_msg=name)


@pytest.mark.parametrize("batch", [1, 3])
def test_prefill_and_decode_match_full_forward(dev, batch):
    model = build(2, n_layers=4).to(dev).eval()
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 256, (batch, 40), generator=g).to(dev)
    with torch.no_grad():
        full = model(idx)
        states = model.init_state(batch, 40, dev)
        out = [model(idx[:, :25], states, 0)]
        for t in range(25, 40):
            out.append(model(idx[:, t:t + 1], states, t))
    got = torch.cat(out, 1)
    scale = float(full.abs().max())
    np.testing.assert_allclose(np64(got), np64(full), rtol=1e-4, atol=1e-5 * scale)


def test_decode_state_matches_reference(dev):
    """Token-by-token decode from a random state equals the reference recurrence."""
    model = build(4, n_layers=2).to(dev).eval()
    p = {k: v.detach().cpu().double() for k, v in model.state_dict().items()}
    g = torch.Generator().manual_seed(5)
    states = model.init_state(4, 8, dev)
    rstates = []
    for s in states:
        s.ssm.copy_(torch.randn(s.ssm.shape, generator=g).to(dev))
        s.conv.copy_(torch.randn(s.conv.shape, generator=g).to(dev))
        rstates.append({"conv": s.conv.detach().cpu().double().clone(), "ssm": s.ssm.detach().cpu().double().clone()})
    idx = torch.randint(0, 256, (4, 6), generator=g)
    with torch.no_grad():
        got = torch.cat([model(idx[:, t:t + 1].to(dev), states, t) for t in range(6)], 1)
    ref = torch.cat([lm_ref.lm_forward(p, idx[:, t:t + 1], n_layers=2, states=rstates) for t in range(6)], 1)
    scale = float(ref.abs().max())
    np.testing.assert_allclose(np64(got), ref.numpy(), rtol=1e-4, atol=1e-5 * scale)
    for s, r in zip(states, rstates):
        np.testing.assert_allclose(np64(s.ssm), r["ssm"].numpy(), rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(np64(s.conv), r["conv"].numpy(), rtol=1e-6, atol=1e-6)


def _random_states(model, B, dev, seed):
    g = torch.Generator().manual_seed(seed)
    states = model.init_state(B, 1, dev)
    for s in states:
        s.ssm.copy_(torch.randn(s.ssm.shape, generator=g))
        s.conv.copy_(torch.randn(s.conv.shape, generator=g))
    return states


def _clone(states):
    from types import SimpleNamespace
    return [SimpleNamespace(conv=s.conv.clone(), ssm=s.ssm.clone()) for s in states]


# the LM shape and dstate 8 / bilinear, dim 256 / dt_rank 8 / width 2 (row-resident kernel);
# dstate 12 and a wider layer (dim 768, dt_rank 24), which take the general kernel
DECODE_SHAPES = [
    dict(n_layers=10),
    dict(n_layers=3, d_state=8, discretization="bilinear"),
    dict(n_layers=3, d_state=12, d_conv=3, discretization="euler"),
    dict(n_layers=2, d_model=384),
    dict(n_layers=2, d_model=128, d_conv=2, discretization="euler"),
]


@pytest.mark.parametrize("shape", DECODE_SHAPES, ids=lambda s: "-".join(f"{k}{v}" for k, v in s.items()))
def test_fused_decode_layer_matches_module_decode(dev, shape):
    """ssm_decode_step (one fused launch per layer) == the module's decode path, incl. states."""
    from ssm_scan.decode import FastDecoder
    torch.manual_seed(6)
    model = MambaLM(**shape).to(dev).eval()
    fast = FastDecoder(model)
    s_ref = _random_states(model, 64, dev, 7)
    s_fast = _clone(s_ref)
    toks = torch.randint(0, 256, (8, 64, 1), generator=torch.Generator().manual_seed(8)).to(dev)
    with torch.no_grad():
        for t in range(8):
            ref = model(toks[t], s_ref, t)[:, 0]
            got = fast.step(toks[t], s_fast)
            scale = float(ref.abs().max())
            np.testing.assert_allclose(np64(got), np64(ref), rtol=1e-4, atol=1e-5 * scale)
    for a, b_ in zip(s_fast, s_ref):
        np.testing.assert_allclose(np64(a.ssm), np64(b_.ssm), rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(np64(a.conv), np64(b_.conv), rtol=1e-5, atol=1e-6)


def test_fused_decode_graph_replays_match_eager(dev):
    """The token step captured in a HIP graph: every replay (with eager work between) equals the
    eager step from the same states and token."""
    from ssm_scan.decode import FastDecoder
    model = build(9, n_layers=3).to(dev).eval()
    fast = FastDecoder(model)
    states = _random_states(model, 16, dev, 10)
    tok = torch.zeros(16, 1, dtype=torch.long, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        snap = _clone(states)
        fast.step(tok, states)                       # warm-up on the side stream
        for s, c in zip(states, snap):
            s.conv.copy_(c.conv)
            s.ssm.copy_(c.ssm)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fast.step(tok, states)
    g = torch.Generator().manual_seed(11)
    for r in range(4):
        before = _clone(states)
        tok.copy_(torch.randint(0, 256, (16, 1), generator=g))
        graph.replay()
        torch.cuda.synchronize()
        eager_states = before
        ref = fast.step(tok, eager_states)           # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref), r
        for a, b_ in zip(states, eager_states):
            assert torch.equal(a.ssm, b_.ssm) and torch.equal(a.conv, b_.conv)
