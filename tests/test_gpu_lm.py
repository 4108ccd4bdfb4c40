"""The Mamba LM of models/lm.py (10 Mamba layers, d_model 256, BASELINE config 3's architecture)
with the scan path on the engine's kernels, against the float64 torch restatement of the
reference model (oracle/lm_ref.py) on identical weights: logits, loss and every parameter
gradient (at B2 x L48 and at config 3's own B16 x L512); streaming prefill with carried states
and a checkpoint in the reference's format against the same restatement; and the recurrent
decode path (prefill + one token at a time) against the full forward (tests/test_models.py:36-48
of the reference).

Tolerances: every LM check holds two bars.  The literal north_star bar (rtol 1e-4 / atol 1e-5 on
every element) and an LM bar scaled to the tensor, which is the stricter one for the small
weight gradients: float32 through 10 layers and float32 GEMMs -- logits rtol 1e-4 / atol 1e-5
x max|logit|, gradients rtol 1e-3 / atol 1e-4 x max|grad| per parameter.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import parity
from ssm_scan.block import MambaLM
from oracle import lm_ref
from ssm_inputs import np64

pytestmark = pytest.mark.gpu


def build(seed=0, n_layers=10):
    torch.manual_seed(seed)
    return MambaLM(n_layers=n_layers)


def ref_params(model):
    return {k: v.detach().cpu().double().requires_grad_() for k, v in model.state_dict().items()}


def lm_close(got, ref, name, rtol=1e-4, atol_rel=1e-5, allow_literal=0):
    """The LM bar: rtol, atol = atol_rel x max|ref| -- and the literal north_star bar (rtol
    1e-4 / atol 1e-5) as well, with at most `allow_literal` elements outside it (none by
    default; the count is printed).  For tensors whose largest element is small (the LM's
    weight gradients) the LM bar is the stricter of the two."""
    g = np64(got) if isinstance(got, torch.Tensor) else np.asarray(got)
    r = ref.detach().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
    lit = parity.outside(g, r)
    scale = max(float(np.abs(r).max()), 1e-12)
    print(f"parity {name}: {lit} of {g.size} outside the literal bar (rtol 1e-4 / atol 1e-5); "
          f"LM bar rtol {rtol:g} / atol {atol_rel * scale:.3g}", flush=True)
    np.testing.assert_allclose(g, r, rtol=rtol, atol=atol_rel * scale, err_msg=name)
    if allow_literal is not None:
        assert lit <= allow_literal, f"{name}: {lit} outside the literal bar (allowed {allow_literal})"
    return lit


def check_lm_grads(model, p, allow_literal=0):
    """Every parameter gradient against the float64 reference: the literal bar with no element
    outside it, and the LM bar (rtol 1e-3, atol 1e-4 x max|grad|), the stricter one for
    gradients whose largest element is below 0.1."""
    named = dict(model.named_parameters())
    assert len(named) == len([k for k in p if k != "head.weight"])
    for name, prm in named.items():
        lm_close(prm.grad, p[name].grad, name, rtol=1e-3, atol_rel=1e-4, allow_literal=allow_literal)


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
    lm_close(logits, rlogits, "logits")
    assert abs(loss.item() - rloss.item()) < 1e-5 * rloss.item()
    check_lm_grads(model, p)


def test_config3_lm_train_step_matches_reference(dev):
    """BASELINE config 3 at its own workload: the 10-layer LM (d_model 256, d_inner 512, dstate
    16, dt_rank 16) forward + backward on B16 x L512 = 8,192 tokens of uniform random bytes
    with next-byte cross-entropy (benchmarks/bench_models.py:48-52, models/lm.py:124-128).  At
    this size the mixer node (ssm_scan.mixer) and the split-K weight gradients
    (ssm_scan.linear, from 2,048 tokens) run, as in the benchmark.  Against oracle/lm_ref in
    float64 with each layer's scan on the C oracle's forward and adjoint: logits, loss and
    every parameter gradient at the literal bar with none outside (and at the LM bar); the
    per-tensor counts are printed."""
    model = build(0).to(dev)
    g = torch.Generator().manual_seed(41)
    data = torch.randint(0, 256, (16, 513), generator=g)
    idx, tgt = data[:, :-1], data[:, 1:]
    logits = model(idx.to(dev))
    loss = F.cross_entropy(logits.reshape(-1, 256), tgt.to(dev).reshape(-1))
    loss.backward()
    torch.cuda.synchronize()
    print(f"config 3: engine loss {loss.item():.8f}", flush=True)
    p = ref_params(model)
    rlogits = lm_ref.lm_forward(p, idx, n_layers=10, scan="c")
    rloss = F.cross_entropy(rlogits.reshape(-1, 256), tgt.reshape(-1))
    rloss.backward()
    print(f"config 3: reference loss {rloss.item():.8f}", flush=True)
    lm_close(logits, rlogits, "logits")
    assert abs(loss.item() - rloss.item()) < 1e-5 * rloss.item()
    check_lm_grads(model, p)


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
    fast = FastDecoder(model, path="block")
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


@pytest.mark.parametrize("path", ["stack", "block"])
def test_fused_decode_graph_replays_match_eager(dev, path):
    """The token step captured in a HIP graph: every replay (with eager work between) equals the
    eager step from the same states and token, bit for bit."""
    from ssm_scan.decode import FastDecoder
    model = build(9, n_layers=3).to(dev).eval()
    fast = FastDecoder(model, path=path)
    assert fast.path == path
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


def test_streaming_prefill_matches_one_call(dev):
    """Prefill in pieces (conv and SSM states carried, pieces of length 1 take the decode step)
    equals one prefill call over the whole input, logits and final states
    (analysis/length_generalization.py:110-116 streams inputs this way)."""
    model = build(12, n_layers=3).to(dev).eval()
    g = torch.Generator().manual_seed(13)
    idx = torch.randint(0, 256, (2, 60), generator=g).to(dev)
    with torch.no_grad():
        s_one = model.init_state(2, 60, dev)
        full = model(idx, s_one, 0)
        s_str = model.init_state(2, 60, dev)
        parts, p0 = [], 0
        for n in (7, 16, 1, 1, 20, 3, 12):
            parts.append(model(idx[:, p0:p0 + n], s_str, p0))
            p0 += n
    assert p0 == 60
    scale = float(full.abs().max())
    np.testing.assert_allclose(np64(torch.cat(parts, 1)), np64(full), rtol=1e-4, atol=1e-5 * scale)
    for a, b_ in zip(s_str, s_one):
        np.testing.assert_allclose(np64(a.ssm), np64(b_.ssm), rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(np64(a.conv), np64(b_.conv), rtol=1e-5, atol=1e-6)
    assert torch.equal(s_str[0].conv, s_one[0].conv)      # first layer: the same in_proj inputs


def test_streaming_prefill_matches_reference(dev):
    """Prefill in pieces of 7, 16, 1, 1, 20, 3 and 12 tokens with the conv and SSM states carried
    between calls (analysis/length_generalization.py:110-116 streams inputs this way; pieces of
    length 1 take the decode step) against the float64 restatement run piece by piece on its
    own carried states (models/mamba.py:104-106,122-123): every piece's logits at the LM bar,
    the final SSM and conv states of every layer at the literal bar."""
    model = build(12, n_layers=3).to(dev).eval()
    p = {k: v.detach().cpu().double() for k, v in model.state_dict().items()}
    g = torch.Generator().manual_seed(13)
    idx = torch.randint(0, 256, (2, 60), generator=g)
    states = model.init_state(2, 60, dev)
    rstates = [{"conv": torch.zeros(2, 512, 3, dtype=torch.float64),
                "ssm": torch.zeros(2, 512, 16, dtype=torch.float64)} for _ in range(3)]
    p0 = 0
    with torch.no_grad():
        for n in (7, 16, 1, 1, 20, 3, 12):
            got = model(idx[:, p0:p0 + n].to(dev), states, p0)
            ref = lm_ref.lm_forward(p, idx[:, p0:p0 + n], n_layers=3, states=rstates)
            lm_close(got, ref, f"logits[{p0}:{p0 + n}]")
            p0 += n
    assert p0 == 60
    for i, (s, r) in enumerate(zip(states, rstates)):
        parity.close(s.ssm, r["ssm"], name=f"ssm state {i}")
        parity.close(s.conv, r["conv"], name=f"conv state {i}")


def _reference_state_dict(n_layers, d_model=256, d_state=16, expand=2, d_conv=4, vocab=256, seed=0):
    """A state_dict under the reference's names and shapes (models/lm.py:92-100,
    models/mamba.py:26-66), drawn here from a seeded generator with the scales of the
    reference's initialization (not taken from this engine's modules)."""
    g = torch.Generator().manual_seed(seed)
    di, R = expand * d_model, -(-d_model // 16)
    rn = lambda *s, std=1.0: torch.randn(*s, generator=g) * std
    un = lambda *s, b=1.0: (torch.rand(*s, generator=g) * 2 - 1) * b
    sd = {"embed.weight": rn(vocab, d_model, std=0.02), "norm_f.weight": 1 + rn(d_model, std=0.1)}
    for i in range(n_layers):
        q = f"blocks.{i}."
        dt = torch.exp(torch.rand(di, generator=g) * (np.log(0.1) - np.log(1e-3)) + np.log(1e-3))
        sd.update({q + "norm1.weight": 1 + rn(d_model, std=0.1),
                   q + "mixer.in_proj.weight": rn(2 * di, d_model, std=0.02),
                   q + "mixer.conv.weight": un(di, 1, d_conv, b=d_conv ** -0.5),
                   q + "mixer.conv.bias": un(di, b=d_conv ** -0.5),
                   q + "mixer.x_proj.weight": rn(R + 2 * d_state, di, std=0.02),
                   q + "mixer.dt_proj.weight": un(di, R, b=R ** -0.5),
                   q + "mixer.dt_proj.bias": dt + torch.log(-torch.expm1(-dt)),
                   q + "mixer.A_log": torch.log(torch.arange(1, d_state + 1.0)).repeat(di, 1) + rn(di, d_state, std=0.1),
                   q + "mixer.D": 1 + rn(di, std=0.1),
                   q + "mixer.out_proj.weight": rn(d_model, di, std=0.02 / np.sqrt(2 * n_layers))})
    sd["head.weight"] = sd["embed.weight"]
    return sd


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
def test_reference_checkpoint_matches_reference_model(dev, method):
    """A checkpoint in the training script's format (training/train_lm.py:166: {"cfg": LMConfig
    dict, "state_dict"}) built under the reference's parameter names, loaded the way
    analysis/evaluate_lm.py:26-30 loads it: the engine's logits on a batch of bytes equal the
    float64 restatement's on the same state_dict at the LM bar."""
    import io
    from ssm_scan.block import load_checkpoint
    sd = _reference_state_dict(3, seed=24)
    cfg = dict(layers="MMM", vocab_size=256, d_model=256, n_head=4, mlp_ratio=4.0, dropout=0.0,
               attn_impl="manual", pos_encoding="rope", attn_query_chunk=1024, d_state=16, expand=2,
               d_conv=4, selective=True, a_mode="s4d", discretization=method, scan="auto", d_block=0,
               chunk_size=0, retention_chunk=64)
    buf = io.BytesIO()
    torch.save({"cfg": cfg, "state_dict": sd}, buf)
    buf.seek(0)
    model = load_checkpoint(buf, dev)
    idx = torch.randint(0, 256, (3, 70), generator=torch.Generator().manual_seed(25))
    with torch.no_grad():
        got = model(idx.to(dev))
    ref = lm_ref.lm_forward({k: v.double() for k, v in sd.items()}, idx, n_layers=3, method=method)
    lm_close(got, ref, f"logits ({method})")


def test_long_sequence_autocast_forward_backward_is_finite(dev):
    """tests/test_gpu.py:68-77 of the reference: a 2-layer LM (d_model 64) on one sequence of
    16,384 bytes, forward under bf16 autocast, loss = mean logsumexp of the logits, backward:
    the loss and every parameter gradient are finite.  One batch row of 128 channels runs the
    scan's time segments in both passes with bf16 inputs."""
    torch.manual_seed(0)
    m = MambaLM(n_layers=2, d_model=64).to(dev)
    x = torch.randint(0, 256, (1, 16384), generator=torch.Generator().manual_seed(26)).to(dev)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = m(x).float().logsumexp(-1).mean()
    loss.backward()
    torch.cuda.synchronize()
    print(f"loss {loss.item():.6f}", flush=True)
    assert torch.isfinite(loss)
    grads = {k: p.grad for k, p in m.named_parameters() if p.grad is not None}
    assert len(grads) == len(list(m.parameters()))
    for k, gr in grads.items():
        assert torch.isfinite(gr).all(), k
        assert gr.abs().sum() > 0, k


def test_streaming_prefill_under_bf16_autocast(dev):
    """The reference streams under torch.autocast(bf16) with float32 states; the pieces equal
    one autocast call over the whole input to bf16 accuracy (2e-2 x max|logit|)."""
    model = build(14, n_layers=2).to(dev).eval()
    idx = torch.randint(0, 256, (1, 48), generator=torch.Generator().manual_seed(15)).to(dev)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        full = model(idx).float()
        st = model.init_state(1, 48, dev, torch.float32)
        parts = [model(idx[:, p0:p0 + 16], st, p0).float() for p0 in range(0, 48, 16)]
    scale = float(full.abs().max())
    np.testing.assert_allclose(np64(torch.cat(parts, 1)), np64(full), rtol=0, atol=2e-2 * scale)
    assert all(s.ssm.dtype == torch.float32 and s.conv.dtype == torch.float32 for s in st)


@pytest.mark.parametrize("scan", ["chunked", "blelloch"])
def test_named_scan_algorithm_matches_fused(dev, scan):
    """Mamba(scan=<algorithm of models/scan.py>) runs that algorithm on the engine; forward
    and gradients equal the fused kernel's (models/lm.py:70-71 passes cfg.scan through)."""
    torch.manual_seed(16)
    fused = MambaLM(n_layers=2).to(dev)
    named = MambaLM(n_layers=2, scan=scan, chunk_size=8).to(dev)
    named.load_state_dict(fused.state_dict())
    idx = torch.randint(0, 256, (2, 40), generator=torch.Generator().manual_seed(17)).to(dev)
    outs = []
    for m in (fused, named):
        logits = m(idx)
        logits.square().mean().backward()
        outs.append((logits, {k: p.grad for k, p in m.named_parameters()}))
    scale = float(outs[0][0].detach().abs().max())
    np.testing.assert_allclose(np64(outs[1][0]), np64(outs[0][0]), rtol=1e-4, atol=1e-5 * scale)
    for k, g0 in outs[0][1].items():
        gs = max(float(g0.abs().max()), 1e-12)
        np.testing.assert_allclose(np64(outs[1][1][k]), np64(g0), rtol=1e-3, atol=1e-4 * gs, err_msg=k)


def test_lm_is_causal(dev):
    """tests/test_models.py:26-34: logits before position 25 do not change when later tokens do
    (bitwise here: every kernel on the path computes a position from earlier positions only),
    and logits from position 25 on do change."""
    torch.manual_seed(0)
    model = MambaLM(n_layers=2).to(dev).eval()
    g = torch.Generator().manual_seed(5)
    x = torch.randint(0, 256, (2, 40), generator=g)
    x2 = x.clone()
    x2[:, 25:] = torch.randint(0, 256, (2, 15), generator=g)
    with torch.no_grad():
        y, y2 = model(x.to(dev)), model(x2.to(dev))
    assert torch.equal(y[:, :25], y2[:, :25])
    assert not torch.allclose(y[:, 25:], y2[:, 25:])


def test_lm_can_overfit_a_batch(dev):
    """tests/test_models.py:96-110: 150 AdamW steps (lr 1e-2) on one batch of 4 x 33 random
    bytes take the cross-entropy from above 5 to below 0.5, every gradient from the engine."""
    torch.manual_seed(0)
    model = MambaLM(n_layers=2, d_model=64).to(dev)
    x = torch.randint(0, 256, (4, 33), generator=torch.Generator().manual_seed(0)).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-2)
    for step in range(150):
        loss = torch.nn.functional.cross_entropy(model(x[:, :-1]).reshape(-1, 256), x[:, 1:].reshape(-1))
        opt.zero_grad()
        loss.backward()
        opt.step()
        if step == 0:
            first = loss.item()
    print(f"loss {first:.3f} -> {loss.item():.4f}", flush=True)
    assert first > 5.0 and loss.item() < 0.5, (first, loss.item())


def test_lti_ablation_has_constant_delta(dev):
    """selective=False freezes delta to a learned constant (tests/test_models.py:60-64)."""
    torch.manual_seed(18)
    m = MambaLM(n_layers=1, d_model=32, selective=False).to(dev)
    u = torch.randn(2, 10, 32, device=dev)
    _, delta = m.blocks[0].mixer(u, return_delta=True)
    assert torch.equal(delta, delta[:, :1].expand_as(delta))


def test_scalar_decay_shares_decay_and_decodes_consistently(dev):
    """a_mode="scalar": one decay per channel; prefill + decode equals the full forward
    (tests/test_models.py:144-155)."""
    torch.manual_seed(19)
    m = MambaLM(n_layers=2, d_model=64, a_mode="scalar").to(dev).eval()
    mixer = m.blocks[0].mixer
    _, A, _, _ = mixer.ssm_params(torch.randn(1, 3, mixer.d_inner, device=dev))
    assert torch.equal(A, A[:, :1].expand_as(A))
    x = torch.randint(0, 256, (2, 25), generator=torch.Generator().manual_seed(20)).to(dev)
    with torch.no_grad():
        full = m(x)
        st = m.init_state(2, 25, dev)
        parts = [m(x[:, :9], st, 0)] + [m(x[:, t:t + 1], st, t) for t in range(9, 25)]
    scale = float(full.abs().max())
    np.testing.assert_allclose(np64(torch.cat(parts, 1)), np64(full), rtol=1e-4, atol=1e-5 * scale)


def test_generate_and_checkpoint_round_trip(dev):
    """generate() (models/lm.py:130-147) is reproducible under a seed, and a checkpoint in the
    training script's format reloads to the same logits."""
    import io
    from ssm_scan.block import load_checkpoint
    model = build(21, n_layers=2).to(dev).eval()
    prompt = torch.randint(0, 256, (2, 5), generator=torch.Generator().manual_seed(22)).to(dev)
    torch.manual_seed(23)
    a = model.generate(prompt, 6, temperature=0.8, top_k=20)
    torch.manual_seed(23)
    b = model.generate(prompt, 6, temperature=0.8, top_k=20)
    assert a.shape == (2, 11) and torch.equal(a, b) and torch.equal(a[:, :5], prompt)
    buf = io.BytesIO()
    cfg = dict(layers="MM", vocab_size=256, d_model=256, d_state=16, expand=2, d_conv=4)
    torch.save({"cfg": cfg, "state_dict": model.state_dict()}, buf)
    buf.seek(0)
    again = load_checkpoint(buf, dev)
    with torch.no_grad():
        assert torch.equal(again(prompt), model(prompt))


# the row-resident kernel's shapes (the LM preset; dstate 8 bilinear) and the general kernel's:
# dstate 12, conv width 5 and 6 (> 4), dim 640 and 768 (> 512)
ORACLE_DECODE_SHAPES = [
    dict(n_layers=10),
    dict(n_layers=3, d_state=8, discretization="bilinear"),
    dict(n_layers=3, d_state=12, d_conv=5, discretization="euler"),
    dict(n_layers=2, d_model=384),
    dict(n_layers=2, d_model=320, d_state=12, d_conv=6),
]


# the stack kernels' shapes: the LM preset; dstate 8 bilinear over a ragged batch; dim 240 and
# 488 (ragged channel tiles), width 1 and 2; d_model 512
# (two passes over d_model, dt_rank 32, dim 1024); a single block; batch 1 with a vocabulary of
# 300 (a ragged last vocabulary tile of the head)
STACK_DECODE_SHAPES = [
    (dict(n_layers=10), 64),
    (dict(n_layers=3, d_state=8, discretization="bilinear"), 37),
    (dict(n_layers=2, d_model=120, d_conv=1, discretization="euler"), 5),
    (dict(n_layers=2, d_model=244, d_conv=2), 19),
    (dict(n_layers=2, d_model=512), 64),
    (dict(n_layers=1, d_model=128, d_state=8), 9),
    (dict(n_layers=2, vocab_size=300), 1),
]


def _decoder_vs_oracle(dev, shape, B, path, T=8):
    from ssm_scan.decode import FastDecoder
    from parity import close
    torch.manual_seed(11)
    model = MambaLM(**shape).to(dev).eval()
    m = model.blocks[0].mixer
    fast = FastDecoder(model, path=path)
    assert fast.path == path
    states = _random_states(model, B, dev, 12)
    rstates = [{"conv": s.conv.cpu().double().clone(), "ssm": s.ssm.cpu().double().clone()} for s in states]
    p = {k: v.detach().cpu().double() for k, v in model.state_dict().items()}
    toks = torch.randint(0, 256, (T, B, 1), generator=torch.Generator().manual_seed(13))
    for t in range(T):
        got = fast.step(toks[t].to(dev), states)
        with torch.no_grad():
            ref = lm_ref.lm_forward(p, toks[t], n_layers=shape["n_layers"], d_state=m.d_state, dt_rank=m.dt_rank,
                                    d_conv=m.d_conv, states=rstates, method=m.discretization)[:, 0]
        close(got, ref, rtol=1e-4, atol=1e-5 * float(ref.abs().max()), name=f"logits token {t}")
    for i, (s, r) in enumerate(zip(states, rstates)):
        close(s.ssm, r["ssm"], name=f"layer {i} ssm state")
        close(s.conv, r["conv"], name=f"layer {i} conv state")


@pytest.mark.parametrize("shape", ORACLE_DECODE_SHAPES, ids=lambda s: "-".join(f"{k}{v}" for k, v in s.items()))
def test_fast_decoder_matches_float64_reference(dev, shape):
    """FastDecoder.step's per-block path (in_proj GEMM, the fused decode launch, out_proj +
    residual GEMM per block) against the float64 restatement of the reference's recurrent decode
    (models/mamba.py:104-125, lm_ref.lm_forward with states), batch 64, 8 tokens from random conv
    and ssm states: logits after every token, then every layer's ssm and conv state.

    Tolerances: states at the float32 bar (rtol 1e-4 / atol 1e-5); logits rtol 1e-4 with atol
    1e-5 x max|logit| (logits are float32 GEMMs over d_model terms of the final hidden state)."""
    _decoder_vs_oracle(dev, shape, 64, "block")


@pytest.mark.parametrize("shape,batch", STACK_DECODE_SHAPES,
                         ids=lambda v: "-".join(f"{k}{x}" for k, x in v.items()) if isinstance(v, dict) else f"B{v}")
def test_decode_stack_matches_float64_reference(dev, shape, batch):
    """FastDecoder.step's stack path (ssm_decode_stack: two launches per block with the GEMMs
    inside) against the same float64 restatement and at the same bar as the per-block path."""
    _decoder_vs_oracle(dev, shape, batch, "stack")


def _random_stack_shapes(count, seed):
    """Seeded shapes inside the stack kernels' limits: d_model a multiple of 4 whose dt_rank
    (ceil(d_model / 16)) is 8, 16 or 32, expand 1 or 2, dstate 8 or 16, conv width 1-4, every
    discretization, batch 1-70, 1-3 blocks."""
    import random
    rng = random.Random(seed)
    out = []
    for _ in range(count):
        dm = rng.choice([116, 120, 124, 128, 244, 248, 252, 256, 500, 504, 508, 512])
        expand = rng.choice([1, 2])
        shape = dict(n_layers=rng.randint(1, 3), d_model=dm, expand=expand, d_state=rng.choice([8, 16]),
                     d_conv=rng.randint(1, 4), discretization=rng.choice(["zoh", "euler", "bilinear"]))
        out.append((shape, rng.randint(1, 70)))
    return out


@pytest.mark.parametrize("shape,batch", _random_stack_shapes(8, 2024),
                         ids=lambda v: "-".join(f"{k}{x}" for k, x in v.items()) if isinstance(v, dict) else f"B{v}")
def test_decode_stack_random_shapes_match_float64_reference(dev, shape, batch):
    """The stack path on seeded random shapes within its limits, 3 tokens each, against the
    float64 restatement at the same bar as the fixed shapes."""
    _decoder_vs_oracle(dev, shape, batch, "stack", T=3)


@pytest.mark.parametrize("path", ["stack", "block"])
def test_decoders_at_a_large_batch_match_float64_reference(dev, path):
    """Both decode paths at batch 1000 (250 row tiles of the stack kernels, 1000 workgroups of
    the per-block kernel), 2 tokens, against the float64 restatement at the same bar."""
    _decoder_vs_oracle(dev, dict(n_layers=2), 1000, path, T=2)


def test_decode_stack_token_outside_vocabulary_reads_zero_row(dev):
    """A token id outside [0, vocab) reads a zero embedding row in the stack path (the reference's
    embedding raises instead): the step equals the step of a model whose row 7 is zero, given
    token 7 there: states, and the logits of every other vocabulary entry (the head is tied to the
    embedding).  Such a step raises the device status word that bad_tokens_seen() reports (a step
    with valid ids does not), and step(check_ids=True) raises IndexError before any launch on
    both paths, as the reference's nn.Embedding does (models/lm.py:125)."""
    from ssm_scan.decode import FastDecoder
    torch.manual_seed(31)
    model = MambaLM(n_layers=2).to(dev).eval()
    zeroed = MambaLM(n_layers=2).to(dev).eval()
    zeroed.load_state_dict(model.state_dict())
    with torch.no_grad():
        zeroed.embed.weight[7].zero_()
    s1 = _random_states(model, 6, dev, 32)
    s2 = _clone(s1)
    tok = torch.tensor([3, 300, -1, 5, 255, 1 << 40], device=dev)
    fast, fast_zeroed = FastDecoder(model, path="stack"), FastDecoder(zeroed, path="stack")
    got = fast.step(tok, s1)
    ref = fast_zeroed.step(torch.tensor([3, 7, 7, 5, 255, 7], device=dev), s2)
    keep = torch.arange(got.shape[1], device=dev) != 7
    assert torch.equal(got[:, keep], ref[:, keep])
    for a, b_ in zip(s1, s2):
        assert torch.equal(a.ssm, b_.ssm) and torch.equal(a.conv, b_.conv)
    assert fast.bad_tokens_seen() and not fast.bad_tokens_seen()    # reported once, then cleared
    assert not fast_zeroed.bad_tokens_seen()
    fast.step(torch.tensor([3, 7, 0, 5, 255, 9], device=dev), s1)
    assert not fast.bad_tokens_seen()
    for path in ("stack", "block"):
        before = _clone(s1)
        with pytest.raises(IndexError):
            FastDecoder(model, path=path).step(tok, s1, check_ids=True)
        for a, b_ in zip(s1, before):                                # nothing ran
            assert torch.equal(a.ssm, b_.ssm) and torch.equal(a.conv, b_.conv)


def test_decode_stack_limits_fall_back_to_blocks(dev):
    """Shapes past the stack kernels' limits take the per-block path; asking for the stack path
    with them is an error."""
    from ssm_scan.decode import FastDecoder
    for shape in (dict(d_state=12), dict(d_model=250)):
        model = MambaLM(n_layers=1, **shape).to(dev).eval()
        assert FastDecoder(model).path == "block"
        with pytest.raises(ValueError):
            FastDecoder(model, path="stack")


# the row-resident kernel (LM preset) and the general one (dstate 12, width 5)
BF16_STATE_SHAPES = [dict(n_layers=4), dict(n_layers=2, d_state=12, d_conv=5)]


@pytest.mark.parametrize("shape", BF16_STATE_SHAPES, ids=lambda s: "-".join(f"{k}{v}" for k, v in s.items()))
def test_fast_decoder_bf16_conv_state(dev, shape):
    """The states of a model run under bf16 autocast (conv state bf16, SSM state float32,
    models/mamba.py:86-91): FastDecoder.step inside a bf16 autocast region computes in float32
    and stores the new conv inputs rounded to bf16.  Checked, batch 16 and 6 tokens, against the
    float64 restatement whose conv state is rounded to bf16 after every update the same way.

    The rounding of a conv input to bf16 may fall on the other side of a rounding boundary in
    float64 than in float32 (rarely): a flipped input moves the logits by ~1e-5 absolute, which
    is outside the bf16 bar (rtol 2e-2 / atol 1e-5) only for logits near zero -- measured 0-2 of
    4,096 per token, so up to 4 per token may sit outside it; the states are held to the bar
    with none outside, and the count outside the float32 bar is printed."""
    from ssm_scan.decode import FastDecoder
    from parity import close, outside
    torch.manual_seed(21)
    model = MambaLM(**shape).to(dev).eval()
    m = model.blocks[0].mixer
    fast = FastDecoder(model)
    B, T = 16, 6
    g = torch.Generator().manual_seed(22)
    states = model.init_state(B, 1, dev, dtype=torch.bfloat16)
    for s_ in states:
        s_.ssm.copy_(torch.randn(s_.ssm.shape, generator=g))
        s_.conv.copy_(torch.randn(s_.conv.shape, generator=g))
    assert states[0].conv.dtype == torch.bfloat16 and states[0].ssm.dtype == torch.float32
    rstates = [{"conv": s_.conv.double().cpu(), "ssm": s_.ssm.double().cpu()} for s_ in states]
    p = {k: v.detach().cpu().double() for k, v in model.state_dict().items()}
    toks = torch.randint(0, 256, (T, B, 1), generator=g)
    for t in range(T):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got = fast.step(toks[t].to(dev), states)
        assert got.dtype == torch.float32
        with torch.no_grad():
            ref = lm_ref.lm_forward(p, toks[t], n_layers=shape["n_layers"], d_state=m.d_state, dt_rank=m.dt_rank,
                                    d_conv=m.d_conv, states=rstates, method=m.discretization)[:, 0]
        for r in rstates:
            r["conv"] = r["conv"].to(torch.bfloat16).double()
        scale = float(ref.abs().max())
        print(f"token {t}: logits outside the float32 bar: {outside(got, ref, 1e-4, 1e-5 * scale)}", flush=True)
        close(got, ref, rtol=2e-2, atol=1e-5, name=f"logits token {t}", allow=4)
    for i, (s_, r) in enumerate(zip(states, rstates)):
        close(s_.ssm, r["ssm"], rtol=2e-2, atol=1e-5, name=f"layer {i} ssm state")
        close(s_.conv.float(), r["conv"], rtol=2e-2, atol=1e-5, name=f"layer {i} conv state")
