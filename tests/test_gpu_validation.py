"""Host-side argument checks of the Python entry points that launch kernels: the C ABI takes
pointers and strides, so every operand's shape (and device) is checked against the dimensions
the kernels are given before anything is launched.  Each case here is rejected on the host;
no kernel runs with the bad operand."""

import pytest
import torch

from ssm_scan.block import MambaLM
from ssm_scan.decode import FastDecoder
from ssm_scan.norm import rms_norm
from ssm_scan.scan import discretize
from ssm_scan.step import ssm_step

pytestmark = pytest.mark.gpu


def _step_operands(dev, B=3, D=8, N=4):
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(dev)
    return dict(h=mk(B, D, N), x=mk(B, D), delta=mk(B, D).abs(), A=-mk(D, N).abs(), Bm=mk(B, N), Cm=mk(B, N),
                D=mk(D), z=mk(B, D), delta_bias=mk(D))


@pytest.mark.parametrize("name,shape", [("delta", (3, 7)), ("A", (8, 5)), ("Bm", (2, 4)), ("Cm", (3, 5)),
                                        ("D", (7,)), ("z", (3, 9)), ("delta_bias", (9,)), ("h", (3, 8, 5))])
def test_step_rejects_mismatched_operands(dev, name, shape):
    ops = _step_operands(dev)
    ops[name] = torch.zeros(shape, device=dev)
    with pytest.raises(ValueError):
        ssm_step(ops.pop("h"), ops.pop("x"), ops.pop("delta"), ops.pop("A"), ops.pop("Bm"), ops.pop("Cm"), **ops)


def test_rms_norm_rejects_a_short_weight(dev):
    with pytest.raises(ValueError):
        rms_norm(torch.randn(4, 64, device=dev), torch.ones(32, device=dev))


@pytest.mark.parametrize("name", ["delta", "A", "Bm"])
def test_discretize_rejects_mismatched_operands(dev, name):
    ops = dict(delta=torch.rand(2, 5, 8, device=dev), A=-torch.rand(8, 4, device=dev),
               Bm=torch.randn(2, 5, 4, device=dev), x=torch.randn(2, 5, 8, device=dev))
    ops[name] = ops[name][..., :-1]
    with pytest.raises(ValueError):
        discretize(ops["delta"], ops["A"], ops["Bm"], ops["x"])


@pytest.mark.parametrize("path", ["stack", "block"])
def test_decoder_rejects_states_that_do_not_match_the_tokens(dev, path):
    """States sized for another batch, a missing block's state or tokens on the host are
    rejected before the step launches anything (the kernels size every state buffer from the
    token count)."""
    model = MambaLM(n_layers=2).to(dev).eval()
    fast = FastDecoder(model, path=path)
    tok = torch.zeros(4, 1, dtype=torch.long, device=dev)
    with pytest.raises(ValueError):
        fast.step(tok, model.init_state(3, 1, dev))
    with pytest.raises(ValueError):
        fast.step(tok, model.init_state(4, 1, dev)[:1])
    with pytest.raises(RuntimeError):
        fast.step(tok.cpu(), model.init_state(4, 1, dev))


def test_decoder_reads_a_strided_token_view(dev):
    """A strided view of token ids (a column of a (B, T) prompt) gives the step of its
    contiguous copy, bit for bit."""
    model = MambaLM(n_layers=2).to(dev).eval()
    fast = FastDecoder(model, path="stack")
    prompt = torch.randint(0, 256, (5, 7), generator=torch.Generator().manual_seed(1)).to(dev)
    s1, s2 = model.init_state(5, 1, dev), model.init_state(5, 1, dev)
    got = fast.step(prompt[:, 3], s1)
    ref = fast.step(prompt[:, 3].contiguous(), s2)
    assert torch.equal(got, ref)
    for a, b in zip(s1, s2):
        assert torch.equal(a.ssm, b.ssm) and torch.equal(a.conv, b.conv)
