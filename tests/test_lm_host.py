"""Host-side LM logic on the CPU (no kernel calls): the reference's checkpoint format
(training/train_lm.py:166, `{"cfg": LMConfig dict, "state_dict"}`) and parameter names
(models/lm.py:92-100, models/mamba.py:26-66, models/common.py:8-16), the config mapping,
and the constant state size of an SSM (tests/test_models.py:82-87)."""

import pytest
import torch

from ssm_scan.block import MambaLM, load_checkpoint


def reference_param_shapes(n_layers, d_model=256, d_state=16, expand=2, d_conv=4, vocab=256):
    """Names and shapes of LM(LMConfig(layers="M" * n)).state_dict(), restated from the
    reference modules (tied head and embedding appear under both names)."""
    di, R = expand * d_model, -(-d_model // 16)
    out = {"embed.weight": (vocab, d_model), "norm_f.weight": (d_model,), "head.weight": (vocab, d_model)}
    for i in range(n_layers):
        p = f"blocks.{i}."
        out.update({p + "norm1.weight": (d_model,), p + "mixer.in_proj.weight": (2 * di, d_model),
                    p + "mixer.conv.weight": (di, 1, d_conv), p + "mixer.conv.bias": (di,),
                    p + "mixer.x_proj.weight": (R + 2 * d_state, di), p + "mixer.dt_proj.weight": (di, R),
                    p + "mixer.dt_proj.bias": (di,), p + "mixer.A_log": (di, d_state), p + "mixer.D": (di,),
                    p + "mixer.out_proj.weight": (d_model, di)})
    return out


def test_state_dict_names_and_shapes_match_reference():
    m = MambaLM(n_layers=3, d_model=64, d_state=8)
    got = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert got == reference_param_shapes(3, d_model=64, d_state=8)


def test_checkpoint_file_loads(tmp_path):
    torch.manual_seed(0)
    cfg = dict(layers="MMMM", vocab_size=256, d_model=64, n_head=4, mlp_ratio=4.0, dropout=0.0,
               attn_impl="manual", pos_encoding="rope", attn_query_chunk=1024, d_state=16, expand=2,
               d_conv=4, selective=True, a_mode="s4d", discretization="bilinear", scan="auto", d_block=0,
               chunk_size=0, retention_chunk=64)
    sd = {k: torch.randn(s) for k, s in reference_param_shapes(4, d_model=64).items()}
    sd["head.weight"] = sd["embed.weight"]
    path = tmp_path / "model.pt"
    torch.save({"cfg": cfg, "state_dict": sd}, path)
    m = load_checkpoint(str(path))
    assert m.n_layers == 4 and not m.training
    assert all(b.mixer.discretization == "bilinear" for b in m.blocks)
    for k, v in m.state_dict().items():
        assert torch.equal(v, sd[k]), k
    assert m.head.weight is m.embed.weight


@pytest.mark.parametrize("layers", ["AAAA", "MMAM", "RR", ""])
def test_non_mamba_layers_are_rejected(layers):
    with pytest.raises(ValueError):
        MambaLM.from_config({"layers": layers})


def test_config_fields_reach_the_mixers():
    m = MambaLM.from_config({"layers": "MM", "d_model": 32, "d_state": 8, "expand": 3, "d_conv": 2,
                             "a_mode": "scalar", "scan": "chunked", "chunk_size": 16, "d_block": 0})
    mx = m.blocks[1].mixer
    assert (mx.d_inner, mx.d_state, mx.d_conv, mx.a_mode) == (96, 8, 2, "scalar")
    assert (mx.scan, mx.chunk_size, mx.d_block) == ("chunked", 16, None)
    assert tuple(mx.A_log.shape) == (96, 1)


def test_state_size_is_constant_in_length():
    m = MambaLM(n_layers=2, d_model=32)
    s1 = MambaLM.state_nbytes(m.init_state(1, 100, "cpu"))
    s2 = MambaLM.state_nbytes(m.init_state(1, 1000, "cpu"))
    assert s1 == s2 == 2 * (64 * 3 + 64 * 16) * 4


@pytest.mark.parametrize("K,splits", [(4096, 8), (4100, 8), (1024, 8), (8192, 1)])
def test_split_k_weight_gradient_equals_the_plain_product(K, splits):
    """dW = dy^T x summed over token slices (ssm_scan.linear) against the plain product, in
    float64: ragged K and small K fall back to the plain product."""
    from ssm_scan.linear import weight_grad
    g = torch.Generator().manual_seed(K)
    dy = torch.randn(K, 48, generator=g, dtype=torch.float64)
    x = torch.randn(K, 40, generator=g, dtype=torch.float64)
    torch.testing.assert_close(weight_grad(dy, x, splits), dy.t() @ x, rtol=1e-12, atol=1e-12)


def test_split_k_linear_gradients_match_nn_linear():
    """The LM's Linear with the split-K weight gradient gives nn.Linear's output and gradients
    (input, weight, bias) in float64."""
    from ssm_scan.linear import linear
    torch.manual_seed(0)
    lin = torch.nn.Linear(40, 48).double()
    x = torch.randn(2, 2048, 40, dtype=torch.float64, requires_grad=True)
    y = linear(lin, x)
    gy = torch.randn_like(y)
    y.backward(gy)
    got = [y.detach(), x.grad.clone(), lin.weight.grad.clone(), lin.bias.grad.clone()]
    x.grad = lin.weight.grad = lin.bias.grad = None
    ref = lin(x)
    ref.backward(gy)
    for a, b in zip(got, [ref.detach(), x.grad, lin.weight.grad, lin.bias.grad]):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_dense_embedding_gradient_on_the_cpu():
    """ssm_scan.linear.embedding: torch's embedding forward, the weight gradient as a one-hot
    product (split over the tokens); equal to torch's gradient to float32 rounding."""
    from ssm_scan.linear import embedding
    torch.manual_seed(0)
    emb = torch.nn.Embedding(300, 24)
    idx = torch.randint(0, 300, (3, 1000))
    gy = torch.randn(3, 1000, 24)
    y = embedding(emb, idx)
    y.backward(gy)
    got = emb.weight.grad.clone()
    emb.weight.grad = None
    emb(idx).backward(gy)
    torch.testing.assert_close(got, emb.weight.grad, rtol=1e-5, atol=1e-5)
    with torch.no_grad():                         # not training: torch's own embedding
        assert torch.equal(embedding(emb, idx), emb(idx))


@pytest.mark.parametrize("method", ["zoh", "bilinear"])
def test_lm_ref_c_oracle_scan_node_matches_time_loop(method):
    """oracle/lm_ref's scan="c" node (each layer's scan, D skip and gate on the C oracle's float64
    forward and adjoint) equals the autograd time loop of the same restatement: the logits and
    every parameter gradient of a 2-layer LM, float64, to 1e-10."""
    from oracle import lm_ref
    torch.manual_seed(3)
    m = MambaLM(n_layers=2, d_model=32, d_state=8)
    sd = m.state_dict()
    g = torch.Generator().manual_seed(4)
    idx = torch.randint(0, 256, (2, 24), generator=g)
    w = torch.randn(2, 24, 256, generator=g, dtype=torch.float64)
    res = []
    for scan in ("loop", "c"):
        p = {k: v.detach().double().requires_grad_() for k, v in sd.items()}
        logits = lm_ref.lm_forward(p, idx, 2, d_state=8, dt_rank=2, method=method, scan=scan)
        (logits * w).sum().backward()
        res.append((logits.detach(), {k: t.grad for k, t in p.items() if t.grad is not None}))
    torch.testing.assert_close(res[1][0], res[0][0], rtol=1e-10, atol=1e-12)
    assert res[0][1].keys() == res[1][1].keys() and len(res[0][1]) == 2 + 2 * 10
    for k, g0 in res[0][1].items():
        torch.testing.assert_close(res[1][1][k], g0, rtol=1e-10, atol=1e-12, msg=k)
