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
