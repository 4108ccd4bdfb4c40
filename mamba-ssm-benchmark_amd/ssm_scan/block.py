"""The Mamba (S6) mixer of models/mamba.py on the HIP engine, and the byte-level LM of
models/lm.py restricted to Mamba layers -- the callers of the scan path.

Same parameters (names, shapes, initialization) and the same forward / decode interface as
the reference, so a state_dict moves between the two.  in_proj, x_proj and out_proj are torch GEMMs
(the weight gradients split over the tokens, ssm_scan.linear); the scan-path work runs in the
engine's kernels:
  conv + SiLU                   ssm_scan.conv.causal_conv1d          (models/mamba.py:101-107)
  dt_proj (+ bias, softplus)    fused into the scan kernels' delta   (models/mamba.py:75-76)
                                staging (the step kernel: bias + softplus)
  selective scan, D skip, gate  ssm_scan.selective_scan_fn           (models/mamba.py:120-124)
  decode step                   ssm_scan.ssm_step (state in place)   (models/mamba.py:113-123)

Prefill in pieces (models/lm.py's `model(x[:, p0:p0 + chunk], states, p0)`, as
analysis/length_generalization.py:110-116 streams a long input) carries both the conv state and
the SSM state between calls, so the pieces compute what one call over the whole input does.
Checkpoints written by training/train_lm.py:166 (`{"cfg", "state_dict"}`) load with
`load_checkpoint` when every layer is a Mamba layer.
"""

import math
from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F

from .conv import causal_conv1d
from .hip_scan import selective_scan_fn
from .linear import embedding, linear
from .mixer import mixer, mixer_applies
from .norm import rms_norm
from .scan import selective_scan
from .step import ssm_step


class Mamba(nn.Module):
    """models/mamba.py:26-126 (Mamba) with the scan path on the HIP engine."""

    def __init__(self, d_model, d_state=16, expand=2, d_conv=4, dt_rank=None, selective=True,
                 discretization="zoh", scan="auto", d_block=None, chunk_size=None,
                 dt_min=1e-3, dt_max=0.1, a_mode="s4d"):
        super().__init__()
        self.d_inner = d_inner = expand * d_model
        self.d_state, self.d_conv = d_state, d_conv
        self.dt_rank = dt_rank or math.ceil(d_model / 16)
        self.selective, self.discretization = selective, discretization
        # scan: "auto" / "triton" run the fused kernel (gate and skip inside); a named algorithm
        # of models/scan.py runs that algorithm on the engine with the gate applied after it
        self.scan, self.d_block, self.chunk_size = scan, d_block, chunk_size

        self.in_proj = nn.Linear(d_model, 2 * d_inner, bias=False)
        self.conv = nn.Conv1d(d_inner, d_inner, d_conv, groups=d_inner, bias=True)
        # dt initialized log-uniform in [dt_min, dt_max], stored as softplus^-1 (models/mamba.py:40-42)
        dt = torch.exp(torch.rand(d_inner) * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min))
        dt = dt.clamp(min=1e-4)
        inv_softplus_dt = dt + torch.log(-torch.expm1(-dt))
        if selective:
            self.x_proj = nn.Linear(d_inner, self.dt_rank + 2 * d_state, bias=False)
            self.dt_proj = nn.Linear(self.dt_rank, d_inner, bias=True)
            self.dt_proj._no_reinit = True
            std = self.dt_rank ** -0.5
            with torch.no_grad():
                nn.init.uniform_(self.dt_proj.weight, -std, std)
                self.dt_proj.bias.copy_(inv_softplus_dt)
        else:
            self.dt_bias = nn.Parameter(inv_softplus_dt)
            self.B = nn.Parameter(torch.randn(d_state) / math.sqrt(d_state))
            self.C = nn.Parameter(torch.randn(d_state) / math.sqrt(d_state))
        if a_mode not in ("s4d", "scalar"):
            raise ValueError(f"unknown a_mode {a_mode!r}")
        self.a_mode = a_mode
        if a_mode == "s4d":   # S4D-real: A_n = -(n + 1) for every channel (models/mamba.py:61)
            A = torch.arange(1, d_state + 1, dtype=torch.float32).repeat(d_inner, 1)
        else:                 # one decay per channel shared by the states
            A = torch.empty(d_inner, 1).uniform_(1.0, 16.0)
        self.A_log = nn.Parameter(torch.log(A))
        self.D = nn.Parameter(torch.ones(d_inner))
        self.out_proj = nn.Linear(d_inner, d_model, bias=False)
        self.out_proj._residual_out = True

    def ssm_inputs(self, x, lowrank=False, a_log=False):
        """x (B, L, d_inner) -> raw delta (pre bias/softplus), delta bias, A, B, C (views).
        With lowrank (selective only) the raw delta is the pair (dt (B, L, dt_rank), dt_proj
        weight): the fused kernels apply the projection while they stage delta.  With a_log
        the A returned is A_log itself (the fused kernels form -exp(A_log))."""
        Bsz, L, _ = x.shape
        ct = torch.promote_types(x.dtype, torch.float32)
        if self.selective:
            dt, Bm, Cm = linear(self.x_proj, x).split([self.dt_rank, self.d_state, self.d_state], dim=-1)
            # bias + softplus run in the kernel
            delta = (dt, self.dt_proj.weight) if lowrank else F.linear(dt, self.dt_proj.weight)
            bias = self.dt_proj.bias
        else:
            delta = x.new_zeros(()).expand(Bsz, L, self.d_inner)
            bias = self.dt_bias
            Bm = self.B.to(x.dtype).expand(Bsz, L, -1)
            Cm = self.C.to(x.dtype).expand(Bsz, L, -1)
        A = self.A_log.to(ct) if a_log else -torch.exp(self.A_log.to(ct))
        if self.a_mode == "scalar":
            A = A.expand(-1, self.d_state)
        return delta, bias.to(ct), A, Bm, Cm

    def ssm_params(self, x):
        """models/mamba.py:70-84: x (B, L, d_inner) -> delta (softplus applied), A, B, C.  For
        inspection; the forward hands the projection, bias and softplus to the kernels."""
        delta, bias, A, Bm, Cm = self.ssm_inputs(x)
        return F.softplus(delta.to(bias.dtype) + bias), A, Bm, Cm

    def init_state(self, batch, max_len, device, dtype):
        return SimpleNamespace(
            conv=torch.zeros(batch, self.d_inner, self.d_conv - 1, device=device, dtype=dtype),
            ssm=torch.zeros(batch, self.d_inner, self.d_state, device=device,
                            dtype=torch.promote_types(dtype, torch.float32)),
        )

    @staticmethod
    def state_nbytes(state):
        return state.conv.numel() * state.conv.element_size() + state.ssm.numel() * state.ssm.element_size()

    def _conv(self, x, state):
        if state is None:
            return causal_conv1d(x, self.conv.weight, self.conv.bias)
        if state.conv.dtype == x.dtype:
            return causal_conv1d(x, self.conv.weight, self.conv.bias, state=state.conv)
        # a state kept in another dtype (float32 state under bf16 autocast): the previous
        # inputs are read in x's dtype and the new ones stored back (models/mamba.py:104-106)
        cs = state.conv.to(x.dtype)
        out = causal_conv1d(x, self.conv.weight, self.conv.bias, state=cs)
        state.conv.copy_(cs)
        return out

    def forward(self, u, state=None, pos=0, return_delta=False):
        Bsz, L, _ = u.shape
        if mixer_applies(self, u, state, return_delta):   # one autograd node in_proj -> out_proj
            return linear(self.out_proj, mixer(self, linear(self.in_proj, u)))
        x, z = linear(self.in_proj, u).chunk(2, dim=-1)
        x = self._conv(x, state)
        decode = state is not None and L == 1
        fused = not decode and self.scan in ("auto", "triton")
        delta, bias, A, Bm, Cm = self.ssm_inputs(x, lowrank=fused and self.selective, a_log=fused)
        if return_delta or getattr(self, "record_delta", False):   # models/mamba.py:109-110
            raw = F.linear(*delta) if isinstance(delta, tuple) else delta
            full_delta = F.softplus(raw.to(bias.dtype) + bias)
            if getattr(self, "record_delta", False):
                self.last_delta = full_delta.detach()
        h0 = None if state is None else state.ssm
        if decode:                                                # recurrent decode step
            y = ssm_step(state.ssm, x[:, 0], delta[:, 0], A, Bm[:, 0], Cm[:, 0], D=self.D, z=z[:, 0],
                         delta_bias=bias, delta_softplus=True, method=self.discretization).unsqueeze(1)
        elif fused:
            dt, proj = delta if isinstance(delta, tuple) else (delta, None)
            y, last = selective_scan_fn(x, dt, A, Bm, Cm, D=self.D, z=z, delta_bias=bias, delta_softplus=True,
                                        h0=h0, method=self.discretization, return_last_state=True,
                                        delta_proj=proj, A_is_log=True)
        else:
            y, last = selective_scan(x, F.softplus(delta.to(bias.dtype) + bias), A, Bm, Cm, h0=h0,
                                     method=self.discretization, scan=self.scan, d_block=self.d_block,
                                     chunk_size=self.chunk_size)
            y = (y + x * self.D.to(x.dtype)) * F.silu(z)
        if state is not None and L > 1:
            state.ssm.copy_(last)
        out = linear(self.out_proj, y)
        return (out, full_delta) if return_delta else out


class RMSNorm(nn.Module):
    """models/common.py RMSNorm: x / rms(x) * weight (ssm_scan.norm: one kernel per pass for
    float32 rows)."""

    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        return rms_norm(x, self.weight, self.eps)


class Block(nn.Module):
    """Pre-norm residual Mamba block (models/lm.py:59-89 with kind "M")."""

    def __init__(self, d_model, dropout=0.0, **kw):
        super().__init__()
        self.kind = "M"
        self.norm1 = RMSNorm(d_model)
        self.mixer = Mamba(d_model, **kw)
        self.drop = nn.Dropout(dropout)

    def forward(self, x, state=None, pos=0):
        return x + self.drop(self.mixer(self.norm1(x), state, pos))


# LMConfig fields (models/lm.py:31-55) that shape a Mamba-only LM, with the reference's defaults
_CFG_DEFAULTS = dict(vocab_size=256, d_model=256, dropout=0.0, d_state=16, expand=2, d_conv=4, selective=True,
                     a_mode="s4d", discretization="zoh", scan="auto", d_block=0, chunk_size=0)


class MambaLM(nn.Module):
    """The byte-level LM of models/lm.py with n_layers Mamba blocks and tied embeddings."""

    def __init__(self, n_layers=10, vocab_size=256, d_model=256, d_state=16, expand=2, d_conv=4, dropout=0.0,
                 **kw):
        super().__init__()
        self.n_layers = n_layers
        self.embed = nn.Embedding(vocab_size, d_model)
        self.blocks = nn.ModuleList([Block(d_model, dropout=dropout, d_state=d_state, expand=expand,
                                           d_conv=d_conv, **kw)
                                     for _ in range(n_layers)])
        self.norm_f = RMSNorm(d_model)
        self.head = nn.Linear(d_model, vocab_size, bias=False)
        self.head.weight = self.embed.weight
        self.apply(self._init)

    def _init(self, m):   # models/lm.py:_init
        if isinstance(m, nn.Linear) and not getattr(m, "_no_reinit", False):
            std = 0.02 / math.sqrt(2 * self.n_layers) if getattr(m, "_residual_out", False) else 0.02
            nn.init.normal_(m.weight, 0.0, std)
            if m.bias is not None:
                nn.init.zeros_(m.bias)
        elif isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, 0.0, 0.02)

    def num_params(self, non_embedding=True):
        n = sum(p.numel() for p in self.parameters())
        return n - self.embed.weight.numel() if non_embedding else n

    @classmethod
    def from_config(cls, cfg):
        """Builds the LM an LMConfig dict describes (models/lm.py:31-55, :92-100).  Only layer
        pattern letters "M" are served by this engine; others raise ValueError."""
        cfg = dict(cfg)
        layers = cfg.get("layers", "")
        if not layers or set(layers) != {"M"}:
            raise ValueError(f"only Mamba layers ('M') run on this engine, got layers={layers!r}")
        kw = {k: cfg.get(k, v) for k, v in _CFG_DEFAULTS.items()}
        kw["d_block"] = kw["d_block"] or None
        kw["chunk_size"] = kw["chunk_size"] or None
        return cls(n_layers=len(layers), **kw)

    def init_state(self, batch, max_len, device, dtype=torch.float32):
        return [b.mixer.init_state(batch, max_len, device, dtype) for b in self.blocks]

    @staticmethod
    def state_nbytes(states, length=None):
        """Bytes of the recurrent state (models/lm.py:116-122): constant in the sequence length."""
        return sum(Mamba.state_nbytes(s) for s in states)

    def forward(self, idx, states=None, pos=0):
        x = embedding(self.embed, idx)
        for i, block in enumerate(self.blocks):
            x = block(x, None if states is None else states[i], pos)
        return linear(self.head, self.norm_f(x))

    @torch.no_grad()
    def generate(self, prompt, n_new, temperature=1.0, top_k=None, max_len=None):
        """Autoregressive sampling (models/lm.py:130-147): prefill, then one step per token."""
        Bsz, T = prompt.shape
        states = self.init_state(Bsz, max_len or T + n_new, prompt.device)
        logits = self(prompt, states, 0)[:, -1]
        out = [prompt]
        for t in range(n_new):
            logits = logits.float() / max(temperature, 1e-6)
            if top_k:
                v, _ = torch.topk(logits, top_k)
                logits[logits < v[:, [-1]]] = float("-inf")
            nxt = torch.multinomial(F.softmax(logits, -1), 1)
            out.append(nxt)
            if t < n_new - 1:
                logits = self(nxt, states, T + t)[:, -1]
        return torch.cat(out, 1)


def load_checkpoint(src, device="cpu"):
    """A checkpoint of training/train_lm.py:166 (`{"cfg": LMConfig dict, "state_dict": ...}`, a
    path or the loaded dict) as a MambaLM in eval mode, the way analysis/evaluate_lm.py:26-30
    loads it.  Files are read with torch.load(weights_only=True)."""
    ck = torch.load(src, map_location="cpu", weights_only=True) if isinstance(src, (str, bytes)) or \
        hasattr(src, "read") or hasattr(src, "__fspath__") else src
    model = MambaLM.from_config(ck["cfg"])
    model.load_state_dict(ck["state_dict"])
    return model.to(device).eval()
