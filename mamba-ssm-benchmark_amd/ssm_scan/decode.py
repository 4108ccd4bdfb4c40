"""Fast recurrent decode of a Mamba LM: three launches per layer.

Per layer the token step is
    xz = u @ (W_in diag(norm_w))^T          one GEMM (the block's RMSNorm weight folded in)
    ssm_decode_step(...)                    one fused launch: RMSNorm scale, conv step + SiLU
                                            with the conv state, x_proj, dt_proj + softplus, the
                                            state update, D skip and SiLU(z) gate
    u += y @ W_out^T                        one GEMM with the residual, in place (addmm_)
which computes what models/mamba.py:93-124 (L = 1 with a state) and the pre-norm residual
block of models/lm.py compute, in place of ~20 small launches per layer.  The step is
allocation-free apart from torch's caching allocator, so it can be captured in a HIP graph.
The folded weights are taken from the model when the decoder is built; call refresh() after
the model's parameters change.
"""

import ctypes

import torch

from . import _abi
from .hip_scan import METHODS


class FastDecoder:
    def __init__(self, model):
        if next(model.parameters()).dtype != torch.float32:
            raise ValueError("the fused decode layer runs in float32")
        self.model = model
        self.refresh()

    @torch.no_grad()
    def refresh(self):
        self.layers = []
        for blk in self.model.blocks:
            m = blk.mixer
            if not m.selective:
                raise ValueError("the fused decode layer needs a selective mixer")
            self.layers.append(dict(
                w_in=(m.in_proj.weight * blk.norm1.weight[None, :]).contiguous(),
                conv_w=m.conv.weight.reshape(m.d_inner, m.d_conv).contiguous(),
                conv_b=m.conv.bias.contiguous(),
                x_proj_wt=m.x_proj.weight.t().contiguous(),
                dt_proj_w=m.dt_proj.weight.contiguous(),
                dt_bias=m.dt_proj.bias.contiguous(),
                A_log=m.A_log.expand(m.d_inner, m.d_state).contiguous(),
                Dskip=m.D.contiguous(),
                w_out_t=m.out_proj.weight.t(),
                eps=blk.norm1.eps, mixer=m))

    def _layer(self, L, u, state):
        m = L["mixer"]
        Bsz = u.shape[0]
        xz = torch.mm(u, L["w_in"].t())
        y = torch.empty(Bsz, m.d_inner, dtype=u.dtype, device=u.device)
        a = _abi.DecodeArgs()
        a.batch, a.dim, a.dstate, a.width = Bsz, m.d_inner, m.d_state, m.d_conv
        a.dt_rank, a.d_model = m.dt_rank, u.shape[1]
        a.method = METHODS[m.discretization]
        a.eps = L["eps"]
        a.u, a.xz, a.conv_w, a.conv_b = u.data_ptr(), xz.data_ptr(), L["conv_w"].data_ptr(), L["conv_b"].data_ptr()
        a.conv_state = state.conv.data_ptr()
        a.conv_state_dtype = _abi.DTYPE_CODE[state.conv.dtype]
        a.x_proj_wt, a.dt_proj_w, a.dt_bias = L["x_proj_wt"].data_ptr(), L["dt_proj_w"].data_ptr(), L["dt_bias"].data_ptr()
        a.A_log, a.Dskip = L["A_log"].data_ptr(), L["Dskip"].data_ptr()
        a.ssm_state, a.y = state.ssm.data_ptr(), y.data_ptr()
        rc = _abi.lib().ssm_decode_step(ctypes.byref(a), _abi.stream_handle(u.device))
        _abi.check(rc, "ssm_decode_step")
        return u.addmm_(y, L["w_out_t"])     # residual in place: u is this step's own buffer

    @torch.no_grad()
    def step(self, tok, states):
        """tok (B,) or (B, 1) byte ids; states from model.init_state, contiguous, updated in
        place: the SSM state float32, the conv state float32 or bf16 (the states of a model run
        under bf16 autocast, models/mamba.py:86-91; the new conv inputs are stored rounded to
        bf16).  Returns float32 logits (B, V).  The step computes in float32 also inside a bf16
        autocast region (its results then differ from the autocast path's by the latter's bf16
        rounding).

        The decode GEMMs are skinny (B rows); they are issued through rocBLAS, whose kernels
        for these shapes take a fraction of hipBLASLt's (torch's default), and torch's choice
        is restored afterwards."""
        for s in states:
            if not (s.conv.is_contiguous() and s.ssm.is_contiguous() and s.ssm.dtype == torch.float32
                    and s.conv.dtype in (torch.float32, torch.bfloat16)):
                raise ValueError("decode states must be contiguous: ssm float32, conv float32 or bf16")
        prev = torch.backends.cuda.preferred_blas_library()
        torch.backends.cuda.preferred_blas_library("cublas")   # rocBLAS on ROCm
        try:
            with torch.autocast(device_type="cuda", enabled=False):
                u = self.model.embed(tok.reshape(-1))      # a fresh buffer, updated in place
                for L, s in zip(self.layers, states):
                    u = self._layer(L, u, s)
                return self.model.head(self.model.norm_f(u))
        finally:
            torch.backends.cuda.preferred_blas_library(prev)
