"""Fast recurrent decode of a Mamba LM.

The whole token step runs as one C-ABI call (ssm_decode_stack): per block two launches spread
over the whole GPU (block 0's first reads the tokens' embedding rows),
    in-stage      the residual stream rebuilt from the previous block's out_proj partial sums,
                  the RMSNorm scale, the in_proj GEMM tile (the norm weight folded into its
                  columns), conv step + SiLU with the conv state, the SiLU(z) gate, x_proj
                  partial sums
    scan-stage    x_proj sums finished, dt_proj + softplus, the state update, D skip and gate,
                  out_proj partial sums
and one launch at the end for the last block's sums, the final RMSNorm and the head (its weight
with the norm's folded in); which computes what models/lm.py:124-128 computes at L = 1 with
states (the blocks :82-83, the mixer models/mamba.py:93-124), in place of ~20 small launches
per block.  Shapes past the stack kernels' limits (d_model > 512 or not a multiple of 4,
dim > 1024, dstate not 8 or 16, dt_rank not 8, 16 or 32, conv width > 4) take the per-block
path: three launches per block,
    xz = u @ (W_in diag(norm_w))^T          one GEMM (the block's RMSNorm weight folded in)
    ssm_decode_step(...)                    one fused launch: RMSNorm scale, conv step + SiLU,
                                            x_proj, dt_proj + softplus, the state update, D
                                            skip and SiLU(z) gate
    u += y @ W_out^T                        one GEMM with the residual, in place (addmm_)
The step is allocation-free apart from torch's caching allocator, so it can be captured in a
HIP graph.  The folded weights are taken from the model when the decoder is built; call
refresh() after the model's parameters change.
"""

import ctypes

import torch

from . import _abi
from .hip_scan import METHODS, _require_gpu


STACK_LIMITS = dict(d_model=512, dim=1024, dstate=(8, 16), dt_rank=(8, 16, 32), width=4)


def _four_k(w):
    """(n, k) weight -> (k / 4, n, 4): element [g][c][j] = w[c][4 g + j] (four consecutive k of a
    column in 16 bytes), the layout the stack kernels read; k a multiple of 4."""
    n, k = w.shape
    return w.reshape(n, k // 4, 4).permute(1, 0, 2).contiguous()


class FastDecoder:
    def __init__(self, model, path="auto"):
        """path: "auto" (the stack path where the shape allows it), "stack" or "block"."""
        if next(model.parameters()).dtype != torch.float32:
            raise ValueError("the fused decode layer runs in float32")
        if path not in ("auto", "stack", "block"):
            raise ValueError(f"unknown decode path {path!r}")
        self.model = model
        m0 = model.blocks[0].mixer
        dm = model.blocks[0].norm1.weight.numel()
        fits = (dm <= STACK_LIMITS["d_model"] and dm % 4 == 0 and m0.d_inner <= STACK_LIMITS["dim"]
                and m0.d_inner % 4 == 0
                and m0.d_state in STACK_LIMITS["dstate"] and m0.dt_rank in STACK_LIMITS["dt_rank"]
                and m0.d_conv <= STACK_LIMITS["width"])
        if path == "stack" and not fits:
            raise ValueError("the model's shape is past the stack decode kernels' limits")
        self.path = "stack" if (path == "stack" or (path == "auto" and fits)) else "block"
        self._ws = {}
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
            if self.path == "stack":
                L = self.layers[-1]
                L["w_in4"] = _four_k(L["w_in"])
                L["w_out4"] = _four_k(m.out_proj.weight)
        if self.path == "stack":  # the head with the final RMSNorm weight folded into its columns
            self.head_w4 = _four_k(self.model.head.weight * self.model.norm_f.weight[None, :])

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

    def _stack(self, tok, states):
        """The whole token step in one call: embedding rows, every block, the final norm and
        the head; returns the logits."""
        m = self.layers[0]["mixer"]
        B, dm, V = tok.numel(), self.model.head.weight.shape[1], self.model.head.weight.shape[0]
        tok = tok.reshape(-1).to(torch.long).contiguous()  # a strided view of ids is copied
        u = torch.empty(B, dm, dtype=torch.float32, device=tok.device)
        logits = torch.empty(B, V, dtype=torch.float32, device=tok.device)
        n = len(self.layers)
        blocks = (_abi.DecodeBlock * n)()
        for i, (L, st) in enumerate(zip(self.layers, states)):
            k = blocks[i]
            k.w_in4, k.conv_w, k.conv_b = L["w_in4"].data_ptr(), L["conv_w"].data_ptr(), L["conv_b"].data_ptr()
            k.x_proj_wt, k.dt_proj_w = L["x_proj_wt"].data_ptr(), L["dt_proj_w"].data_ptr()
            k.dt_bias, k.A_log, k.Dskip = L["dt_bias"].data_ptr(), L["A_log"].data_ptr(), L["Dskip"].data_ptr()
            k.w_out4 = L["w_out4"].data_ptr()
            k.conv_state, k.ssm_state = st.conv.data_ptr(), st.ssm.data_ptr()
            k.eps = L["eps"]
        a = _abi.DecodeStackArgs()
        a.batch, a.dim, a.dstate, a.width = u.shape[0], m.d_inner, m.d_state, m.d_conv
        a.dt_rank, a.d_model = m.dt_rank, u.shape[1]
        a.method = METHODS[m.discretization]
        a.conv_state_dtype = _abi.DTYPE_CODE[states[0].conv.dtype]
        a.n_blocks = n
        a.blocks = blocks
        a.u = u.data_ptr()
        a.tokens, a.embed = tok.data_ptr(), self.model.embed.weight.data_ptr()
        a.head_w4, a.logits, a.vocab = self.head_w4.data_ptr(), logits.data_ptr(), V
        a.head_eps = self.model.norm_f.eps
        lib = _abi.lib()
        need = lib.ssm_decode_stack_workspace_bytes(ctypes.byref(a))
        key = (u.device, need)
        if key not in self._ws:
            ws = torch.empty(need, dtype=torch.uint8, device=u.device)
            off = lib.ssm_decode_stack_status_offset(ctypes.byref(a))
            status = ws[off:off + 4].view(torch.int32)
            status.zero_()            # the library sets it, never clears it
            self._ws[key] = (ws, status)
        ws = self._ws[key][0]
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
        _abi.check(lib.ssm_decode_stack(ctypes.byref(a), _abi.stream_handle(u.device)), "ssm_decode_stack")
        return logits

    def _check(self, tok, states):
        """Host-side checks before any launch: the kernels size every state buffer from the
        token count and the model's dimensions."""
        dev = self.layers[0]["w_in"].device
        _require_gpu(self.layers[0]["w_in"], tok, *[t for s in states for t in (s.conv, s.ssm)])
        B = tok.numel()
        if tok.device != dev:
            raise ValueError(f"tokens on {tok.device}, the model on {dev}")
        if len(states) != len(self.layers):
            raise ValueError(f"{len(states)} states for {len(self.layers)} blocks")
        for i, (L, s) in enumerate(zip(self.layers, states)):
            m = L["mixer"]
            want_ssm, want_conv = (B, m.d_inner, m.d_state), (B, m.d_inner, m.d_conv - 1)
            if tuple(s.ssm.shape) != want_ssm or tuple(s.conv.shape) != want_conv:
                raise ValueError(f"block {i}: states {tuple(s.ssm.shape)} / {tuple(s.conv.shape)}, expected "
                                 f"{want_ssm} / {want_conv} for {B} tokens")
            if s.ssm.device != dev or s.conv.device != dev:
                raise ValueError(f"block {i}: states on {s.ssm.device} / {s.conv.device}, the model on {dev}")
            if not (s.conv.is_contiguous() and s.ssm.is_contiguous() and s.ssm.dtype == torch.float32
                    and s.conv.dtype in (torch.float32, torch.bfloat16)):
                raise ValueError("decode states must be contiguous: ssm float32, conv float32 or bf16")

    def _check_ids(self, tok):
        """The reference's nn.Embedding raises on ids outside the vocabulary (models/lm.py:125).
        Both paths check the ids on the host before any launch (a host read of the ids)."""
        V = self.model.embed.weight.shape[0]
        bad = (tok < 0) | (tok >= V)
        if bool(bad.any()):
            raise IndexError(f"token id outside the vocabulary [0, {V}): {tok[bad].reshape(-1)[:8].tolist()}")

    def bad_tokens_seen(self, clear=True):
        """Whether a stack-path step since the last clear read a token id outside the vocabulary
        (its embedding row read as zeros): the status word ssm_decode_stack raises on the device,
        read here with one host synchronization; `clear` zeroes it again."""
        seen = False
        for _, status in self._ws.values():
            if bool(status.item()):
                seen = True
                if clear:
                    status.zero_()
        return seen

    @torch.no_grad()
    def step(self, tok, states, check_ids=False):
        """tok (B,) or (B, 1) byte ids; states from model.init_state, contiguous, updated in
        place: the SSM state float32, the conv state float32 or bf16 (the states of a model run
        under bf16 autocast, models/mamba.py:86-91; the new conv inputs are stored rounded to
        bf16).  Returns float32 logits (B, V).  The step computes in float32 also inside a bf16
        autocast region (its results then differ from the autocast path's by the latter's bf16
        rounding).  With check_ids, ids outside the vocabulary raise IndexError before any launch
        (one host read of the ids); without it the stack path reads a zero embedding row for
        them and raises the status word that bad_tokens_seen() reports.

        The decode GEMMs are skinny (B rows); they are issued through rocBLAS, whose kernels
        for these shapes take a fraction of hipBLASLt's (torch's default), and torch's choice
        is restored afterwards."""
        self._check(tok, states)
        if check_ids:
            self._check_ids(tok)
        prev = torch.backends.cuda.preferred_blas_library()
        torch.backends.cuda.preferred_blas_library("cublas")   # rocBLAS on ROCm
        try:
            with torch.autocast(device_type="cuda", enabled=False):
                if self.path == "stack":
                    if len({s.conv.dtype for s in states}) != 1:
                        raise ValueError("the stack path needs one conv state dtype for every block")
                    return self._stack(tok, states)
                u = self.model.embed(tok.reshape(-1))      # a fresh buffer, updated in place
                for L, s in zip(self.layers, states):
                    u = self._layer(L, u, s)
                return self.model.head(self.model.norm_f(u))
        finally:
            torch.backends.cuda.preferred_blas_library(prev)
