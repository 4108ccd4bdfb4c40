"""The LM's Linear layers (in_proj, x_proj, out_proj, the tied head) with a split-K weight
gradient, and its token embedding with a dense weight gradient.

A Linear layer's weight gradient is dW = dY^T X, contracted over the tokens (B * L of them).
At config 3 (8,192 tokens) the library GEMM for the layers' (out, in) shapes (1024, 256),
(256, 512), (48, 512) and (256, 256) tiles only the small output -- 32 to 256 workgroups on
256 CUs -- and walks all 8,192 tokens inside each tile.  Splitting the tokens into S slices,
S independent products in one batched GEMM followed by a fixed-order sum over the slices,
fills the GPU: on one MI355X (float32) 45 / 26 / 26 / 25 us against 60 / 55 / 45 / 53 us.
The forward and the input gradient stay the plain GEMMs of F.linear; the parameters are the
nn.Linear modules' own (models/mamba.py, models/lm.py use nn.Linear).
"""

import torch
import torch.nn.functional as F

SPLITS = 8          # token slices of the weight gradient
MIN_TOKENS = 2048   # below this the plain product already fills the GPU as well

_get_blas = getattr(torch._C, "_get_blas_preferred_backend", None)
_set_blas = getattr(torch._C, "_set_blas_preferred_backend", None)
_ROCBLAS = torch._C._BlasBackend.Cublas if hasattr(torch._C, "_BlasBackend") else None  # rocBLAS on ROCm


class rocblas:
    """Within the block torch's GEMMs go to rocBLAS (the previous choice is restored after).
    For the LM's GEMMs (thousands of tokens, widths 48 to 1024) rocBLAS's kernels take about
    the GPU time of hipBLASLt's, torch's default on ROCm, while its host cost per call is a
    fraction of it; the eager config-3 training step is bound by the host issuing its ~300
    launches, and went from 7.3 to 5.7 ms per step (GPU time 5.30 -> 5.36 ms)."""

    __slots__ = ("prev",)

    def __enter__(self):
        self.prev = _get_blas() if _get_blas is not None and _ROCBLAS is not None else _ROCBLAS
        if self.prev != _ROCBLAS:
            _set_blas(_ROCBLAS)
        return self

    def __exit__(self, *exc):
        if self.prev != _ROCBLAS:
            _set_blas(self.prev)
        return False


def weight_grad(dy, x, splits=SPLITS):
    """dy (K, O), x (K, I) -> dy^T x (O, I).  Split over K when K is a multiple of `splits`
    and at least MIN_TOKENS; the slices' products are summed in slice order."""
    K = dy.shape[0]
    if splits <= 1 or K % splits or K < MIN_TOKENS:
        return dy.t() @ x
    kc = K // splits
    a = dy.reshape(splits, kc, dy.shape[1]).transpose(1, 2)   # (S, O, kc)
    b = x.reshape(splits, kc, x.shape[1]).contiguous()         # (S, kc, I), right operand dense
    return torch.bmm(a, b).sum(0)


class _SplitKLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        with rocblas():
            return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1])
        dx = dw = db = None
        with rocblas():
            if ctx.needs_input_grad[0]:
                dx = (dy2 @ w).reshape(x.shape)
            if ctx.needs_input_grad[1]:
                dw = weight_grad(dy2, x.reshape(-1, x.shape[-1]))
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = dy2.sum(0)
        return dx, dw, db


def linear(layer, x):
    """layer(x) for an nn.Linear; while its weight is trained on at least MIN_TOKENS tokens
    (grad mode, no autocast, matching dtypes) the weight gradient is the split-K product."""
    w = layer.weight
    if (torch.is_grad_enabled() and w.requires_grad and not torch.is_autocast_enabled(x.device.type)
            and x.dtype == w.dtype and x.numel() // max(x.shape[-1], 1) >= MIN_TOKENS):
        return _SplitKLinear.apply(x, w, layer.bias)
    with rocblas():
        return layer(x)


MAX_DENSE_VOCAB = 4096  # vocabularies up to this size take the one-hot product


class _DenseGradEmbedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, idx, weight):
        ctx.save_for_backward(idx)
        ctx.vocab = weight.shape[0]
        return F.embedding(idx, weight)

    @staticmethod
    def backward(ctx, dy):
        (idx,) = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1])
        classes = torch.arange(ctx.vocab, device=idx.device)
        onehot = (idx.reshape(-1, 1) == classes).to(dy2.dtype)   # (tokens, vocab)
        with rocblas():
            return None, weight_grad(onehot, dy2)


def embedding(layer, idx):
    """layer(idx) for a plain nn.Embedding.  While it is trained (grad mode, float32, vocabulary
    <= MAX_DENSE_VOCAB) the weight gradient is onehot(idx)^T dY, a dense product (split-K over
    the tokens): the same sums as torch's embedding backward, which sorts the indices with
    sizes it reads back on the host -- this one makes no host reads, so a training step that
    contains it can be captured in a HIP graph, and it runs in a fixed order."""
    w = layer.weight
    plain = (layer.padding_idx is None and layer.max_norm is None and not layer.scale_grad_by_freq
             and not layer.sparse)
    if (plain and torch.is_grad_enabled() and w.requires_grad and w.dtype == torch.float32
            and w.shape[0] <= MAX_DENSE_VOCAB and not torch.is_autocast_enabled(w.device.type)):
        return _DenseGradEmbedding.apply(idx, w)
    return layer(idx)
