"""torch-CPU restatement of the reference's CPU scan path -- bench.py's cpu_baseline only.

On a CPU tensor the reference's selective_scan(scan="auto") resolves to "chunked"
(models/scan.py:286-287,314): SelectiveScanFn (models/scan.py:193-255) over channel tiles of
d_block = max(1, 2^24 // (B L N)) (:182-190), each tile discretized (:39-55), scanned with
scan_chunked (:142-165, chunk = default_chunk(L), Hillis-Steele over chunk ends :87-98),
contracted with C, and a custom backward that recomputes states and runs the reverse scan.
The D skip and SiLU gate of models/mamba.py:124 are applied outside with torch autograd, as
there.  This file is test infrastructure: it is timed as the CPU baseline and never shipped.
"""

import math

import torch


def discretize(delta, A, Bm, x):
    """models/scan.py:39-49 (zoh)."""
    dA = delta.unsqueeze(-1) * A
    Bx = x.unsqueeze(-1) * Bm.unsqueeze(2)
    return torch.exp(dA), torch.expm1(dA) / A * Bx


def hillis_steele(a, b, h0=None):
    """models/scan.py:79-98."""
    if h0 is not None:
        b = b.clone()
        b[:, 0] = b[:, 0] + a[:, 0] * h0
    L = a.shape[1]
    off = 1
    while off < L:
        b = torch.cat([b[:, :off], torch.addcmul(b[:, off:], a[:, off:], b[:, :-off])], 1)
        if off * 2 < L:
            a = torch.cat([a[:, :off], a[:, off:] * a[:, :-off]], 1)
        off *= 2
    return b


def default_chunk(L):
    return max(4, 1 << math.ceil(math.log2(max(1.0, math.sqrt(L)))))     # models/scan.py:138-139


def scan_chunked(a, b, h0=None):
    """models/scan.py:142-165."""
    B, L = a.shape[:2]
    rest = a.shape[2:]
    C = default_chunk(L)
    nc = -(-L // C)
    if nc * C != L:
        pad = (B, nc * C - L) + rest
        a = torch.cat([a, torch.ones(pad, dtype=a.dtype)], 1)
        b = torch.cat([b, torch.zeros(pad, dtype=b.dtype)], 1)
    a4 = a.reshape((B, nc, C) + rest)
    b4 = b.reshape((B, nc, C) + rest)
    h = torch.empty_like(b4)
    h[:, :, 0] = b4[:, :, 0]
    for t in range(1, C):
        h[:, :, t] = torch.addcmul(b4[:, :, t], a4[:, :, t], h[:, :, t - 1])
    P = torch.cumprod(a4, dim=2)
    h_end = hillis_steele(P[:, :, -1], h[:, :, -1], h0)
    zero = torch.zeros_like(h_end[:, :1]) if h0 is None else h0.unsqueeze(1)
    h_in = torch.cat([zero, h_end[:, :-1]], 1)
    h.addcmul_(P, h_in.unsqueeze(2))
    return h.reshape((B, nc * C) + rest)[:, :L]


def _blocks(Bsz, L, D, N):
    d_block = min(D, max(1, (1 << 24) // (Bsz * L * N)))                # models/scan.py:185-190
    return [(i, min(i + d_block, D)) for i in range(0, D, d_block)]


class ChunkedScanFn(torch.autograd.Function):
    """models/scan.py:193-255 with scan = scan_chunked, method = zoh, h0 = None."""

    @staticmethod
    def forward(ctx, x, delta, A, Bm, Cm):
        Bsz, L, D = x.shape
        y = torch.empty_like(x)
        for i, j in _blocks(Bsz, L, D, A.shape[1]):
            a, b = discretize(delta[..., i:j], A[i:j], Bm, x[..., i:j])
            h = scan_chunked(a, b)
            y[..., i:j] = torch.einsum("bldn,bln->bld", h, Cm)
        ctx.save_for_backward(x, delta, A, Bm, Cm)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, delta, A, Bm, Cm = ctx.saved_tensors
        dx, ddelta, dA = torch.zeros_like(x), torch.zeros_like(delta), torch.zeros_like(A)
        dBm, dCm = torch.zeros_like(Bm), torch.zeros_like(Cm)
        Bsz, L, D = x.shape
        for i, j in _blocks(Bsz, L, D, A.shape[1]):
            with torch.enable_grad():
                ins = [t.detach().requires_grad_() for t in (delta[..., i:j], A[i:j], Bm, x[..., i:j])]
                a, b = discretize(*ins)
            with torch.no_grad():
                h = scan_chunked(a.detach(), b.detach())
                dy_blk = dy[..., i:j]
                dCm += torch.einsum("bld,bldn->bln", dy_blk, h)
                g = dy_blk.unsqueeze(-1) * Cm.unsqueeze(2)
                a_next = torch.cat([a.detach()[:, 1:], torch.ones_like(a[:, :1])], 1)
                dh = scan_chunked(a_next.flip(1), g.flip(1)).flip(1)
                h_prev = torch.cat([torch.zeros_like(h[:, :1]), h[:, :-1]], 1)
                da = dh * h_prev
            g_delta, g_A, g_B, g_x = torch.autograd.grad((a, b), ins, (da, dh))
            ddelta[..., i:j] = g_delta
            dA[i:j] = g_A
            dBm += g_B
            dx[..., i:j] = g_x
        return dx, ddelta, dA, dBm, dCm


def fwd_bwd(x, delta, A, Bm, Cm, Dv, z, dy):
    """One training step of the scan block: out = (y + D x) * silu(z); returns the grads."""
    leaves = [t.detach().requires_grad_() for t in (x, delta, A, Bm, Cm, Dv, z)]
    y = ChunkedScanFn.apply(*leaves[:5])
    out = (y + leaves[0] * leaves[5]) * torch.nn.functional.silu(leaves[6])
    return torch.autograd.grad(out, leaves, dy)


def fwd(x, delta, A, Bm, Cm):
    with torch.no_grad():
        return ChunkedScanFn.apply(x, delta, A, Bm, Cm)
