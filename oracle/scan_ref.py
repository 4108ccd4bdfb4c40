"""float64 numpy restatement of the reference selective scan (test infrastructure only).

Every function cites the reference file:line it restates.  Arrays use the
reference's logical layouts: x, delta, z, y (B, L, D); A (D, N); Bm, Cm (B, L, N);
h0 / last (B, D, N).  All arithmetic is float64.
"""

import math

import numpy as np

DISCRETIZATIONS = ("zoh", "euler", "bilinear")          # models/scan.py:36
METHODS = {"zoh": 0, "euler": 1, "bilinear": 2}         # kernels/triton_scan.py:23-24
SCAN_NAMES = ("reference", "sequential", "hillis_steele", "blelloch", "chunked", "triton", "auto")
SCAN_ELEMENT_BUDGET = 1 << 24                           # models/scan.py:182
BLOCK_D = 16                                            # kernels/triton_scan.py:231
HBUF_BUDGET = 1 << 27                                   # kernels/triton_scan.py:242


# ----------------------------------------------------------------------------- discretization

def discretize(delta, A, Bm, x, method="zoh"):
    """models/scan.py:39-55.  delta, x (B, L, D); A (D, N); Bm (B, L, N) -> a, b (B, L, D, N)."""
    dA = delta[..., None] * A
    Bx = x[..., None] * Bm[:, :, None, :]
    if method == "zoh":
        return np.exp(dA), np.expm1(dA) / A * Bx
    if method == "euler":
        return np.exp(dA), delta[..., None] * Bx
    if method == "bilinear":
        inv = 1.0 / (1.0 - 0.5 * dA)
        return (1.0 + 0.5 * dA) * inv, delta[..., None] * inv * Bx
    raise ValueError(f"unknown discretization {method!r}")


def zoh_matrix(A, B, delta):
    """models/scan.py:58-62: dense ZOH  Ad = expm(A delta),  Bd = A^{-1} (Ad - I) B."""
    from scipy.linalg import expm
    Ad = expm(A * delta)
    return Ad, np.linalg.solve(A, (Ad - np.eye(A.shape[0])) @ B)


# ----------------------------------------------------------------------------- scan algorithms

def scan_sequential(a, b, h0=None):
    """models/scan.py:70-76."""
    h = np.zeros_like(b[:, 0]) if h0 is None else h0
    out = np.empty_like(b)
    for t in range(a.shape[1]):
        h = a[:, t] * h + b[:, t]
        out[:, t] = h
    return out


def _fold_h0(a, b, h0):
    """models/scan.py:79-84."""
    if h0 is None:
        return b
    b = b.copy()
    b[:, 0] = b[:, 0] + a[:, 0] * h0
    return b


def scan_hillis_steele(a, b, h0=None):
    """models/scan.py:87-98: recursive doubling; after step k position t holds the
    composition of the 2^k elements ending at t."""
    b = _fold_h0(a, b, h0)
    L = a.shape[1]
    off = 1
    while off < L:
        b = np.concatenate([b[:, :off], b[:, off:] + a[:, off:] * b[:, :-off]], 1)
        if off * 2 < L:
            a = np.concatenate([a[:, :off], a[:, off:] * a[:, :-off]], 1)
        off *= 2
    return b


def scan_blelloch(a, b, h0=None):
    """models/scan.py:101-135: pad to a power of two with (1, 0), up-sweep, down-sweep
    from the identity, exclusive prefixes (A_t, S_t), then h = a * (A_t h0 + S_t) + b."""
    Bsz, L = a.shape[:2]
    rest = a.shape[2:]
    P = 1 << (L - 1).bit_length()
    Ap = np.ones((Bsz, P) + rest)
    Sp = np.zeros((Bsz, P) + rest)
    Ap[:, :L] = a
    Sp[:, :L] = b
    s = 2
    while s <= P:                      # up-sweep: right <- right o left
        for i in range(s - 1, P, s):
            l = i - s // 2
            Sp[:, i] = Ap[:, i] * Sp[:, l] + Sp[:, i]
            Ap[:, i] = Ap[:, i] * Ap[:, l]
        s *= 2
    Ap[:, P - 1] = 1.0
    Sp[:, P - 1] = 0.0
    s = P
    while s >= 2:                      # down-sweep: left <- right; right <- left_old o right
        for i in range(s - 1, P, s):
            l = i - s // 2
            tA, tS = Ap[:, l].copy(), Sp[:, l].copy()
            Ap[:, l], Sp[:, l] = Ap[:, i].copy(), Sp[:, i].copy()
            Sp[:, i] = Sp[:, i] * tA + tS
            Ap[:, i] = Ap[:, i] * tA
        s //= 2
    prev = Sp[:, :L] if h0 is None else Sp[:, :L] + Ap[:, :L] * h0[:, None]
    return b + a * prev


def default_chunk(L):
    """models/scan.py:138-139 (floating-point form, exactly as written there)."""
    return max(4, 1 << math.ceil(math.log2(max(1.0, math.sqrt(L)))))


def scan_chunked(a, b, h0=None, chunk_size=None):
    """models/scan.py:142-165: sequential inside chunks of C, Hillis-Steele over chunk
    ends (with h0), then h += P * h_in.  Ragged L is padded with (1, 0)."""
    Bsz, L = a.shape[:2]
    rest = a.shape[2:]
    C = chunk_size or default_chunk(L)
    nc = -(-L // C)
    if nc * C != L:
        pad = (Bsz, nc * C - L) + rest
        a = np.concatenate([a, np.ones(pad)], 1)
        b = np.concatenate([b, np.zeros(pad)], 1)
    a4 = a.reshape((Bsz, nc, C) + rest)
    b4 = b.reshape((Bsz, nc, C) + rest)
    h = np.empty_like(b4)
    h[:, :, 0] = b4[:, :, 0]
    for t in range(1, C):
        h[:, :, t] = b4[:, :, t] + a4[:, :, t] * h[:, :, t - 1]
    P = np.cumprod(a4, axis=2)
    h_end = scan_hillis_steele(P[:, :, -1], h[:, :, -1], h0)
    zero = np.zeros_like(h_end[:, :1]) if h0 is None else h0[:, None]
    h_in = np.concatenate([zero, h_end[:, :-1]], 1)
    h = h + P * h_in[:, :, None]
    return h.reshape((Bsz, nc * C) + rest)[:, :L]


SCANS = {"sequential": scan_sequential, "hillis_steele": scan_hillis_steele,
         "blelloch": scan_blelloch, "chunked": scan_chunked}          # models/scan.py:168-173


def scan_vjp(a, h0, h, dh):
    """Adjoint of scan_sequential, as models/scan.py:233-248 computes it inside
    SelectiveScanFn.backward: lambda_t = dh_t + a_{t+1} lambda_{t+1} (the reverse scan of
    :239-240), da_t = lambda_t h_{t-1} (h_{-1} = h0 or 0), db_t = lambda_t, dh0 = a_0 lambda_0.
    Returns (da, db, dh0)."""
    L = a.shape[1]
    lam = np.empty_like(dh)
    acc = np.zeros_like(dh[:, 0])
    for t in range(L - 1, -1, -1):
        acc = dh[:, t] + (a[:, t + 1] * acc if t + 1 < L else 0.0)
        lam[:, t] = acc
    hz = np.zeros_like(h[:, 0]) if h0 is None else h0
    h_prev = np.concatenate([hz[:, None], h[:, :-1]], 1)
    return lam * h_prev, lam, (None if h0 is None else a[:, 0] * lam[:, 0])


def discretize_vjp(delta, A, Bm, x, ga, gb, method="zoh"):
    """Vector-Jacobian product of discretize (the autograd.grad of models/scan.py:249):
    given ga = dL/da, gb = dL/db (B, L, D, N) returns (ddelta, dA, dBm, dx).  Closed-form
    derivatives of the three discretizations (ZOH db/dA uses f(z) = (z e^z - expm1 z)/z^2,
    a 4-term series below |z| < 1e-3 as kernels/triton_scan.py:199-200 does)."""
    z = delta[..., None] * A
    Bx = x[..., None] * Bm[:, :, None, :]
    dt = delta[..., None]
    if method == "zoh":
        a = np.exp(z)
        e = np.expm1(z)
        small = np.abs(z) < 1e-3
        zs = np.where(small, 1.0, z)
        f = np.where(small, 0.5 + z / 3.0 + z * z / 8.0 + z ** 3 / 30.0, (zs * a - e) / (zs * zs))
        dadz, dbdd, d2f, coef = a, a, dt * dt * f, e / A
    elif method == "euler":
        a = np.exp(z)
        dadz, dbdd, d2f, coef = a, np.ones_like(z), np.zeros_like(z), dt * np.ones_like(z)
    elif method == "bilinear":
        u = 1.0 / (1.0 - 0.5 * z)
        dadz, dbdd, d2f, coef = u * u, u * u, 0.5 * dt * dt * u * u, dt * u
    else:
        raise ValueError(f"unknown discretization {method!r}")
    ddelta = np.sum(ga * dadz * A + gb * dbdd * Bx, axis=3)
    dA = np.sum(ga * dadz * dt + gb * d2f * Bx, axis=(0, 1))
    dBm = np.sum(gb * coef * x[..., None], axis=2)
    dx = np.sum(gb * coef * Bm[:, :, None, :], axis=3)
    return ddelta, dA, dBm, dx


# ----------------------------------------------------------------------------- selective scan

def silu(v):
    return v / (1.0 + np.exp(-v))


def selective_scan_fwd(x, delta, A, Bm, Cm, h0=None, method="zoh", D=None, z=None,
                       return_states=False):
    """Forward of selective_scan_reference (models/scan.py:264-274) plus the D skip and
    SiLU gate of models/mamba.py:124:  out = (y + D x) * silu(z).

    Returns (out, y, last) and, with return_states, the (B, L, D, N) states."""
    x, delta, A, Bm, Cm = (np.asarray(v, np.float64) for v in (x, delta, A, Bm, Cm))
    Bsz, L, Dm = x.shape
    N = A.shape[1]
    h = np.zeros((Bsz, Dm, N)) if h0 is None else np.asarray(h0, np.float64).copy()
    y = np.empty((Bsz, L, Dm))
    hs = np.empty((Bsz, L, Dm, N)) if return_states else None
    for t in range(L):
        a, b = discretize(delta[:, t:t + 1], A, Bm[:, t:t + 1], x[:, t:t + 1], method)
        h = a[:, 0] * h + b[:, 0]
        y[:, t] = np.einsum("bdn,bn->bd", h, Cm[:, t])
        if return_states:
            hs[:, t] = h
    out = y.copy()
    if D is not None:
        out = out + x * np.asarray(D, np.float64)
    if z is not None:
        out = out * silu(np.asarray(z, np.float64))
    if return_states:
        return out, y, h, hs
    return out, y, h


def selective_scan_bwd(x, delta, A, Bm, Cm, dout, h0=None, method="zoh", D=None, z=None,
                       dlast=None, mag=False):
    """Hand-written adjoint of selective_scan_fwd.

    Recurrence and per-method derivatives follow kernels/triton_scan.py:171-226 (reverse
    walk: dh += dy C; dC = sum_d dy h; da = dh h_prev; method terms; dh *= a) and the
    reduction semantics of models/scan.py:219-255 (dA summed over batch and time, dB/dC
    over channels, dh0 = a_0 dh_0).  Gate/skip: out = (y + D x) s z, s = sigmoid(z):
    dy = dout s z, dz = dout (y + D x) s (1 + z (1 - s)), dD = sum dy x, dx += dy D.

    Returns dict with dx, ddelta, dA, dB, dC and (when present) dD, dz, dh0.  With mag, also
    ddelta_mag, dA_mag, dB_mag and dC_mag: per element the sum of the magnitudes of the terms it
    adds (over the states for ddelta, over batch and time for dA, over the channels for dB and
    dC), the
    scale of the float32 rounding a kernel summing those terms can leave in it."""
    x, delta, A, Bm, Cm, dout = (np.asarray(v, np.float64) for v in (x, delta, A, Bm, Cm, dout))
    Bsz, L, Dm = x.shape
    N = A.shape[1]
    _, y, _, hs = selective_scan_fwd(x, delta, A, Bm, Cm, h0, method, return_states=True)
    g = {}
    dy = dout
    if z is not None:
        zz = np.asarray(z, np.float64)
        s = 1.0 / (1.0 + np.exp(-zz))
        pre = y + (x * np.asarray(D, np.float64) if D is not None else 0.0)
        g["dz"] = dout * pre * s * (1.0 + zz * (1.0 - s))
        dy = dout * zz * s
    dx = np.zeros_like(x)
    if D is not None:
        Dv = np.asarray(D, np.float64)
        g["dD"] = np.einsum("bld,bld->d", dy, x)
        dx = dx + dy * Dv
    ddelta = np.zeros_like(delta)
    dA = np.zeros_like(A)
    ddelta_mag, dA_mag, dB_mag, dC_mag = np.zeros_like(delta), np.zeros_like(A), np.zeros_like(Bm), np.zeros_like(Cm)
    dB = np.zeros_like(Bm)
    dC = np.zeros_like(Cm)
    dh = np.zeros((Bsz, Dm, N)) if dlast is None else np.asarray(dlast, np.float64).copy()
    hz = np.zeros((Bsz, Dm, N)) if h0 is None else np.asarray(h0, np.float64)
    for t in range(L - 1, -1, -1):
        h_t = hs[:, t]
        hp = hs[:, t - 1] if t > 0 else hz
        dyt = dy[:, t]                                   # (B, D)
        dt = delta[:, t][..., None]                      # (B, D, 1)
        xt = x[:, t][..., None]                          # (B, D, 1)
        Bt = Bm[:, t][:, None, :]                        # (B, 1, N)
        Ct = Cm[:, t][:, None, :]
        dC[:, t] = np.einsum("bd,bdn->bn", dyt, h_t)
        if mag:
            dC_mag[:, t] = np.einsum("bd,bdn->bn", np.abs(dyt), np.abs(h_t))
        dh = dh + dyt[..., None] * Ct
        zt = dt * A
        Bx = Bt * xt
        da = dh * hp
        if method == "zoh":
            a = np.exp(zt)
            e = np.expm1(zt)
            coef = e / A
            small = np.abs(zt) < 1e-3
            zs = np.where(small, 1.0, zt)
            f = np.where(small, 0.5 + zt / 3.0 + zt * zt / 8.0 + zt ** 3 / 30.0,
                         (zs * a - e) / (zs * zs))
            td, tA = da * A * a + dh * a * Bx, da * dt * a + dh * dt * dt * f * Bx
            ddelta[:, t] = np.sum(td, axis=2)
            dA += np.sum(tA, axis=0)
            tB = dh * coef * xt
            dB[:, t] = np.sum(tB, axis=1)
            dx[:, t] += np.sum(dh * coef * Bt, axis=2)
        elif method == "euler":
            a = np.exp(zt)
            td, tA = da * A * a + dh * Bx, da * dt * a
            ddelta[:, t] = np.sum(td, axis=2)
            dA += np.sum(tA, axis=0)
            tB = dh * dt * xt
            dB[:, t] = np.sum(tB, axis=1)
            dx[:, t] += np.sum(dh * dt * Bt, axis=2)
        elif method == "bilinear":
            u = 1.0 / (1.0 - 0.5 * zt)
            a = (1.0 + 0.5 * zt) * u
            u2 = u * u
            td, tA = da * A * u2 + dh * u2 * Bx, da * dt * u2 + dh * 0.5 * dt * dt * u2 * Bx
            ddelta[:, t] = np.sum(td, axis=2)
            dA += np.sum(tA, axis=0)
            tB = dh * dt * u * xt
            dB[:, t] = np.sum(tB, axis=1)
            dx[:, t] += np.sum(dh * dt * u * Bt, axis=2)
        else:
            raise ValueError(f"unknown discretization {method!r}")
        if mag:
            ddelta_mag[:, t] = np.sum(np.abs(td), axis=2)
            dA_mag += np.sum(np.abs(tA), axis=0)
            dB_mag[:, t] = np.sum(np.abs(tB), axis=1)
        dh = dh * a
    g.update(dx=dx, ddelta=ddelta, dA=dA, dB=dB, dC=dC)
    if mag:
        g.update(ddelta_mag=ddelta_mag, dA_mag=dA_mag, dB_mag=dB_mag, dC_mag=dC_mag)
    if h0 is not None:
        g["dh0"] = dh
    return g


# ----------------------------------------------------------------------------- decode step

def ssm_step(h, x, delta, A, Bm, Cm, method="zoh", D=None, z=None):
    """Recurrent decode step of models/mamba.py:113-118,122-124 for one token.
    h (B, D, N); x, delta, z (B, D); Bm, Cm (B, N).  Returns (out (B, D), h_new)."""
    a, b = discretize(delta[:, None], A, Bm[:, None], x[:, None], method)
    h_new = a[:, 0] * h + b[:, 0]
    y = np.einsum("bdn,bn->bd", h_new, Cm)
    if D is not None:
        y = y + x * D
    if z is not None:
        y = y * silu(z)
    return y, h_new


def conv1d_causal(x_bdl, w, bias=None, state=None, activation=True):
    """Depthwise causal conv of models/mamba.py:101-107.  x (B, D, L), w (D, K), bias (D,),
    state (B, D, K-1) = the previous K-1 inputs (zeros when None, i.e. F.pad).
    Returns (y (B, D, L) after SiLU when activation, new_state (B, D, K-1))."""
    Bsz, Dm, L = x_bdl.shape
    K = w.shape[1]
    prev = np.zeros((Bsz, Dm, K - 1)) if state is None else state
    xp = np.concatenate([prev, x_bdl], -1)
    y = np.zeros((Bsz, Dm, L))
    for k in range(K):
        y += w[None, :, k, None] * xp[:, :, k:k + L]
    if bias is not None:
        y += bias[None, :, None]
    if activation:
        y = silu(y)
    return y, xp[:, :, -(K - 1):] if K > 1 else np.zeros((Bsz, Dm, 0))


# ----------------------------------------------------------------------------- integer plans

def cdiv(a, b):
    return -(-a // b)


def blocks(shape_bld, N, d_block):
    """models/scan.py:185-190."""
    Bsz, L, D = shape_bld
    if not d_block:
        d_block = max(1, SCAN_ELEMENT_BUDGET // (Bsz * L * N))
    d_block = min(d_block, D)
    return [(i, min(i + d_block, D)) for i in range(0, D, d_block)]


def block_d(Bsz, D):
    """kernels/triton_scan.py:245-250."""
    bd = BLOCK_D
    while bd > 4 and Bsz * cdiv(D, bd) < 128:
        bd //= 2
    return bd


def bwd_tile(Bsz, L, N, bd):
    """kernels/triton_scan.py:305 (channel tile of the backward's state scratch)."""
    return max(bd, (HBUF_BUDGET // (Bsz * L * N)) // bd * bd)


def resolve_scan(scan, is_gpu, method, N, has_engine=True):
    """models/scan.py:286-287 with _triton_ok :305-314: 'auto' picks the fused GPU engine
    when it is available, the input is on the GPU, the method is known and N is a power
    of two; otherwise 'chunked'.  Other names pass through; unknown names are KeyError
    (models/scan.py:261)."""
    if scan == "auto":
        ok = has_engine and is_gpu and method in DISCRETIZATIONS and N & (N - 1) == 0
        return "triton" if ok else "chunked"
    if scan not in SCAN_NAMES:
        raise KeyError(scan)
    return scan
