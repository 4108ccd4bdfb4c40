"""ctypes mirror of include/ssm_scan.h and the loader of libssmscan.so.

The library is loaded after ``import torch`` so that it binds to the HIP runtime torch
already loaded (both use the soname libamdhip64.so.7); the kernels then run on torch's
streams and device memory.  A missing library is an error: there is no fallback path.
"""

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libssmscan.so")
ABI_VERSION = 8

OK, EINVAL, EKEY, ESPACE, EHIP = 0, 1, 2, 3, 4
ZOH, EULER, BILINEAR = 0, 1, 2
F32, BF16, F16, F64 = 0, 1, 2, 3
SCAN_IDS = {"reference": 0, "sequential": 1, "hillis_steele": 2, "blelloch": 3, "chunked": 4,
            "triton": 5, "auto": 6}
SCAN_NAMES = {v: k for k, v in SCAN_IDS.items()}
DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.float64: F64}

c_i64, c_i32, c_vp = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p


class Tensor(ctypes.Structure):
    _fields_ = [("data", c_vp), ("stride", c_i64 * 3)]


class FwdArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seqlen", c_i64), ("dim", c_i64), ("dstate", c_i64),
                ("method", c_i32), ("dtype", c_i32),
                ("x", Tensor), ("delta", Tensor), ("A", Tensor), ("Bm", Tensor), ("Cm", Tensor),
                ("Dskip", Tensor), ("z", Tensor), ("delta_bias", Tensor),
                ("delta_softplus", c_i32), ("segments", c_i32),
                ("h0", Tensor), ("out", Tensor), ("last", Tensor),
                ("saved", c_vp), ("workspace", c_vp), ("workspace_bytes", c_i64),
                ("delta_proj", Tensor), ("delta_rank", c_i64),
                ("A_is_log", c_i32), ("reserved1", c_i32)]


class BwdArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seqlen", c_i64), ("dim", c_i64), ("dstate", c_i64),
                ("method", c_i32), ("dtype", c_i32),
                ("x", Tensor), ("delta", Tensor), ("A", Tensor), ("Bm", Tensor), ("Cm", Tensor),
                ("Dskip", Tensor), ("z", Tensor), ("delta_bias", Tensor),
                ("delta_softplus", c_i32), ("segments", c_i32),
                ("h0", Tensor), ("saved", c_vp), ("dout", Tensor), ("dlast", Tensor),
                ("dx", Tensor), ("ddelta", Tensor), ("dA", Tensor), ("dBm", Tensor), ("dCm", Tensor),
                ("dD", Tensor), ("dz", Tensor), ("ddelta_bias", Tensor), ("dh0", Tensor),
                ("workspace", c_vp), ("workspace_bytes", c_i64),
                ("delta_proj", Tensor), ("delta_rank", c_i64),
                ("A_is_log", c_i32), ("reserved1", c_i32)]


class StepArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("dim", c_i64), ("dstate", c_i64),
                ("method", c_i32), ("dtype", c_i32),
                ("x", Tensor), ("delta", Tensor), ("A", Tensor), ("Bm", Tensor), ("Cm", Tensor),
                ("Dskip", Tensor), ("z", Tensor), ("delta_bias", Tensor),
                ("delta_softplus", c_i32), ("reserved0", c_i32),
                ("h", Tensor), ("out", Tensor)]


class DecodeArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("dim", c_i64), ("dstate", c_i64), ("width", c_i64), ("dt_rank", c_i64),
                ("d_model", c_i64), ("method", c_i32), ("conv_state_dtype", c_i32),
                ("eps", ctypes.c_float), ("reserved1", ctypes.c_float),
                ("u", c_vp), ("xz", c_vp), ("conv_w", c_vp), ("conv_b", c_vp), ("conv_state", c_vp),
                ("x_proj_wt", c_vp), ("dt_proj_w", c_vp), ("dt_bias", c_vp), ("A_log", c_vp), ("Dskip", c_vp),
                ("ssm_state", c_vp), ("y", c_vp)]



class DecodeBlock(ctypes.Structure):
    _fields_ = [("w_in4", c_vp), ("conv_w", c_vp), ("conv_b", c_vp), ("x_proj_wt", c_vp), ("dt_proj_w", c_vp),
                ("dt_bias", c_vp), ("A_log", c_vp), ("Dskip", c_vp), ("w_out4", c_vp),
                ("conv_state", c_vp), ("ssm_state", c_vp), ("eps", ctypes.c_float), ("reserved0", c_i32)]


class DecodeStackArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("dim", c_i64), ("dstate", c_i64), ("width", c_i64), ("dt_rank", c_i64),
                ("d_model", c_i64), ("method", c_i32), ("conv_state_dtype", c_i32),
                ("n_blocks", c_i32), ("reserved0", c_i32),
                ("blocks", ctypes.POINTER(DecodeBlock)), ("u", c_vp),
                ("workspace", c_vp), ("workspace_bytes", c_i64),
                ("tokens", c_vp), ("embed", c_vp), ("head_w4", c_vp), ("logits", c_vp), ("vocab", c_i64),
                ("head_eps", ctypes.c_float), ("reserved1", c_i32)]

class LscanArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seqlen", c_i64), ("width", c_i64),
                ("algo", c_i32), ("dtype", c_i32), ("reverse", c_i32), ("reserved0", c_i32),
                ("chunk", c_i64),
                ("a", Tensor), ("b", Tensor), ("h0", Tensor), ("h", Tensor),
                ("workspace", c_vp), ("workspace_bytes", c_i64)]


class LscanBwdArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seqlen", c_i64), ("width", c_i64),
                ("algo", c_i32), ("dtype", c_i32), ("reverse", c_i32), ("reserved0", c_i32),
                ("chunk", c_i64),
                ("a", Tensor), ("h0", Tensor), ("h", Tensor), ("dh", Tensor),
                ("da", Tensor), ("db", Tensor), ("dh0", Tensor),
                ("workspace", c_vp), ("workspace_bytes", c_i64)]


class DiscArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seqlen", c_i64), ("dim", c_i64), ("dstate", c_i64),
                ("method", c_i32), ("dtype", c_i32),
                ("delta", Tensor), ("x", Tensor), ("A", Tensor), ("Bm", Tensor),
                ("a", c_vp), ("b", c_vp), ("da", c_vp), ("db", c_vp),
                ("ddelta", Tensor), ("dx", Tensor), ("dA", Tensor), ("dBm", Tensor),
                ("workspace", c_vp), ("workspace_bytes", c_i64)]


class ConvArgs(ctypes.Structure):
    _fields_ = [("batch", c_i64), ("seqlen", c_i64), ("dim", c_i64), ("width", c_i64),
                ("dtype", c_i32), ("silu", c_i32),
                ("x", Tensor), ("weight", Tensor), ("bias", Tensor), ("state_in", Tensor),
                ("out", Tensor), ("state_out", Tensor), ("dout", Tensor), ("dx", Tensor),
                ("dweight", Tensor), ("dbias", Tensor),
                ("workspace", c_vp), ("workspace_bytes", c_i64)]


class NormArgs(ctypes.Structure):
    _fields_ = [("rows", c_i64), ("dim", c_i64), ("dtype", c_i32), ("reserved0", c_i32),
                ("eps", ctypes.c_double),
                ("x", Tensor), ("weight", Tensor), ("out", Tensor), ("rstd", c_vp),
                ("dout", Tensor), ("dx", Tensor), ("dweight", c_vp),
                ("workspace", c_vp), ("workspace_bytes", c_i64)]


# name -> (restype, argtypes)
_SIGS = {
    "ssm_abi_version": (c_i32, []),
    "ssm_last_error": (ctypes.c_char_p, []),
    "ssm_fwd_check": (c_i32, [ctypes.POINTER(FwdArgs)]),
    "ssm_bwd_check": (c_i32, [ctypes.POINTER(BwdArgs)]),
    "ssm_step_check": (c_i32, [ctypes.POINTER(StepArgs)]),
    "ssm_decode_check": (c_i32, [ctypes.POINTER(DecodeArgs)]),
    "ssm_decode_stack_check": (c_i32, [ctypes.POINTER(DecodeStackArgs)]),
    "ssm_lscan_check": (c_i32, [ctypes.POINTER(LscanArgs)]),
    "ssm_lscan_bwd_check": (c_i32, [ctypes.POINTER(LscanBwdArgs)]),
    "ssm_disc_check": (c_i32, [ctypes.POINTER(DiscArgs)]),
    "ssm_conv_check": (c_i32, [ctypes.POINTER(ConvArgs)]),
    "ssm_norm_check": (c_i32, [ctypes.POINTER(NormArgs)]),
    "ssm_fwd_saved_bytes": (c_i64, [ctypes.POINTER(FwdArgs)]),
    "ssm_fwd_workspace_bytes": (c_i64, [ctypes.POINTER(FwdArgs)]),
    "ssm_bwd_workspace_bytes": (c_i64, [ctypes.POINTER(BwdArgs)]),
    "ssm_lscan_workspace_bytes": (c_i64, [ctypes.POINTER(LscanArgs)]),
    "ssm_lscan_bwd_workspace_bytes": (c_i64, [ctypes.POINTER(LscanBwdArgs)]),
    "ssm_disc_workspace_bytes": (c_i64, [ctypes.POINTER(DiscArgs)]),
    "ssm_conv_workspace_bytes": (c_i64, [ctypes.POINTER(ConvArgs)]),
    "ssm_norm_workspace_bytes": (c_i64, [ctypes.POINTER(NormArgs)]),
    "ssm_decode_stack_workspace_bytes": (c_i64, [ctypes.POINTER(DecodeStackArgs)]),
    "ssm_decode_stack_status_offset": (c_i64, [ctypes.POINTER(DecodeStackArgs)]),
    "ssm_fwd": (c_i32, [ctypes.POINTER(FwdArgs), c_vp]),
    "ssm_fwd_noalloc": (c_i32, [ctypes.POINTER(FwdArgs), c_vp]),
    "ssm_bwd": (c_i32, [ctypes.POINTER(BwdArgs), c_vp]),
    "ssm_step": (c_i32, [ctypes.POINTER(StepArgs), c_vp]),
    "ssm_decode_step": (c_i32, [ctypes.POINTER(DecodeArgs), c_vp]),
    "ssm_decode_stack": (c_i32, [ctypes.POINTER(DecodeStackArgs), c_vp]),
    "ssm_lscan": (c_i32, [ctypes.POINTER(LscanArgs), c_vp]),
    "ssm_lscan_bwd": (c_i32, [ctypes.POINTER(LscanBwdArgs), c_vp]),
    "ssm_disc_fwd": (c_i32, [ctypes.POINTER(DiscArgs), c_vp]),
    "ssm_disc_bwd": (c_i32, [ctypes.POINTER(DiscArgs), c_vp]),
    "ssm_conv_fwd": (c_i32, [ctypes.POINTER(ConvArgs), c_vp]),
    "ssm_conv_bwd": (c_i32, [ctypes.POINTER(ConvArgs), c_vp]),
    "ssm_norm_fwd": (c_i32, [ctypes.POINTER(NormArgs), c_vp]),
    "ssm_norm_bwd": (c_i32, [ctypes.POINTER(NormArgs), c_vp]),
    "ssm_default_chunk": (c_i64, [c_i64]),
    "ssm_scan_blocks": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.POINTER(c_i64), c_i64]),
    "ssm_block_d": (c_i64, [c_i64, c_i64]),
    "ssm_bwd_tile": (c_i64, [c_i64, c_i64, c_i64, c_i64]),
    "ssm_resolve_scan": (c_i32, [c_i32, c_i32, c_i32, c_i64, c_i32]),
}
EXPORTED = tuple(_SIGS)

_lib = None


def lib():
    """The loaded engine library; raises if it is not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(make -C mamba-ssm-benchmark_amd/csrc)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.ssm_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libssmscan ABI version {ver} != expected {ABI_VERSION}")
        _lib = handle
    return _lib


_ERRORS = {EINVAL: ValueError, EKEY: KeyError, ESPACE: ValueError, EHIP: RuntimeError}


def check(rc, what):
    if rc != OK:
        msg = (lib().ssm_last_error() or b"").decode(errors="replace")
        raise _ERRORS.get(rc, RuntimeError)(f"{what}: {msg}")


_ABSENT = Tensor()  # null data, zero strides; an argument struct copies it on assignment


def view(t):
    """ssm_tensor for a torch tensor (None -> absent); strides in elements, padded to 3."""
    if t is None:
        return _ABSENT
    st = t.stride()
    if len(st) > 3:
        raise ValueError(f"expected a tensor of at most 3 dims, got shape {tuple(t.shape)}")
    return Tensor(t.data_ptr(), st + (0,) * (3 - len(st)))


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device):
    """The raw handle of torch's current stream on `device`, which the launches are enqueued on
    (read without building a torch.cuda.Stream object: this is on every launch's host path)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


class on_device:
    """The engine launches on the current device: make `device` current for the block, and
    skip torch.cuda.device's two device exchanges when it already is (the usual case)."""

    __slots__ = ("idx", "prev")

    def __init__(self, device):
        self.idx = device.index

    def __enter__(self):
        cur = torch.cuda.current_device()
        self.prev = cur if self.idx is not None and self.idx != cur else None
        if self.prev is not None:
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
