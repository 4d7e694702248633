"""ctypes binding of libflash_hog_hip.so, the C ABI declared in include/flash_hog.h.

This mirrors the plugin loader of the reference's native path
(flash_hog/jax/_tk_gpu.py:26-58): the library path comes from the
FLASH_HOG_HIP_LIB environment variable or the in-tree build, the library is
loaded once, and a missing library is an error (there is no fallback path).

The torch-level helpers below take device tensors, check them, allocate the
outputs and the fp32 row-statistic workspace with torch's caching allocator,
and enqueue the kernels on torch's current stream for the tensors' device.
Their `causal` argument is a bool (top-left when true) or the C ABI's code
(0 none, 1 top-left, 2 bottom-right). attention_fwd, attention_bwd and
attention_bwdbwd hand the work to the torch extension _lib/_fhog_torch when
it is built (the same checks, allocations and C-ABI call in C++, a few
microseconds of host time instead of 9-20), bound to the entry points of the
library loaded here; FLASH_HOG_TORCH_EXT=0 keeps them in Python.
"""

from __future__ import annotations

import ctypes
import functools
import importlib.machinery
import importlib.util
import os
import pathlib
import sysconfig
import warnings

import torch

LIB_ENV = "FLASH_HOG_HIP_LIB"
LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libflash_hog_hip.so"

FHOG_OK = 0
FHOG_ERR_INVALID_ARGUMENT = 1
FHOG_ERR_UNSUPPORTED = 2
FHOG_ERR_LAUNCH = 3

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

SIGNATURES = {
    "fhog_abi_version": (_i, []),
    "fhog_status_string": (ctypes.c_char_p, [_i]),
    "fhog_last_error": (ctypes.c_char_p, []),
    "fhog_row_stat_bytes": (ctypes.c_size_t, [_i, _i, _i]),
    "fhog_attention_supported": (_i, [_i] * 9 + [_f]),
    "fhog_attention_fwd": (_i, [_p, _p, _p, _p, _p, _p] + [_i] * 8 + [_f]),
    "fhog_attention_bwd": (_i, [_p] * 11 + [_i] * 8 + [_f]),
    "fhog_attention_bwdbwd": (_i, [_p] * 17 + [_i] * 8 + [_f]),
    "fhog_attention_bwdbwd_stage": (_i, [_p, _i] + [_p] * 16 + [_i] * 8 + [_f]),
    "fhog_attention_bwdbwd_noalloc": (_i, [_p] * 14 + [_i] * 8 + [_f]),
}


class FlashHogError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def library_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get(LIB_ENV) or LIB_PATH)


@functools.cache
def lib() -> ctypes.CDLL:
    path = library_path()
    if not path.exists():
        raise ImportError(
            f"Flash-HOG HIP library not found at {path}; build it with "
            f"`python flash-hog_amd/build.py` (or set {LIB_ENV})")
    handle = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


TORCH_EXT_ENV = "FLASH_HOG_TORCH_EXT"
TORCH_EXT_PATH = LIB_PATH.parent / ("_fhog_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


@functools.cache
def torch_ext():
    """The _fhog_torch extension bound to lib()'s entry points, or None when it
    is not built, cannot be loaded (built for another torch or Python, an
    undefined symbol: a warning says why, once) or FLASH_HOG_TORCH_EXT=0; the
    Python wrappers then do the same work. A missing kernel library is still
    an error (lib() raises), since the wrappers need it too. The result,
    None included, is cached."""
    if os.environ.get(TORCH_EXT_ENV, "1") == "0" or not TORCH_EXT_PATH.exists():
        return None
    L = lib()
    name = "flash_hog._lib._fhog_torch"
    try:
        loader = importlib.machinery.ExtensionFileLoader(name, str(TORCH_EXT_PATH))
        mod = importlib.util.module_from_spec(importlib.util.spec_from_loader(name, loader))
        loader.exec_module(mod)
        addr = lambda fn: ctypes.cast(fn, ctypes.c_void_p).value
        mod.bind(addr(L.fhog_attention_fwd), addr(L.fhog_attention_bwd), addr(L.fhog_attention_bwdbwd),
                 addr(L.fhog_last_error), addr(L.fhog_status_string), FlashHogError)
    except (ImportError, OSError, AttributeError) as exc:
        warnings.warn(f"Flash-HOG torch extension {TORCH_EXT_PATH} not loaded ({exc}); "
                      "using the Python wrappers", RuntimeWarning, stacklevel=2)
        return None
    return mod


def check(status: int) -> None:
    if status != FHOG_OK:
        L = lib()
        msg = L.fhog_last_error().decode() or L.fhog_status_string(status).decode()
        raise FlashHogError(status, msg)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch._C._cuda_getCurrentRawStream(device.index)


class _on_device:
    """Makes `device` current for the duration of a kernel call (the C ABI
    enqueues on the stream it is given, but the launch runs on the current
    device); a no-op when it already is."""

    __slots__ = ("index", "prev")

    def __init__(self, device: torch.device):
        self.index = device.index

    def __enter__(self):
        self.prev = torch.cuda.current_device()
        if self.prev != self.index:
            torch.cuda.set_device(self.index)

    def __exit__(self, *exc):
        if self.prev != self.index:
            torch.cuda.set_device(self.prev)
        return False


def _check_inputs(named, dtype=None):
    first = None
    for name, t in named:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU device, got {t.device}")
        if first is None:
            first = t
            dev = t.get_device()
        elif t.get_device() != dev:
            raise ValueError(f"{name} is on {t.device}, expected {first.device}")
        if dtype is not None and t.dtype != dtype:
            raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    return first


def _contig(*xs):
    return tuple(x if x.is_contiguous() else x.contiguous() for x in xs)


def _dims(q: torch.Tensor, k: torch.Tensor):
    """(B, Tq, Tk, N, Nk, H) of q (B, Tq, N, H) and k (B, Tk, Nk, H); N must be a
    multiple of Nk (grouped-query attention when N > Nk)."""
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError(f"expected (B, T, N, H) tensors, got q{tuple(q.shape)} k{tuple(k.shape)}")
    B, Tq, N, Hd = q.shape
    Bk, Tk, Nk, Hk = k.shape
    if Bk != B or Hk != Hd:
        raise ValueError(f"q{tuple(q.shape)} and k{tuple(k.shape)} disagree on batch or head_dim")
    if Nk == 0 or N % Nk != 0:
        raise ValueError(f"query heads ({N}) must be a multiple of key/value heads ({Nk})")
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"unsupported dtype {q.dtype}")
    return B, Tq, Tk, N, Nk, Hd


def causal_code(causal) -> int:
    """C ABI causal code: False/True map to none/top-left; ints pass through
    (0 none, 1 top-left, 2 bottom-right; the library rejects others)."""
    return int(causal)


def _expect(name, t, shape, dtype=None):
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")


def attention_supported(batch: int, n_q: int, n_k: int, heads: int, kv_heads: int, head_dim: int, dtype,
                        causal, scale: float, device: int = -1) -> tuple[bool, str]:
    """(True, "") if the library has kernels for these arguments (and, for
    device >= 0, that HIP device is a gfx950 GPU), else (False, the reason the
    entry points would give). Launches and allocates nothing."""
    if dtype not in DTYPE_CODES:
        return False, f"unsupported dtype {dtype}"
    status = lib().fhog_attention_supported(int(device), batch, n_q, n_k, heads, kv_heads, head_dim,
                                            DTYPE_CODES[dtype], causal_code(causal), float(scale))
    return status == 0, "" if status == 0 else lib().fhog_last_error().decode()


def attention_fwd(q, k, v, causal, scale: float):
    """O (B, T, N, H) in q's dtype and the natural-log logsumexp L (B, N, T) fp32."""
    ext = torch_ext()
    if ext is not None:
        return ext.attention_fwd(q, k, v, causal_code(causal), float(scale))
    _check_inputs([("q", q), ("k", k), ("v", v)], q.dtype)
    B, Tq, Tk, N, Nk, Hd = _dims(q, k)
    _expect("v", v, k.shape)
    q, k, v = _contig(q, k, v)
    o = torch.empty_like(q)
    lse = torch.empty((B, N, Tq), device=q.device, dtype=torch.float32)
    with _on_device(q.device):
        check(lib().fhog_attention_fwd(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse),
            B, Tq, Tk, N, Nk, Hd, DTYPE_CODES[q.dtype], causal_code(causal), float(scale)))
    return o, lse


def attention_bwd(q, k, v, o, dout, lse, causal, scale: float):
    """dQ, dK, dV of attention given its residual; also returns D (B, N, T) fp32."""
    ext = torch_ext()
    if ext is not None:
        return ext.attention_bwd(q, k, v, o, dout, lse, causal_code(causal), float(scale))
    _check_inputs([("q", q), ("k", k), ("v", v), ("o", o), ("dout", dout)], q.dtype)
    _check_inputs([("q", q), ("lse", lse)])
    B, Tq, Tk, N, Nk, Hd = _dims(q, k)
    _expect("v", v, k.shape)
    _expect("o", o, q.shape)
    _expect("dout", dout, q.shape)
    _expect("lse", lse, (B, N, Tq), torch.float32)
    q, k, v, o, dout, lse = _contig(q, k, v, o, dout, lse)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((B, N, Tq), device=q.device, dtype=torch.float32)
    with _on_device(q.device):
        check(lib().fhog_attention_bwd(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(dout), _ptr(lse),
            _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta),
            B, Tq, Tk, N, Nk, Hd, DTYPE_CODES[q.dtype], causal_code(causal), float(scale)))
    return dq, dk, dv, delta


def attention_bwdbwd(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale: float,
                     return_stats: bool = False):
    """dQ2, dK2, dV2, ddO of the double backward [and the row statistics D, dD, B]."""
    ext = torch_ext()
    if ext is not None:
        dq2, dk2, dv2, ddo, stats = ext.attention_bwdbwd(q, k, v, o, dout, ddq, ddk, ddv, lse, causal_code(causal),
                                                         float(scale))
        return (dq2, dk2, dv2, ddo, tuple(stats.unbind(0))) if return_stats else (dq2, dk2, dv2, ddo)
    _check_inputs([("q", q), ("k", k), ("v", v), ("o", o), ("dout", dout),
                   ("ddq", ddq), ("ddk", ddk), ("ddv", ddv)], q.dtype)
    _check_inputs([("q", q), ("lse", lse)])
    B, Tq, Tk, N, Nk, Hd = _dims(q, k)
    _expect("v", v, k.shape)
    for name, t in (("o", o), ("dout", dout), ("ddq", ddq)):
        _expect(name, t, q.shape)
    for name, t in (("ddk", ddk), ("ddv", ddv)):
        _expect(name, t, k.shape)
    _expect("lse", lse, (B, N, Tq), torch.float32)
    q, k, v, o, dout, ddq, ddk, ddv, lse = _contig(q, k, v, o, dout, ddq, ddk, ddv, lse)
    dq2, dk2, dv2, ddo = (torch.empty_like(x) for x in (q, k, v, dout))
    stats = torch.empty((3, B, N, Tq), device=q.device, dtype=torch.float32)
    with _on_device(q.device):
        check(lib().fhog_attention_bwdbwd(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(dout),
            _ptr(ddq), _ptr(ddk), _ptr(ddv), _ptr(lse),
            _ptr(dq2), _ptr(dk2), _ptr(dv2), _ptr(ddo),
            _ptr(stats[0]), _ptr(stats[1]), _ptr(stats[2]),
            B, Tq, Tk, N, Nk, Hd, DTYPE_CODES[q.dtype], causal_code(causal), float(scale)))
    if return_stats:
        return dq2, dk2, dv2, ddo, (stats[0], stats[1], stats[2])
    return dq2, dk2, dv2, ddo


def attention_bwdbwd_noalloc(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale: float, out=None):
    """attention_bwdbwd through fhog_attention_bwdbwd_noalloc: the row
    statistics live in the library's static device scratch, so the call needs
    no workspace. `out` = (dq2, dk2, dv2, ddo) preallocated outputs (allocated
    here when None)."""
    _check_inputs([("q", q), ("k", k), ("v", v), ("o", o), ("dout", dout),
                   ("ddq", ddq), ("ddk", ddk), ("ddv", ddv)], q.dtype)
    _check_inputs([("q", q), ("lse", lse)])
    B, Tq, Tk, N, Nk, Hd = _dims(q, k)
    _expect("v", v, k.shape)
    for name, t in (("o", o), ("dout", dout), ("ddq", ddq)):
        _expect(name, t, q.shape)
    for name, t in (("ddk", ddk), ("ddv", ddv)):
        _expect(name, t, k.shape)
    _expect("lse", lse, (B, N, Tq), torch.float32)
    q, k, v, o, dout, ddq, ddk, ddv, lse = _contig(q, k, v, o, dout, ddq, ddk, ddv, lse)
    if out is None:
        out = tuple(torch.empty_like(x) for x in (q, k, v, dout))
    for name, t, like in zip(("dq2", "dk2", "dv2", "ddo"), out, (q, k, v, dout)):
        _expect(name, t, like.shape, like.dtype)
        if not t.is_contiguous() or t.device != q.device:
            raise ValueError(f"{name} must be contiguous on {q.device}")
    dq2, dk2, dv2, ddo = out
    with _on_device(q.device):
        check(lib().fhog_attention_bwdbwd_noalloc(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(dout),
            _ptr(ddq), _ptr(ddk), _ptr(ddv), _ptr(lse),
            _ptr(dq2), _ptr(dk2), _ptr(dv2), _ptr(ddo),
            B, Tq, Tk, N, Nk, Hd, DTYPE_CODES[q.dtype], causal_code(causal), float(scale)))
    return dq2, dk2, dv2, ddo
