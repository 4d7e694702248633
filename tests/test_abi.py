"""The C-ABI library loads, exports what include/flash_hog.h declares and
rejects invalid calls before touching the GPU (no kernels run here)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

REPO = pathlib.Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "flash_hog.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fhog_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from flash_hog import _hip

    if not _hip.library_path().exists():
        pytest.fail(f"{_hip.library_path()} missing: run python flash-hog_amd/build.py")
    return _hip.lib()


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("fhog_attention_fwd", "fhog_attention_bwd", "fhog_attention_bwdbwd",
              "fhog_last_error", "fhog_status_string", "fhog_abi_version", "fhog_row_stat_bytes"):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_python_signatures_cover_the_header():
    from flash_hog import _hip

    assert set(_hip.SIGNATURES) == set(declared_functions())


def test_status_strings(lib):
    assert lib.fhog_abi_version() == 103
    assert lib.fhog_status_string(0) == b"ok"
    assert lib.fhog_status_string(1) == b"invalid argument"
    assert lib.fhog_status_string(2) == b"unsupported"
    assert lib.fhog_status_string(3) == b"kernel launch failed"
    assert lib.fhog_status_string(99) == b"unknown status"


def test_row_stat_bytes(lib):
    assert lib.fhog_row_stat_bytes(4, 16, 2048) == 4 * 16 * 2048 * 4
    assert lib.fhog_row_stat_bytes(0, 16, 2048) == 0


def _bwdbwd_args(ptr=16, batch=1, n_q=16, n_k=16, heads=1, kv_heads=1, head_dim=64, dtype=2, causal=1,
                 scale=0.125):
    return [None] + [ptr] * 16 + [batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale]


@pytest.mark.parametrize("kwargs,status,needle", [
    (dict(ptr=None), 1, "q is null"),
    (dict(ptr=8), 1, "not 16-byte aligned"),
    (dict(batch=0), 1, "sizes must be >= 1"),
    (dict(n_k=0), 1, "sizes must be >= 1"),
    (dict(dtype=7), 1, "unknown dtype"),
    (dict(heads=3, kv_heads=2), 1, "multiple of kv_heads"),
    (dict(causal=3), 1, "causal must be 0 (none), 1 (top-left) or 2 (bottom-right)"),
    (dict(causal=-1), 1, "causal must be"),
    (dict(head_dim=96), 2, "head_dim must be 64, 128 or 256"),
    (dict(head_dim=96, dtype=0), 2, "fp32 head_dim must be 64 or 128"),
    (dict(head_dim=256, dtype=0), 2, "fp32 head_dim must be 64 or 128"),
    (dict(scale=float("nan")), 1, "scale"),
    (dict(scale=float("inf")), 1, "scale must be finite"),
    (dict(scale=0.0), 2, "scale must be nonzero"),
    (dict(scale=-0.0), 2, "scale must be nonzero"),
])
def test_bwdbwd_rejects_invalid_arguments(lib, kwargs, status, needle):
    st = lib.fhog_attention_bwdbwd(*_bwdbwd_args(**kwargs))
    assert st == status
    assert needle in lib.fhog_last_error().decode()


def test_fwd_and_bwd_reject_invalid_arguments(lib):
    st = lib.fhog_attention_fwd(None, None, 16, 16, 16, 16, 1, 8, 8, 1, 1, 64, 2, 0, 0.125)
    assert st == 1 and "q is null" in lib.fhog_last_error().decode()
    st = lib.fhog_attention_bwd(None, *([16] * 9), None, 1, 8, 8, 1, 1, 64, 2, 0, 0.125)
    assert st == 1 and "delta is null" in lib.fhog_last_error().decode()


def test_error_message_is_per_thread(lib):
    import threading

    lib.fhog_attention_bwdbwd(*_bwdbwd_args(ptr=None))
    seen = {}

    def other():
        seen["msg"] = lib.fhog_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == b""
    assert b"q is null" in lib.fhog_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from flash_hog import _hip

    monkeypatch.setenv(_hip.LIB_ENV, str(tmp_path / "nope.so"))
    _hip.lib.cache_clear()
    try:
        with pytest.raises(ImportError, match="not found"):
            _hip.lib()
    finally:
        monkeypatch.delenv(_hip.LIB_ENV)
        _hip.lib.cache_clear()


def _noalloc_args(ptr=16, batch=1, n_q=16, n_k=16, heads=1, kv_heads=1, head_dim=64, dtype=2, causal=1,
                  scale=0.125):
    return [None] + [ptr] * 13 + [batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale]


@pytest.mark.parametrize("kwargs,status,needle", [
    (dict(ptr=None), 1, "q is null"),
    (dict(ptr=8), 1, "not 16-byte aligned"),
    (dict(scale=0.0), 2, "scale must be nonzero"),
    (dict(head_dim=96), 2, "head_dim must be 64, 128 or 256"),
    # 1048577 (batch, head, query) rows: one more than the static scratch holds
    (dict(batch=1, heads=1, kv_heads=1, n_q=(1 << 20) + 1, n_k=64), 2, "exceeds the static scratch"),
    (dict(batch=64, heads=16, kv_heads=16, n_q=1025, n_k=1025), 2, "exceeds the static scratch"),
])
def test_bwdbwd_noalloc_rejects_before_touching_the_gpu(lib, kwargs, status, needle):
    st = lib.fhog_attention_bwdbwd_noalloc(*_noalloc_args(**kwargs))
    assert st == status
    assert needle in lib.fhog_last_error().decode()


def test_library_imports_no_allocating_hip_routine():
    """No entry point allocates or frees device or host memory through HIP."""
    import shutil
    import subprocess

    from flash_hog import _hip

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--undefined-only", str(_hip.library_path())], capture_output=True,
                         text=True, check=True).stdout
    imported = set(re.findall(r"\b(hip[A-Za-z0-9_]+)", out))
    assert imported, out
    allocating = {n for n in imported if re.search(r"Malloc|Free|Alloc|HostRegister|MemPool", n)}
    assert not allocating, sorted(allocating)


@pytest.mark.parametrize("kwargs,status,needle", [
    (dict(), 0, ""),
    (dict(head_dim=128, n_q=77, n_k=300, causal=2), 0, ""),
    (dict(dtype=0), 0, ""),
    (dict(heads=8, kv_heads=2, scale=-0.3), 0, ""),
    (dict(head_dim=128, dtype=0), 0, ""),
    (dict(head_dim=256, dtype=1, heads=4, kv_heads=2), 0, ""),
    (dict(head_dim=96), 2, "head_dim must be 64, 128 or 256"),
    (dict(head_dim=256, dtype=0), 2, "fp32 head_dim must be 64 or 128"),
    (dict(heads=3, kv_heads=2), 1, "multiple of kv_heads"),
    (dict(scale=0.0), 2, "scale must be nonzero"),
    (dict(n_q=0), 1, "sizes must be >= 1"),
])
def test_supported_answers_as_the_entry_points_would(lib, kwargs, status, needle):
    """fhog_attention_supported (device -1: arguments only, no HIP call)
    returns the status and message that the entry points give for the same
    arguments."""
    args = dict(batch=1, n_q=16, n_k=16, heads=1, kv_heads=1, head_dim=64, dtype=2, causal=1, scale=0.125)
    args.update(kwargs)
    st = lib.fhog_attention_supported(-1, *args.values())
    assert st == status
    assert needle in lib.fhog_last_error().decode()
    if status:
        assert lib.fhog_attention_bwdbwd(*_bwdbwd_args(**args)) == status


def test_supported_python_api_without_gpu():
    """Mirrors flash_hog/jax/_tk_gpu.py:70-80: keyword arguments, a bool, and
    False on a machine with no gfx950 GPU (here: none at all)."""
    import torch

    import flash_hog
    from flash_hog import _hip

    kw = dict(is_causal=True, seq_len=2048, head_dim=64, num_q_heads=16, num_kv_heads=16)
    if not torch.cuda.is_available():
        assert flash_hog.supported(**kw) is False
    assert _hip.attention_supported(4, 2048, 2048, 16, 16, 64, torch.bfloat16, True, 0.125) == (True, "")
    ok, why = _hip.attention_supported(4, 2048, 2048, 16, 16, 96, torch.bfloat16, True, 0.125)
    assert not ok and "head_dim must be 64, 128 or 256" in why
    ok, why = _hip.attention_supported(4, 2048, 2048, 16, 16, 64, torch.float64, True, 0.125)
    assert not ok and "dtype" in why
    with pytest.raises(ValueError, match="causal_alignment"):
        flash_hog.supported(**kw, causal_alignment="diagonal")
    # head_dim < 1 has no default scale (0 ** -0.5): False, even with a device named
    for hd in (0, -64):
        assert flash_hog.supported(**{**kw, "head_dim": hd}, device=0) is False
        assert flash_hog.supported(**{**kw, "head_dim": hd}) is False


def test_unloadable_torch_extension_falls_back(monkeypatch, tmp_path):
    """An extension file that exists but cannot be loaded (built for another
    torch or Python) gives one warning and the Python wrappers, not an error
    from every call; the result is cached, so the load is not retried."""
    import warnings

    import torch

    from flash_hog import _hip

    bad = tmp_path / _hip.TORCH_EXT_PATH.name
    bad.write_bytes(b"\x7fELF but not a shared object")
    monkeypatch.setattr(_hip, "TORCH_EXT_PATH", bad)
    _hip.torch_ext.cache_clear()
    try:
        with pytest.warns(RuntimeWarning, match="not loaded"):
            assert _hip.torch_ext() is None
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            assert _hip.torch_ext() is None
        # the capability query and the Python wrappers' checks still run
        assert _hip.attention_supported(4, 2048, 2048, 16, 16, 64, torch.bfloat16, True, 0.125) == (True, "")
        q = torch.zeros(1, 8, 2, 64, dtype=torch.bfloat16)
        with pytest.raises(ValueError, match="must be on a GPU device"):
            _hip.attention_fwd(q, q, q, 1, 0.125)
    finally:
        _hip.torch_ext.cache_clear()


def test_torch_extension_is_built_and_bound():
    """The torch extension _fhog_torch (C++ calls of the C ABI) is built in-tree
    and bound to the loaded library's entry points."""
    from flash_hog import _hip

    assert _hip.TORCH_EXT_PATH.exists(), f"{_hip.TORCH_EXT_PATH} missing: run python flash-hog_amd/build.py"
    ext = _hip.torch_ext()
    assert ext is not None
    for name in ("attention_fwd", "attention_bwd", "attention_bwdbwd"):
        assert callable(getattr(ext, name))


def _python_path(monkeypatch):
    from flash_hog import _hip

    monkeypatch.setattr(_hip, "torch_ext", lambda: None)


@pytest.mark.parametrize("which", ["fwd", "bwd", "bwdbwd"])
def test_torch_extension_rejects_as_the_python_wrappers_do(which, monkeypatch):
    """Host tensors are refused by the extension with the Python wrappers'
    exception and message, and a non-tensor argument with a TypeError, before
    anything reaches the GPU."""
    import torch

    from flash_hog import _hip

    q = torch.zeros(1, 8, 2, 64, dtype=torch.bfloat16)
    lse = torch.zeros(1, 2, 8)
    args = {"fwd": (q, q, q), "bwd": (q, q, q, q, q, lse), "bwdbwd": (q, q, q, q, q, q, q, q, lse)}[which]
    fn = getattr(_hip, "attention_" + which)

    def outcome(*a):
        with pytest.raises((ValueError, TypeError)) as e:
            fn(*a, 1, 0.125)
        return e.type, str(e.value)

    got = outcome(*args)
    assert outcome(args[0], 3, *args[2:])[0] is TypeError
    _python_path(monkeypatch)
    assert got == outcome(*args) == (ValueError, "q must be on a GPU device, got cpu")
