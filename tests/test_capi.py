"""The C-ABI library (CPU-side checks): it builds, loads, exports exactly what include/ttsplat.h
declares with the arities the Python binding uses, and rejects bad arguments before launching
anything (so these calls are safe without a GPU)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ttsplat.h")


@pytest.fixture(scope="module")
def lib():
    from ttsplat import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from ttsplat import build
        build.build()
    return _lib.load()


def header_decls():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w]+\s*\*?\s+(tts_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


def test_header_parses():
    d = header_decls()
    assert "tts_assign_bins" in d and "tts_splat_bwd" in d and len(d) >= 20


def test_every_declared_symbol_is_exported(lib):
    so = lib._name
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = set(header_decls()) - exported
    assert not missing, missing


def test_binding_matches_header(lib):
    from ttsplat._lib import SIGNATURES
    d = header_decls()
    assert set(SIGNATURES) == set(d)
    for name, (_, args) in SIGNATURES.items():
        assert len(args) == d[name], name


def test_host_only_entry_points(lib):
    assert lib.tts_version() >> 16 == 0
    assert b"tile side" in lib.tts_strerror(-2)
    assert lib.tts_bin_workspace_bytes(100, 64, 64, 16) > 0
    assert lib.tts_loss_workspace_bytes(5, 5) == 0                 # below the 11x11 window
    ns = ctypes.c_int(0)
    n = lib.tts_loss_partials_count(128, 128, ctypes.byref(ns))
    assert n > ns.value > 0


@pytest.mark.parametrize("S,H,W,K,span,code", [
    (17, 64, 64, 128, 2048, -2),     # tile side
    (16, 60, 64, 128, 2048, -2),     # H not a multiple of S
    (16, 64, 64, 0, 2048, -3),       # K
    (16, 64, 64, 600, 2048, -3),
    (16, 64, 64, 128, 9000, -5),     # span
])
def test_assign_bins_rejects_before_launch(lib, S, H, W, K, span, code):
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    rc = lib.tts_assign_bins(p, 2, p, 1, 4, H, W, S, 1, K, span, p, p, None, None, None, None,
                             p, 1 << 20, None)
    assert rc == code


def test_splat_rejects_bad_tile(lib):
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.tts_splat_fwd(p, p, p, None, 64, 64, 24, 128, 4.0, p, p, p, None) == -2
    assert lib.tts_splat_bwd(p, p, p, None, 64, 64, 16, 2000, 4.0, p, p, p, p, p, None, None) == -3
    assert lib.tts_loss_grad(p, p, 64, 64, 0.2, p, None, None, 0, None) == -4


def test_loss_grad_size_limit(lib):
    """The loss kernels address with 32-bit buffer offsets: images whose statistics planes
    (about H*W*24 bytes) would pass 2^31 are refused before launch; 7680x4320 passes the check
    (and then stops at the missing workspace)."""
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.tts_loss_grad(p, p, 10000, 10000, 0.2, p, None, None, 0, None) == -1
    assert lib.tts_loss_grad_stats(p, p, p, 10000, 10000, 0.2, p, None, None) == -1
    assert lib.tts_loss_target_stats(p, 10000, 10000, p, None) == -1
    assert lib.tts_loss_grad(p, p, 4320, 7680, 0.2, p, None, None, 0, None) == -4
    assert lib.tts_loss_stats_bytes(4320, 7680) == 24 * 4310 * 7670 + 12 * 4320 * 7680


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from ttsplat import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.TTSError):
        _lib.load()


def test_wrappers_refuse_cpu_tensors():
    import torch
    from ttsplat import kernels
    with pytest.raises(ValueError):
        kernels.geom_fwd(torch.zeros(4, 14), torch.zeros(16))


def _null_args(argtypes, ival):
    args = []
    for a in argtypes:
        if a is ctypes.c_float:
            args.append(1.0)
        elif a in (ctypes.c_void_p, ctypes.c_char_p) or issubclass(a, ctypes._Pointer):
            args.append(None)
        else:
            args.append(ival)
    return args


def test_every_compute_entry_point_rejects_null_pointers(lib):
    """Every entry point that takes device buffers, called with all of them NULL, returns a
    negative domain code (TTS_EINVAL, or TTS_ETILE where the tile geometry is checked first)
    before launching anything; the host-only size queries answer without touching memory."""
    from ttsplat._lib import SIGNATURES
    host_only = {"tts_version", "tts_strerror"}
    for name, (res, argtypes) in SIGNATURES.items():
        if name in host_only or res is not ctypes.c_int:
            continue
        if not any(a is ctypes.c_void_p for a in argtypes):
            continue
        for ival in (16, 1):
            rc = getattr(lib, name)(*_null_args(argtypes, ival))
            assert rc in (-1, -2), (name, ival, rc)


def test_slot_scatter_checks_sizes_in_64_bits(lib):
    """T * K past 2^31 with NULL buffers: refused before launch (a 32-bit product would wrap
    negative and skip the pointer checks)."""
    assert lib.tts_slot_scatter(None, None, None, 70000, 40000, None, None) == -1
    assert lib.tts_slot_scatter(None, None, None, 0, 40000, None, None) == 0
