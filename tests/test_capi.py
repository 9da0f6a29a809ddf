"""The C-ABI library on the CPU (no GPU calls): it loads, exports every entry point that
include/kushkash_amd.h declares with the argument list the Python binding uses, reports its ABI
revision, and rejects bad arguments with the reference's error convention (-1 unsupported shape ->
ValueError, kushkash/_cpu.py:38-40) before touching a device. The product has no CPU fallback."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import kushkash_amd
from kushkash_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "kushkash_amd.h"


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB.exists():
        kushkash_amd.build()
    return _lib.lib()


def header_functions() -> dict[str, int]:
    """name -> parameter count of every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|const char\s*\*)\s*(kush_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_header_declares_the_entry_points():
    fns = header_functions()
    assert set(fns) == {"kush_append", "kush_write", "kush_decode", "kush_append_decode", "kush_combine", "kush_fwht",
                        "kush_unpack", "kush_last_error",
                        "kush_abi_version"}


def test_library_exports_every_header_symbol(lib):
    raw = ctypes.CDLL(str(_lib.LIB))
    for name, n in header_functions().items():
        assert hasattr(raw, name), name
        assert len(_lib.SIGNATURES[name]) == n, (name, n, len(_lib.SIGNATURES[name]))
    assert set(_lib.SIGNATURES) == set(header_functions())


def test_abi_version(lib):
    m = re.search(r"ABI revision of this header \((\d+)\)", HEADER.read_text())
    assert m and int(m.group(1)) == lib.kush_abi_version() == _lib.ABI_VERSION


def _decode_args(**kw):
    a = dict(head_dim=128, bits=4, group=7, dtype=2, q=None, out=None, cache=None, bs=0, hs=0, tail_k=None,
             tail_idx=None, bt=None, seq_lens=None, bt_stride=0, bt_cols=0, hkv=4, scale=1.0, n_splits=1, part_ml=None,
             part_o=None, sync=None, waves=0, seq_order=None, n_seqs=1, rot=0, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,code,msg", [
    (dict(head_dim=96), -1, "unsupported head_dim"),
    (dict(bits=3), -1, "unsupported bits"),
    (dict(dtype=7), -1, "unsupported dtype"),
    (dict(n_seqs=-1), -2, "bad n_seqs"),
    (dict(group=0), -2, "bad n_seqs"),
    (dict(n_splits=4), -2, "needs the partial buffers"),
    (dict(bs=8), -2, "16-byte aligned"),
    (dict(waves=3), -2, "waves"),
    (dict(rot=2), -2, "rot"),
])
def test_decode_rejects_bad_arguments(lib, kw, code, msg):
    assert lib.kush_decode(*_decode_args(**kw)) == code
    assert msg in lib.kush_last_error().decode()


def test_error_codes_map_to_reference_exceptions(lib):
    with pytest.raises(ValueError, match="unsupported head_dim"):
        _lib.call("kush_decode", *_decode_args(head_dim=96))
    with pytest.raises(RuntimeError, match="kush_decode failed \\(-2\\)"):
        _lib.call("kush_decode", *_decode_args(n_seqs=-1))


def test_combine_and_writes_reject_bad_arguments(lib):
    assert lib.kush_combine(128, 7, 2, None, None, None, 0, 4, 1, 0, None) == -2
    assert lib.kush_combine(96, 7, 2, None, None, None, 2, 4, 1, 0, None) == -1
    assert lib.kush_combine(128, 7, 2, None, None, None, 2, 4, 1, 2, None) == -2           # rot is 0 or 1
    assert lib.kush_append(96, 4, 2, None, None, 0, 0, None, 0, 0, None, None, 0, 0, None, None, 0, 4, 1, 0,
                           None) == -1
    assert lib.kush_append(128, 4, 2, None, None, 0, 0, None, 0, 0, None, None, 0, 0, None, None, 0, 4, 1, 3,
                           None) == -2
    assert lib.kush_write(128, 5, 2, None, None, 0, 0, None, None, None, None, None, 1, 0, None, 0, 0, None, None,
                          0, 4, 0, None) == -1
    assert lib.kush_write(128, 4, 2, None, None, 0, 0, None, None, None, None, None, 1, 0, None, 0, 0, None, None,
                          0, 4, -1, None) == -2


def test_ops_is_gpu_only():
    """No CPU fallback: the product's Ops refuses a CPU device (the oracle lives under tests' reach only)."""
    with pytest.raises(ValueError, match="GPU"):
        kushkash_amd.Ops(torch.device("cpu"), 128, 4, 7, torch.bfloat16)
    with pytest.raises(ValueError):
        kushkash_amd.KushCache(1, 4, 28, 128, device="cpu", dtype=torch.float32)


def test_package_does_not_import_the_oracle():
    """The product never imports or loads the oracle (it is test infrastructure only)."""
    pkg = Path(kushkash_amd.__file__).resolve().parent
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        src = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", src, re.M), f
        assert "libkush_oracle" not in src and "kush_cpu_" not in src, f
