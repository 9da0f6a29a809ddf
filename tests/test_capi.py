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


def header_params(header: Path = HEADER) -> dict[str, list[str]]:
    """name -> parameter declarations (type and name) of every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int32_t|const char\s*\*)\s*(kush_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = [] if params in ("", "void") else [" ".join(x.split()) for x in params.split(",")]
    return out


def header_functions() -> dict[str, int]:
    """name -> parameter count of every function declared in the header."""
    return {k: len(v) for k, v in header_params().items()}


def test_header_declares_the_entry_points():
    fns = header_functions()
    assert set(fns) == {"kush_append", "kush_append_ex", "kush_write", "kush_write_ex", "kush_decode",
                        "kush_decode_ex", "kush_append_decode", "kush_decode_noalloc", "kush_combine",
                        "kush_combine_ex", "kush_fwht", "kush_unpack", "kush_last_error", "kush_abi_version"}


# The reference's launch argument sets (restated from _cpu.py:12-19 and the
# kernels' parameter lists, gpu.mojo:207-212, :241-246, :566-572, :469-471), by parameter meaning.
REFERENCE_ARGS = {
    "kush_append": ["head_dim", "bits", "dtype", "k", "v", "k_row_stride", "v_row_stride", "seq_lens", "pos_offset",
                    "advance", "tail_idx", "cache", "block_stride", "head_stride", "tail_k", "block_table",
                    "bt_row_stride", "hkv", "n_seqs", "stream"],
    "kush_write": ["head_dim", "bits", "dtype", "k", "v", "k_row_stride", "v_row_stride", "query_start_loc",
                   "seq_lens", "tail_idx", "job_seq", "job_page", "n_jobs", "mode", "cache", "block_stride",
                   "head_stride", "tail_k", "block_table", "bt_row_stride", "hkv", "stream"],
    "kush_decode": ["head_dim", "bits", "group", "dtype", "q", "out", "cache", "block_stride", "head_stride", "tail_k",
                    "tail_idx", "block_table", "seq_lens", "bt_row_stride", "hkv", "scale", "n_splits", "part_ml",
                    "part_o", "n_seqs", "stream"],
    "kush_combine": ["head_dim", "group", "dtype", "out", "part_ml", "part_o", "n_splits", "hkv", "n_seqs", "stream"],
}


def _names(params: list[str]) -> list[str]:
    return [re.sub(r"[^\w]", "", p.split()[-1].lstrip("*")) for p in params]


@pytest.mark.parametrize("name", sorted(REFERENCE_ARGS))
def test_entry_points_take_the_reference_argument_lists(name):
    """Each replacing entry point takes exactly the reference's argument list, in its order (a binding
    written from the reference's launch arguments works by position); its `_ex` variant is that list
    followed by this library's extensions, after the stream, never inserted mid-list."""
    params = header_params()
    assert _names(params[name]) == REFERENCE_ARGS[name]
    ext = params[name + "_ex"]
    assert ext[:len(params[name])] == params[name]
    assert len(ext) > len(params[name])
    if name == "kush_decode":                  # the fused append + decode starts with the decode list too
        fused = params["kush_append_decode"]   # (it writes the cache and tail: those lose their const)
        assert _names(fused[:len(params[name])]) == REFERENCE_ARGS[name]
        assert fused[-5:] == ext[-5:]


def test_library_exports_every_header_symbol(lib):
    raw = ctypes.CDLL(str(_lib.LIB))
    for name, n in header_functions().items():
        assert hasattr(raw, name), name
        assert len(_lib.SIGNATURES[name]) == n, (name, n, len(_lib.SIGNATURES[name]))
    assert set(_lib.SIGNATURES) == set(header_functions())


def test_cpu_library_exports_every_cpu_header_symbol():
    """libkushcpu.so (the CPU path) exports what include/kushkash_amd_cpu.h declares, with the parameter
    names and types its binding uses: the reference's CPU ABI (kush/cpu.mojo:476-562) plus one
    test hook, every argument int64 except the decode's float scale, int32 results."""
    from kushkash_amd import _cpu
    if not _cpu.LIB.exists():
        kushkash_amd.build()
    params = header_params(HEADER.parent / "kushkash_amd_cpu.h")
    assert set(params) == set(_cpu.PARAMS) == {"kush_cpu_append", "kush_cpu_write", "kush_cpu_decode",
                                               "kush_cpu_fwht", "kush_cpu_unpack", "kush_cpu_half_bits"}
    raw = ctypes.CDLL(str(_cpu.LIB))
    for name, decl in params.items():
        assert _names(decl) == _cpu.PARAMS[name].split(), name
        assert [p.split()[0] for p in decl] == ["float" if p.endswith(" scale") else "int64_t" for p in decl], name
        assert hasattr(raw, name), name
    # the reference's argument counts (kushkash/_cpu.py:10-25): 18, 20, 16, 3, 22
    assert [len(_cpu.SIGNATURES[n]) for n in ("kush_cpu_append", "kush_cpu_write", "kush_cpu_decode",
                                               "kush_cpu_fwht", "kush_cpu_unpack")] == [18, 20, 16, 3, 22]
    assert _cpu.SIGNATURES["kush_cpu_decode"][14] is ctypes.c_float


def test_timeline_build_is_the_library_plus_its_reader(lib):
    """libkushhip_timeline.so (bench.py --timeline) exports every entry point of the header and the
    timeline reader; the product library has no reader (its kernels record nothing)."""
    import importlib
    kbuild = importlib.import_module("kushkash_amd.build")
    if not kbuild.TIMELINE_LIB.exists():
        kushkash_amd.build()
    tl = ctypes.CDLL(str(kbuild.TIMELINE_LIB))
    for name in header_functions():
        assert hasattr(tl, name), name
    assert tl.kush_abi_version() == _lib.ABI_VERSION
    assert hasattr(tl, "kush_timeline_read")
    assert not hasattr(ctypes.CDLL(str(_lib.LIB)), "kush_timeline_read")


def test_missing_library_names_the_build(monkeypatch, tmp_path):
    """No library -> a RuntimeError naming the build command on the first call, never a silent
    fallback (the reference's loader surfaces its driver error the same way: tests/test_cpu.py:235-254)."""
    monkeypatch.setattr(_lib, "LIB", tmp_path / "libkushhip.so")
    _lib.lib.cache_clear()
    try:
        with pytest.raises(RuntimeError, match=r"libkushhip\.so is not built; run `python -m kushkash_amd\.build`"):
            _lib.call("kush_abi_version")
    finally:
        monkeypatch.undo()
        _lib.lib.cache_clear()


def test_library_of_another_abi_is_refused(monkeypatch, tmp_path):
    """A library built from other sources (another ABI revision) is refused when loaded, before any
    entry point runs with a mismatched argument list."""
    class Fn:
        def __init__(self, ret):
            self.ret = ret

        def __call__(self, *args):
            return self.ret

    class OtherAbi:
        def __getattr__(self, name):
            fn = Fn(_lib.ABI_VERSION - 1 if name == "kush_abi_version" else 0)
            setattr(self, name, fn)
            return fn

    fake = tmp_path / "libkushhip.so"
    fake.write_bytes(b"")
    monkeypatch.setattr(_lib, "LIB", fake)
    monkeypatch.setattr(ctypes, "CDLL", lambda path: OtherAbi())
    _lib.lib.cache_clear()
    try:
        with pytest.raises(RuntimeError, match=f"has ABI {_lib.ABI_VERSION - 1}, expected {_lib.ABI_VERSION}"):
            _lib.lib()
    finally:
        monkeypatch.undo()
        _lib.lib.cache_clear()


def test_abi_version(lib):
    m = re.search(r"ABI revision of this header \((\d+)\)", HEADER.read_text())
    assert m and int(m.group(1)) == lib.kush_abi_version() == _lib.ABI_VERSION


def _decode_args(**kw):
    a = dict(head_dim=128, bits=4, group=7, dtype=2, q=None, out=None, cache=None, bs=0, hs=0, tail_k=None,
             tail_idx=None, bt=None, seq_lens=None, bt_stride=0, hkv=4, scale=1.0, n_splits=1, part_ml=None,
             part_o=None, n_seqs=1, stream=None, bt_cols=0, sync=None, waves=0, seq_order=None, rot=0)
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
    assert lib.kush_decode_ex(*_decode_args(**kw)) == code
    assert msg in lib.kush_last_error().decode()
    if not {"waves", "rot"} & set(kw):         # the reference-list entry point checks the same arguments
        assert lib.kush_decode(*_decode_args(**kw)[:21]) == code
        assert msg in lib.kush_last_error().decode()


def test_error_codes_map_to_reference_exceptions(lib):
    with pytest.raises(ValueError, match="unsupported head_dim"):
        _lib.call("kush_decode", *_decode_args(head_dim=96)[:21])
    with pytest.raises(RuntimeError, match="kush_decode_ex failed \\(-2\\)"):
        _lib.call("kush_decode_ex", *_decode_args(n_seqs=-1))


def test_combine_and_writes_reject_bad_arguments(lib):
    assert lib.kush_combine(128, 7, 2, None, None, None, 0, 4, 1, None) == -2
    assert lib.kush_combine(96, 7, 2, None, None, None, 2, 4, 1, None) == -1
    assert lib.kush_combine_ex(128, 7, 2, None, None, None, 2, 4, 1, None, 2) == -2         # rot is 0 or 1
    app = [96, 4, 2, None, None, 0, 0, None, 0, 0, None, None, 0, 0, None, None, 0, 4, 1, None]
    assert lib.kush_append(*app) == -1
    assert lib.kush_append_ex(*app, 0) == -1
    app[0] = 128
    assert lib.kush_append_ex(*app, 3) == -2
    wr = [128, 5, 2, None, None, 0, 0, None, None, None, None, None, 1, 0, None, 0, 0, None, None, 0, 4, None]
    assert lib.kush_write(*wr) == -1
    wr[1] = 4
    assert lib.kush_write_ex(*wr, -1) == -2
    wr[13] = 3
    assert lib.kush_write(*wr) == -2                                                     # mode 0, 1 or 2
    wr[13], wr[12] = 2, 1 << 29
    assert lib.kush_write(*wr) == -2                                 # 2^31 page tasks (jobs x kv heads) or more


def test_ops_devices():
    """Ops runs on a ROCm device or on the host (its own CPU library, fp32 as the reference's CPU path;
    never the oracle, which lives under the tests' reach only); any other device is refused."""
    with pytest.raises(ValueError, match="GPU .* or on the host"):
        kushkash_amd.Ops(torch.device("meta"), 128, 4, 7, torch.float32)
    with pytest.raises(ValueError, match="fp32"):
        kushkash_amd.Ops(torch.device("cpu"), 128, 4, 7, torch.bfloat16)
    ops = kushkash_amd.Ops(torch.device("cpu"), 128, 4, 7, torch.float32)
    assert ops._cpu.LIB.name == "libkushcpu.so" and ops._cpu.LIB.parent == Path(kushkash_amd.__file__).parent


def test_package_does_not_import_the_oracle():
    """The product never imports or loads the oracle (it is test infrastructure only)."""
    pkg = Path(kushkash_amd.__file__).resolve().parent
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        src = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", src, re.M), f
        assert "libkush_oracle" not in src and "kush_oracle" not in src, f
    # the CPU path's entry points keep the reference's CPU names (kush_cpu_*): the package binds them
    # from its own host library, built from csrc/kush_cpu.cpp, never from the oracle's
    from kushkash_amd import _cpu
    assert Path(_cpu.lib()._name).resolve() == pkg / "libkushcpu.so"
    assert _cpu.LIB == pkg / "libkushcpu.so"
