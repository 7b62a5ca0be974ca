"""The C-ABI library loads, exports every symbol include/aac_attn.h declares,
and rejects bad arguments on the host (no GPU work is issued here)."""
import ctypes
import re
from pathlib import Path

import pytest

from awesome_acceleration_amd import _lib
from awesome_acceleration_amd.build import LIB_PATH

HEADER = Path(__file__).resolve().parent.parent / "include" / "aac_attn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(aac_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def declared_prototypes():
    """name -> (return type, [parameter types]) parsed from the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(aac_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(3).split(",") if p.strip() and p.strip() != "void"]
        # drop the parameter name: the type is everything before the last identifier
        types = [re.sub(r"\b\w+$", "", p).strip() for p in params]
        out[m.group(2)] = (m.group(1).split()[-1] if m.group(1).split() else "", types)
    return out


def _type_class(c_type: str) -> str:
    t = c_type.replace("const", "").strip()
    if "*" in t:
        return "char*" if t.replace(" ", "") == "char*" else "pointer"
    return {"int": "int32", "int32_t": "int32", "int64_t": "int64", "float": "float",
            "size_t": "size_t"}[t]


def _ctypes_class(ct) -> str:
    if ct in (ctypes.c_void_p,):
        return "pointer"
    if ct is ctypes.c_char_p:
        return "char*"
    if ct is ctypes.c_float:
        return "float"
    if ct is ctypes.c_size_t:
        return "size_t"
    return {4: "int32", 8: "int64"}[ctypes.sizeof(ct)]


def test_binding_parameter_types_match_the_header():
    """Every argtype of the ctypes binding has the width and kind of the
    header's parameter at that position (a drift would corrupt arguments)."""
    protos = declared_prototypes()
    assert sorted(protos) == sorted(_lib.SIGNATURES)
    for name, (res, args) in _lib.SIGNATURES.items():
        ret, params = protos[name]
        assert len(params) == len(args), (name, len(params), len(args))
        for i, (cp, ct) in enumerate(zip(params, args)):
            assert _type_class(cp) == _ctypes_class(ct), (name, i, cp, ct)
        if ret == "char*" or name == "aac_strerror":
            assert res is ctypes.c_char_p
        else:
            assert _type_class(ret) == _ctypes_class(res), (name, ret, res)


def test_library_exports_every_declared_symbol():
    assert LIB_PATH.exists(), "build the library first (__graft_entry__.build())"
    handle = ctypes.CDLL(str(LIB_PATH))
    for name in declared_functions():
        assert hasattr(handle, name), name


def test_abi_version_and_messages():
    L = _lib.lib()
    assert L.aac_abi_version() == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert L.aac_strerror(code)
    assert b"unknown" in L.aac_strerror(-99)


def test_host_side_argument_rejection():
    L = _lib.lib()
    # null pointers with work to do -> AAC_ERR_INVALID_ARGUMENT, before any launch
    assert L.aac_kv_store(None, None, 1024, 1024, None, None, 16, None, 4, 8, 128, 0, None) == -1
    # zero tokens is a no-op success
    assert L.aac_kv_store(None, None, 1024, 1024, None, None, 16, None, 0, 8, 128, 0, None) == 0
    # unknown dtype
    assert L.aac_kv_store(None, None, 1024, 1024, None, None, 16, None, 4, 8, 128, 9, None) == -2
    # head_dim other than 128 is not built for decode
    assert L.aac_decode_paged(None, 0, None, None, 1, 16, None, 1, None, 1, 0, 4, 2, 64, 1.0,
                              None, 0, None, 0, 0, 0, None) == -2
    # Hq not a multiple of Hkv
    assert L.aac_decode_paged(None, 0, None, None, 1, 16, None, 1, None, 1, 0, 6, 4, 128, 1.0,
                              None, 0, None, 0, 0, 0, None) == -5
    # prefill: fp32 is not supported on the MFMA path
    assert L.aac_prefill_varlen(None, None, None, 0, 0, 0, None, None, 1, 1, 1, 16, 8, 128,
                                1.0, 1, None, 0, None, 0, 2, None) == -2
    # KV export/import: unknown dtype, a table too short for the length, nothing to
    # move, null pointers with work to do, a misaligned buffer
    ex, im = L.aac_kv_export_paged, L.aac_kv_import_paged
    assert ex(None, 0, 0, 2, 4, 16, 8, 128, None, 1, 8, None, 9, None) == -2
    assert ex(None, 0, 0, 2, 4, 16, 8, 128, None, 2, 40, None, 0, None) == -5
    assert im(None, None, 0, 0, 2, 4, 16, 8, 128, None, 2, 40, 0, None) == -5
    assert ex(None, 0, 0, 0, 4, 16, 8, 128, None, 1, 8, None, 0, None) == 0
    assert im(None, None, 0, 0, 2, 4, 16, 8, 128, None, 1, 0, 0, None) == 0
    assert ex(None, 0, 0, 2, 4, 16, 8, 128, None, 1, 8, None, 0, None) == -1
    assert ex(16, 0, 0, 2, 4, 16, 8, 128, 64, 1, 8, 24, 0, None) == -3


def test_workspace_sizing():
    L = _lib.lib()
    # context that fits one partition needs no workspace
    assert L.aac_decode_workspace_bytes(4, 16, 8, 128, 256, 1, 0, 256) == 0
    # 8 blocks of 256 split in 512-token partitions: 4 partitions x (128 + 1) floats
    n = L.aac_decode_workspace_bytes(256, 16, 8, 128, 256, 8, 0, 512)
    assert n == 256 * 16 * 4 * 129 * 4


def test_check_raises_runtime_error():
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(-1, "probe")


def test_header_compiles_as_c_and_links(tmp_path):
    """A plain C99 program includes include/aac_attn.h, links the library and
    calls its host-side paths (tests/c_abi_check.c): the boundary is usable
    from C, not only through ctypes."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "c_abi_check"
    src = Path(__file__).resolve().parent / "c_abi_check.c"
    libdir = LIB_PATH.parent
    r = subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-I", str(HEADER.parent), str(src),
                        "-o", str(exe), f"-L{libdir}", "-laac_attn", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr


def test_generated_prefill_assembly_matches_its_generator():
    """csrc/prefill_wide_asm.inc is written by csrc/gen_prefill_wide_asm.py;
    the committed file must be exactly what the generator prints, so a change
    to either one cannot drift from the other."""
    import subprocess
    import sys
    gen = Path(__file__).resolve().parent.parent / "awesome_acceleration_amd" / "csrc" / "gen_prefill_wide_asm.py"
    r = subprocess.run([sys.executable, str(gen), "--check"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
