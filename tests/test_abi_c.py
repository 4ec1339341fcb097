"""The C ABI from a C consumer: include/lia_hip.h compiled as C11 with -Wall -Werror, every
struct's sizeof / offsetof compared with the ctypes structures of the Python binding and with
the field order of the Rust #[repr(C)] block of the integration guide (the Rust binding a
maintainer adds on the reference side), and liblia_hip.so linked from C
and called (host packing, workspace sizing, validation errors; no GPU work)."""
import ctypes as C
import os
import re
import shutil
import subprocess

import pytest

from conftest import ROOT

SRC = os.path.join(ROOT, "tests", "abi", "abi_layout.c")
LIBDIR = os.path.join(ROOT, "lia.rs_amd")

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")


@pytest.fixture(scope="module")
def abi_exe(tmp_path_factory, lia):
    lia.lib()  # the library is built
    exe = str(tmp_path_factory.mktemp("abi") / "abi_layout")
    cmd = ["gcc", "-std=c11", "-Wall", "-Wextra", "-pedantic", "-Werror",
           "-I", os.path.join(ROOT, "include"), SRC, "-L", LIBDIR, "-llia_hip",
           "-Wl,-rpath," + LIBDIR, "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.fixture(scope="module")
def c_layout(abi_exe):
    out = subprocess.run([abi_exe], capture_output=True, text=True, check=True).stdout
    layout = {}
    for line in out.splitlines():
        struct, field, off, size = line.split()
        layout.setdefault(struct, {})[field] = (int(off), int(size))
    return layout


def _ctypes_structs(lia):
    return {
        "lia_paged_row": lia.PagedRow, "lia_group": lia.Group,
        "lia_paging_limits": lia.PagingLimits, "lia_pack_info": lia.PackInfo,
        "lia_kv_layout": lia.KVLayout, "lia_kv_planes": lia.KVPlanes,
        "lia_attention_config": lia.AttentionConfig, "lia_page_io": lia.PageIO,
        "lia_request": lia.Request, "lia_update": lia.Update,
    }


def test_every_header_struct_is_checked(c_layout, lia):
    text = open(os.path.join(ROOT, "include", "lia_hip.h")).read()
    defined = set(re.findall(r"typedef struct (lia_\w+) \{", text))
    assert defined == set(c_layout) == set(_ctypes_structs(lia))


def test_ctypes_structs_match_c(c_layout, lia):
    for name, cls in _ctypes_structs(lia).items():
        fields = c_layout[name]
        assert C.sizeof(cls) == fields["-"][1], name
        c_fields = [f for f in fields if f != "-"]
        assert [f for f, _ in cls._fields_] == c_fields, name
        for f in c_fields:
            desc = getattr(cls, f)
            assert (desc.offset, desc.size) == fields[f], (name, f)


def _rust_structs():
    """struct name -> field names in order, from the integration guide's #[repr(C)] block."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\][^\n]*\n\s*pub struct (lia_\w+)\s*\{(.*?)\}\s*(?://[^\n]*)?\n",
                         text, flags=re.S):
        body = re.sub(r"//[^\n]*", "", m.group(2))
        out[m.group(1)] = re.findall(r"pub (\w+)\s*:", body)
    return out


def test_rust_binding_field_order_matches_c(c_layout):
    rust = _rust_structs()
    for name, fields in c_layout.items():
        assert name in rust, f"{name} missing from the Rust binding"
        assert rust[name] == [f for f in fields if f != "-"], name


def test_calls_from_c(abi_exe, lia):
    out = subprocess.run([abi_exe, "calls"], capture_output=True, text=True, check=True).stdout
    got = dict(line.split(" ", 1) for line in out.strip().splitlines())
    # two sequences (pages 2, 6 and page 4), rows at positions 16, 17 and 3 of 16-token pages
    assert got["pack"] == "0 cu 0 2 3 slots 96 97 67 stride 4 groups 2"
    cfg = lia.AttentionConfig(16, 2, 128, 16, 64, 4, lia.BF16, lia.BF16, lia.BF16, 0.088, 8, 8, 64)
    assert int(got["workspace"]) == lia.workspace_bytes(cfg)
    assert int(got["sink_words"]) == lia.paged_read_sink_words(cfg) > 0
    assert lia.ERRORS[int(got["read_no_sink"])] == "invalid argument"     # LIA_E_ARG: no sink
    assert lia.ERRORS[int(got["read_short_sink"])] == "invalid argument"  # LIA_E_ARG: sink too short
    assert lia.ERRORS[int(got["unsupported"])] == "unsupported geometry"  # LIA_E_UNSUPPORTED
    assert lia.ERRORS[int(got["null_config"])] == "invalid argument"      # LIA_E_ARG
