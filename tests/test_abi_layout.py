"""The ctypes mirrors of the C-ABI argument structs (mugen_amd/_capi.py) match
include/mugen_attn.h field by field: a C program built from the header
prints sizeof and every offsetof, and each must equal what ctypes computes.
A drift would hand the library shifted fields without any error."""
import ctypes
import os
import shutil
import subprocess

import pytest

from mugen_amd import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

STRUCTS = {
    "GqaDecodeArgs": "mugen_attn_gqa_decode_args",
    "KvQ4Store": "mugen_attn_kv_q4_store",
    "KvQ4AppendArgs": "mugen_attn_kv_q4_append_args",
    "GqaDecodeQ4Args": "mugen_attn_gqa_decode_q4_args",
    "KvAppendArgs": "mugen_attn_kv_append_args",
    "GqaPrefillArgs": "mugen_attn_gqa_prefill_args",
    "MlaDecodeArgs": "mugen_attn_mla_decode_args",
    "RopeParams": "mugen_attn_rope_params",
    "MlaAbsorbArgs": "mugen_attn_mla_absorb_args",
    "MlaLatentWriteArgs": "mugen_attn_mla_latent_write_args",
    "MlaProjectArgs": "mugen_attn_mla_project_args",
}


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "mugen_attn.h"', "int main(void) {"]
    for py, c in STRUCTS.items():
        lines.append(f'  printf("{py} sizeof %zu\\n", sizeof({c}));')
        for name, _ in getattr(_capi, py)._fields_:
            lines.append(f'  printf("{py} {name} %zu\\n", offsetof({c}, {name}));')
    lines += ["  return 0;", "}"]
    d = tmp_path_factory.mktemp("abi")
    src, exe = d / "layout.c", d / "layout"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run([cc, "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {(s, f): int(v) for s, f, v in (line.split() for line in out.splitlines())}


@pytest.mark.parametrize("py", sorted(STRUCTS))
def test_struct_layout(c_layout, py):
    cls = getattr(_capi, py)
    assert c_layout[(py, "sizeof")] == ctypes.sizeof(cls), f"{py}: sizeof differs"
    for name, _ in cls._fields_:
        assert c_layout[(py, name)] == getattr(cls, name).offset, f"{py}.{name}: offset differs"


def test_every_header_struct_mirrored():
    import re
    hdr = open(os.path.join(ROOT, "include", "mugen_attn.h")).read()
    declared = set(re.findall(r"typedef struct (\w+) \{", hdr))
    assert declared == set(STRUCTS.values())
