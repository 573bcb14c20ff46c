"""The C-ABI library: builds for gfx950, loads, exports every symbol the
header declares, and its struct layouts match the ctypes binding.

No compute call is made (CPU-only container).  The struct layout check
compiles a small C program against include/kiv_hip.h with gcc and compares
sizeof/offsetof with the ctypes Structures.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from kiv_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kiv_hip.h"


def header_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kiv_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_native.SIGNATURES)


def test_header_constants_match_binding():
    """The enum values the binding passes (flags, mask kinds, tiers, dtypes)."""
    text = HEADER.read_text()
    consts = {m.group(1): int(m.group(2)) for m in re.finditer(r"(KIV_[A-Z0-9_]+)\s*=\s*(\d+)", text)}
    assert consts["KIV_RETRIEVE_PRUNE"] == _native.RETRIEVE_PRUNE
    assert consts["KIV_MASK_CAUSAL"] == _native.MASK_CAUSAL and consts["KIV_MASK_BOOL"] == _native.MASK_BOOL
    assert consts["KIV_TIER_HOST"] == _native.TIER_HOST and consts["KIV_TIER_HBM"] == _native.TIER_HBM


def test_library_exports_every_declared_symbol():
    if not _native.LIB_PATH.exists():
        pytest.fail(f"{_native.LIB_PATH} not built (run __graft_entry__.build())")
    lib = _native.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.kiv_version() >= 100
    assert lib.kiv_last_error() == b""


def test_invalid_arguments_fail_without_gpu_work():
    lib = _native.lib()
    assert lib.kiv_store_create(None, 0, None) == 1  # KIV_ERR_INVALID
    assert b"null" in lib.kiv_last_error()
    assert lib.kiv_retrieve(None, None, None) == 1
    assert lib.kiv_fine_scan_stats(None, None, None) == 1
    assert lib.kiv_decode_attention(None, None) == 1
    assert lib.kiv_prefill_attention(None, None) == 1
    assert lib.kiv_prefill_workspace_size(0, 12, 128, 4096, 0, 8192) == 0
    # Room for a mask tensor's tile classes (one byte per 64 x 64 tile per q head) ...
    assert lib.kiv_prefill_workspace_size(1, 12, 128, 4096, 0, 8192) >= 12 * 64 * 128
    # ... plus a short query's key-split partial rows (fp32 rows, max and sum).
    assert lib.kiv_prefill_workspace_size(1, 12, 128, 16, 256, 2048) > 12 * 16 * 128 * 4
    assert lib.kiv_store_destroy(None) == 0


def test_struct_layouts_match_c():
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    structs = {
        "kiv_store_config_t": _native.StoreConfig,
        "kiv_store_info_t": _native.StoreInfo,
        "kiv_retrieve_args_t": _native.RetrieveArgs,
        "kiv_attention_args_t": _native.AttentionArgs,
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    work = Path(subprocess.check_output(["mktemp", "-d"], text=True).strip())
    src = work / "layout.c"
    src.write_text("\n".join(lines))
    subprocess.run([gcc, str(src), "-o", str(work / "layout")], check=True)
    out = subprocess.check_output([str(work / "layout")], text=True).split("\n")
    for line in filter(None, out):
        cname, field, val = line.split()
        py = structs[cname]
        want = ctypes.sizeof(py) if field == "size" else getattr(py, field).offset
        assert int(val) == want, (cname, field)
