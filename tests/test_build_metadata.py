"""Build checks on the gfx950 code object inside htrc_amd/libhtrc_flat.so (CPU only).

Kernels that issue direct global->LDS loads (global_load_lds_dwordx4, from inline asm whose
register operands the compiler's wait and hazard handling cannot see) must not spill: a build
whose kernel reloaded spilled per-lane load offsets from scratch into the register each load
reads gave wrong results.  This test extracts the library's own device code object, reads each
kernel's private segment size from its metadata and counts its direct loads in the
disassembly.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "htrc_amd" / "libhtrc_flat.so"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# kernel symbol prefix -> largest private segment allowed: the leaf-16 attend kernel keeps a
# 4-byte reload in its redo pass (rarely taken), which feeds an LDS read, not a load address
ALLOWED = {"_Z12route_kernelILi16ELi2ELi1ELi2EE": 8}


def _tool(name: str) -> str:
    p = LLVM / name
    if p.exists():
        return str(p)
    w = shutil.which(name)
    if w is None:
        pytest.skip(f"{name} not available")
    return w


@pytest.fixture(scope="module")
def code_object(tmp_path_factory):
    if not LIB.exists():
        pytest.skip("libhtrc_flat.so is not built")
    d = tmp_path_factory.mktemp("co")
    fat, co = d / "fatbin.bin", d / "dev.co"
    subprocess.run([_tool("llvm-objcopy"), "-O", "binary", "--only-section=.hip_fatbin", str(LIB), str(fat)],
                   check=True)
    subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fat}",
                    f"--targets={TARGET}", f"--output={co}"], check=True)
    return co


def _private_segments(co: Path) -> dict[str, int]:
    notes = subprocess.run([_tool("llvm-readelf"), "--notes", str(co)], check=True, capture_output=True,
                           text=True).stdout
    sizes, cur = {}, None
    for line in notes.splitlines():
        m = re.match(r"\s*\.name:\s+(\S+)", line)
        if m:
            cur = m.group(1)
            continue
        m = re.match(r"\s*\.private_segment_fixed_size:\s+(\d+)", line)
        if m and cur is not None:
            sizes[cur] = int(m.group(1))
    return sizes


def _direct_loads(co: Path) -> dict[str, int]:
    dis = subprocess.run([_tool("llvm-objdump"), "-d", "--no-show-raw-insn", str(co)], check=True,
                         capture_output=True, text=True).stdout
    counts, cur = {}, None
    for line in dis.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            cur = m.group(1)
            counts[cur] = 0
        elif cur is not None and "global_load_lds" in line:
            counts[cur] += 1
    return counts


def test_kernels_with_direct_lds_loads_do_not_spill(code_object):
    sizes = _private_segments(code_object)
    loads = _direct_loads(code_object)
    assert sizes and loads, "no kernel metadata or disassembly read"
    users = {k: n for k, n in loads.items() if n > 0 and k in sizes}
    # the hot kernels issue them: the attend, select and fp32 tile kernels at least
    for prefix in ("_Z12route_kernel", "_Z19route_select_kernel", "_Z15tile_f32_kernel"):
        assert any(k.startswith(prefix) for k in users), f"no direct loads found in {prefix}*"
    bad = []
    for k in users:
        limit = next((v for p, v in ALLOWED.items() if k.startswith(p)), 0)
        if sizes[k] > limit:
            bad.append((k, sizes[k]))
    assert not bad, f"kernels with direct LDS loads that spill: {bad}"
