"""Code-generation check of this build's own gfx950 code objects (CPU lane).

A vector store wider than 8 bytes reads its data registers over several cycles, and the compiler
emits no wait state before a VALU write of those registers when a buffer store takes an SGPR
offset. Gradient-tile variants whose 16-byte stores were followed at once by such writes gave
intermittently wrong rows (the pair was one of two suspects; neither was isolated). The shipped
kernels have no such pair, and this test keeps it that way: it disassembles the objects
`build()` leaves in `mlx-train-perf_amd/_build/` (the device code object of each, unbundled from
its fat binary) and fails if a 12- or 16-byte store's data registers are written by either of the
next two instructions with no `s_nop` between."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
OBJ_DIR = ROOT / "mlx-train-perf_amd" / "_build"
LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

STORE = re.compile(r"^(buffer|global|flat|scratch)_store_(dwordx3|dwordx4|b96|b128)\s+(.*)$")
VALU_DST = re.compile(r"^(v_\w+)\s+(v\[\d+:\d+\]|v\d+)")


def _vgprs(tok: str) -> set[int]:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _disassemble(obj: Path, tmp: Path) -> list[str]:
    fat, co = tmp / (obj.stem + ".fatbin"), tmp / (obj.stem + ".co")
    subprocess.run([str(LLVM / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", str(obj)], check=True,
                   capture_output=True)
    subprocess.run([str(LLVM / "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fat}",
                    f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
    out = subprocess.run([str(LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(co)], check=True,
                         capture_output=True, text=True).stdout
    return [ln.split("//")[0].strip() for ln in out.splitlines()]


def _store_data_hazards(lines: list[str]) -> list[str]:
    hits = []
    for i, ln in enumerate(lines):
        m = STORE.match(ln)
        if not m:
            continue
        ops = [o.strip() for o in m.group(3).split(",")]
        # buffer/scratch stores: vdata first; global/flat stores: vaddr, vdata.
        data = _vgprs(ops[0] if m.group(1) in ("buffer", "scratch") else ops[1])
        for nxt in lines[i + 1:i + 3]:
            if not nxt or nxt.startswith("s_nop"):
                break
            v = VALU_DST.match(nxt)
            if v and not v.group(1).startswith("v_mfma") and _vgprs(v.group(2)) & data:
                hits.append(f"{ln}  ->  {nxt}")
                break
    return hits


def test_no_wide_store_data_rewritten_by_the_next_instructions(tmp_path):
    objs = sorted(OBJ_DIR.glob("*.o"))
    if not objs or not (LLVM / "llvm-objdump").exists() or shutil.which(str(LLVM / "clang-offload-bundler")) is None:
        pytest.skip("built objects or the ROCm LLVM tools are not here (run build() first)")
    stores, hits = 0, []
    for obj in objs:
        lines = _disassemble(obj, tmp_path)
        stores += sum(1 for ln in lines if STORE.match(ln))
        hits += [f"{obj.name}: {h}" for h in _store_data_hazards(lines)]
    assert stores > 0, "no wide stores found: the disassembly format changed?"
    assert not hits, "\n".join(hits)


def test_the_check_finds_the_pattern():
    """The scanner itself, on the pair the failing variant had."""
    bad = ["buffer_store_dwordx4 v[114:117], v255, s[16:19], s2 offen", "v_fma_f32 v114, v122, s68, -v229"]
    ok = ["buffer_store_dwordx4 v[114:117], v255, s[16:19], s2 offen", "s_nop 0", "v_fma_f32 v114, v122, s68, -v229"]
    other = ["global_store_dwordx4 v[18:19], v[14:17], off", "v_mov_b32 v18, 0"]  # rewrites the address only
    assert _store_data_hazards(bad) and not _store_data_hazards(ok) and not _store_data_hazards(other)
