"""Code-generation checks of this build's own gfx950 code objects (CPU lane). Each disassembles the
objects `build()` leaves in `mlx-train-perf_amd/_build/` (the device code object of each, unbundled
from its fat binary).

1. Wide stores: a 12- or 16-byte store's data registers written by either of the next two
   instructions with no `s_nop` between. Reverted gradient-tile variants with 16-byte stores had
   this pattern and gave intermittently wrong rows. It is a guard, not an explanation: the
   documented gfx9 rule (LLVM's GCNHazardRecognizer::createsVALUHazard) asks for that wait state
   only when the store's soffset is not a register, and those stores took an SGPR soffset, so this
   pair is probably not what went wrong.
2. Lane swaps: a `v_permlane{16,32}_swap` whose operands a VALU op writes within 2 wait states
   (or whose exec a `v_cmpx` writes within 4), the gfx950 hazard the reverted variant's swaps also
   came close to. The shipped kernels' swaps are inline asm with `s_nop 1` before them."""
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


# gfx950 lane-swap hazards (the VALU-write -> v_permlane{16,32}_swap rule of the gfx950 ISA's hazard
# table, as LLVM's GCNHazardRecognizer::checkPermlaneHazards applies it): a VALU write of either
# operand register needs 2 wait states before the swap reads it, and a v_cmpx writing exec needs 4.
# Every wait state is one instruction, s_nop N counts N + 1.
SWAP = re.compile(r"^v_permlane(16|32)_swap_b32(_e32|_e64)?\s+(v\d+),\s*(v\d+)")
_VALU_WAITS, _VCMPX_WAITS = 2, 4


def _wait_states(ln: str) -> int:
    m = re.match(r"^s_nop\s+(\d+|0x[0-9a-fA-F]+)", ln)
    return int(m.group(1), 0) + 1 if m else 1


def _permlane_swap_hazards(lines: list[str]) -> tuple[int, list[str]]:
    """(swaps seen, swaps whose operands a VALU op writes, or whose exec a v_cmpx writes, closer than
    the rule allows), scanning back through the preceding instructions of the listing."""
    n, hits = 0, []
    code = [ln for ln in lines if ln and not ln.endswith(">:") and not ln.startswith(("Disassembly", "<"))]
    for i, ln in enumerate(code):
        m = SWAP.match(ln)
        if not m:
            continue
        n += 1
        regs = _vgprs(m.group(3)) | _vgprs(m.group(4))
        waited = 0
        for prev in reversed(code[max(0, i - 8):i]):
            if prev.startswith("s_endpgm") or prev.startswith("s_branch"):
                break   # a block boundary: nothing before it falls through to the swap
            v = VALU_DST.match(prev)
            if v and waited < _VALU_WAITS and _vgprs(v.group(2)) & regs:
                hits.append(f"{prev}  ->({waited} wait states)->  {ln}")
                break
            if prev.startswith("v_cmpx") and waited < _VCMPX_WAITS:
                hits.append(f"{prev}  ->({waited} wait states, exec)->  {ln}")
                break
            waited += _wait_states(prev)
            if waited >= _VCMPX_WAITS:
                break
    return n, hits


def test_permlane_swap_operands_are_not_written_within_the_hazard_window(tmp_path):
    objs = sorted(OBJ_DIR.glob("*.o"))
    if not objs or not (LLVM / "llvm-objdump").exists() or shutil.which(str(LLVM / "clang-offload-bundler")) is None:
        pytest.skip("built objects or the ROCm LLVM tools are not here (run build() first)")
    swaps, hits = 0, []
    for obj in objs:
        n, h = _permlane_swap_hazards(_disassemble(obj, tmp_path))
        swaps += n
        hits += [f"{obj.name}: {x}" for x in h]
    assert swaps > 0, "no lane swaps found: the attention kernels' row-maximum exchange should use them"
    assert not hits, "\n".join(hits)


def test_the_swap_check_finds_the_pattern():
    """The scanner itself: a write one wait state before the swap (the reverted variant's pattern) and
    a v_cmpx within 4 are caught; s_nop 1 (2 wait states) after the last write passes."""
    one = ["v_mov_b32_e32 v128, v127", "s_nop 0", "v_permlane32_swap_b32_e32 v128, v127"]
    ok = ["v_max3_f32 v127, v127, v64, v128", "v_mov_b32_e32 v128, v127", "s_nop 1",
          "v_permlane32_swap_b32_e32 v128, v127"]
    cmpx = ["v_cmpx_gt_f32_e32 vcc, v1, v2", "s_nop 1", "v_permlane32_swap_b32_e32 v8, v9"]
    other_reg = ["v_mov_b32_e32 v5, v127", "v_permlane32_swap_b32_e32 v128, v127"]
    assert _permlane_swap_hazards(one)[1] and _permlane_swap_hazards(cmpx)[1]
    assert not _permlane_swap_hazards(ok)[1] and not _permlane_swap_hazards(other_reg)[1]
