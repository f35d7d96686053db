"""Generated code: no wide vector store has its data overwritten by the next instruction, and
the kernels on the measured paths spill no registers to scratch.

A vector-memory store of more than 8 bytes reads its data registers after it
issues.  The compiler separates such a store from a following write of those
registers only when the store's scalar offset is the constant 0, and on gfx950
an overwrite that slipped through replaced the first dword of stored results
(csrc/fh_common.h, kStoreSOffset).  This compiles every kernel source for
gfx950 to assembly (no GPU needed) and checks each store of 12 or 16 bytes
against the instruction after it.
"""

import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "flash-hyperconnections_amd"))

import build as fh_build  # noqa: E402

WIDE_STORE = re.compile(r"(buffer|global|flat|scratch)_store_(dwordx3|dwordx4|b96|b128)\b")


def _vgprs(token: str) -> set[int]:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", token)
    return {int(m.group(1))} if m else set()


def overwritten_stores(asm: str) -> list[str]:
    """Wide stores whose next instruction is a VALU write to one of their data VGPRs."""
    lines = [ln.strip() for ln in asm.splitlines()]
    lines = [ln for ln in lines if ln and not ln.startswith((";", ".")) and not ln.endswith(":")]
    found = []
    for here, nxt in zip(lines, lines[1:]):
        op = here.split()[0]
        if not WIDE_STORE.match(op):
            continue
        operands = [t.strip() for t in here[len(op):].split(",")]
        # global_store vaddr, vdata, ...; the others put vdata first.
        data = _vgprs(operands[1] if op.startswith("global") else operands[0])
        if nxt.startswith("v_"):
            dest = nxt.split()[1].rstrip(",")
            if _vgprs(dest) & data:
                found.append(f"{here}  ->  {nxt}")
    return found


def test_scanner_flags_an_overwrite():
    asm = "buffer_store_dwordx4 v[0:3], v69, s[48:51], s0 offen nt\nv_or_b32_e32 v0, 16, v69\n"
    assert overwritten_stores(asm)
    assert not overwritten_stores(asm.replace("v_or_b32_e32 v0", "v_or_b32_e32 v4"))
    assert not overwritten_stores("buffer_store_dwordx2 v[0:1], v69, s[48:51], 0 offen\nv_mov_b32 v0, 1\n")


def _assembly(source: str, out: Path) -> str:
    flags = [f for f in fh_build.HIP_FLAGS if f != "-fPIC"]
    proc = subprocess.run([fh_build.HIPCC, *flags, "--cuda-device-only", "-S", str(fh_build.CSRC / source), "-o",
                           str(out)], capture_output=True, text=True)
    assert proc.returncode == 0, f"{source}: {proc.stderr[-2000:]}"
    return out.read_text()


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    """gfx950 assembly of every kernel source, compiled once for this module's tests."""
    out = tmp_path_factory.mktemp("asm")
    sources = [s for s in fh_build.KERNEL_SOURCES if s.endswith(".hip")]
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:  # one hipcc process per source
        return dict(zip(sources, pool.map(lambda s: _assembly(s, out / (s + ".s")), sources)))


def test_kernels_keep_store_data_until_read(assembly):
    found = [f"{src}: {hit}" for src, text in assembly.items() for hit in overwritten_stores(text)]
    assert not found, "\n".join(found[:5])


KERNEL_SCRATCH = re.compile(r"\.amdhsa_kernel (\S+)\n(?:.*\n)*?\s*\.amdhsa_private_segment_fixed_size (\d+)")

# Kernels on the measured paths: the P = 4 dense (buffer-to-LDS) and count-ordered kernels, the
# P = 8 and tile kernels, and the stream-mixing kernels.  Register spills there would add scratch
# traffic to the HBM-bound launches.
NO_SCRATCH = ("expm_p4_dma_kernel", "expm_p4_sort_kernel", "expm_oct_kernel", "expm_oct16", "expm_tile_kernel",
              "hc_mix_fwd_kernel", "hc_mix_bwd_kernel", "hc_wide_fwd_kernel", "hc_wide_bwd_kernel")


def test_scanner_reads_scratch_sizes():
    asm = ("\t.amdhsa_kernel _Zk1\n\t\t.amdhsa_group_segment_fixed_size 0\n\t\t.amdhsa_private_segment_fixed_size 64\n"
           "\t.amdhsa_kernel _Zk2\n\t\t.amdhsa_private_segment_fixed_size 0\n")
    assert KERNEL_SCRATCH.findall(asm) == [("_Zk1", "64"), ("_Zk2", "0")]


def test_measured_kernels_use_no_scratch(assembly):
    sizes = {name: int(size) for text in assembly.values() for name, size in KERNEL_SCRATCH.findall(text)}
    hot = {name: size for name, size in sizes.items() if any(k in name for k in NO_SCRATCH)}
    assert len(hot) > 60, sorted(hot)  # every instantiation of those kernels was found
    spilling = {name: size for name, size in hot.items() if size}
    assert not spilling, spilling
