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
    flags = [f for f in fh_build.hip_flags(source) if f != "-fPIC"]
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
SPILL = re.compile(r"\bscratch_(store|load)|Folded (Spill|Reload)")

# Kernels on the measured paths: the P = 4 dense (buffer-to-LDS) and count-ordered kernels, the
# P = 8 and tile kernels, and the stream-mixing kernels.  A register spill inside their loops
# (where the per-group, per-matrix or per-token work runs) would add scratch traffic to every
# unit of work; the mixing kernels, which stream at the HBM rate, keep no scratch at all.
NO_SCRATCH = ("expm_p4_dma_kernel", "expm_p4_sort_kernel", "expm_oct_kernel", "expm_oct16", "expm_tile_kernel",
              "hc_mix_fwd_kernel", "hc_mix_bwd_kernel", "hc_wide_fwd_kernel", "hc_wide_bwd_kernel")
NO_SCRATCH_AT_ALL = ("hc_mix_fwd_kernel", "hc_mix_bwd_kernel", "hc_wide_fwd_kernel", "hc_wide_bwd_kernel")


def spills_in_loops(asm: str) -> dict[str, int]:
    """Per function, the spill and reload instructions inside a loop: in blocks the compiler's
    assembly annotates as a loop header or as in a loop."""
    found = {}
    for m in re.finditer(r"^(_Z\S+):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        in_loop, count = False, 0
        for line in asm[m.end():end if end >= 0 else None].splitlines():
            text = line.strip()
            if text.startswith(".LBB") or text.startswith("; %bb."):
                in_loop = "Loop" in text
            elif in_loop and SPILL.search(text):
                count += 1
        if count:
            found[m.group(1)] = count
    return found


def test_scanners_read_scratch_sizes_and_loop_spills():
    asm = ("\t.amdhsa_kernel _Zk1\n\t\t.amdhsa_group_segment_fixed_size 0\n\t\t.amdhsa_private_segment_fixed_size 64\n"
           "\t.amdhsa_kernel _Zk2\n\t\t.amdhsa_private_segment_fixed_size 0\n")
    assert KERNEL_SCRATCH.findall(asm) == [("_Zk1", "64"), ("_Zk2", "0")]
    body = ("_Zk1:\n\tv_mov_b32 v0, 0\n.LBB0_2:  ; =>This Loop Header: Depth=1\n\tv_add_f32 v1, v2, v3\n"
            "\tscratch_store_dword off, v4, off ; 4-byte Folded Spill\n; %bb.3:  ;   in Loop: Header=BB0_2 Depth=1\n"
            "\tscratch_load_dword v4, off, off ; 4-byte Folded Reload\n; %bb.4:\n"
            "\tscratch_store_dword off, v5, off ; 4-byte Folded Spill\n.Lfunc_end0:\n"
            "_Zk2:\n; %bb.0:\n\tscratch_store_dword off, v5, off ; 4-byte Folded Spill\n.Lfunc_end1:\n")
    assert spills_in_loops(body) == {"_Zk1": 2}


def test_measured_kernels_spill_nothing_inside_loops(assembly):
    sizes = {name: int(size) for text in assembly.values() for name, size in KERNEL_SCRATCH.findall(text)}
    hot = {name: size for name, size in sizes.items() if any(k in name for k in NO_SCRATCH)}
    assert len(hot) > 60, sorted(hot)  # every instantiation of those kernels was found
    loops = {}
    for text in assembly.values():
        loops.update(spills_in_loops(text))
    in_loops = {name: count for name, count in loops.items() if any(k in name for k in NO_SCRATCH)}
    assert not in_loops, in_loops
    streaming = {name: size for name, size in hot.items() if any(k in name for k in NO_SCRATCH_AT_ALL) and size}
    assert not streaming, streaming
