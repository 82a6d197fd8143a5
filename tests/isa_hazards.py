"""Checks of the gfx950 code object built here for two instruction hazards that the
compiler guards only in code it can see, not inside inline assembly (test support).

* M0 -> LDS DMA: a scalar write of M0 needs one wait state before an LDS DMA
  (``buffer_load ... lds``), which reads M0 as its LDS address.  The compiler inserts
  ``s_nop 0`` for its own LDS-DMA builtin; the DMA-fed kernels issue the DMA as inline
  assembly and carry the ``s_nop 0`` in it.
* 16-byte store data: a vector-memory store of more than 8 bytes reads its data
  registers after it issues, and a VALU write of those registers needs two wait states
  after the store on gfx940 and later.  An inline-assembly store gets none from the
  compiler; the kernels' stores are builtins.

Both rules are LLVM's AMDGPU hazard recognizer's for this target (the M0 rule checked
on a probe built here: the compiler separates an M0 write from the builtin DMA after
it).  The code object is extracted from the built library's ``.hip_fatbin`` section with
the ROCm LLVM tools (``llvm-objcopy``, ``clang-offload-bundler``, ``llvm-objdump``).
The scan is linear, in address order within each function: a wait state counts one
per instruction, ``s_nop N`` counts N + 1.
"""

from __future__ import annotations

import os
import re
import subprocess
import tempfile
from pathlib import Path

LLVM_BIN = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

STORE_DATA_WAIT_STATES = 2
M0_DMA_WAIT_STATES = 1

_FUNC = re.compile(r"^[0-9a-f]+ <(.+)>:$")
_INST = re.compile(r"^\s+([a-z_][a-z0-9_]*)\s*(.*?)\s*(?://.*)?$")
_VREG = re.compile(r"^v(\d+)$|^v\[(\d+):(\d+)\]$")

# stores whose data is more than 8 bytes, and which operand holds the data
_WIDE_STORES = {
    "buffer_store_dwordx3": 0, "buffer_store_dwordx4": 0,
    "global_store_dwordx3": 1, "global_store_dwordx4": 1,
    "flat_store_dwordx3": 1, "flat_store_dwordx4": 1,
    "scratch_store_dwordx3": 1, "scratch_store_dwordx4": 1,
}


def tools_available() -> bool:
    return all((LLVM_BIN / t).exists() for t in ("llvm-objcopy", "clang-offload-bundler",
                                                  "llvm-objdump"))


def disassemble_library(lib: Path) -> list[str]:
    """Disassembly text of every gfx950 code object in the library's fat binary."""
    out = []
    with tempfile.TemporaryDirectory() as tmp:
        tmp = Path(tmp)
        fatbin = tmp / "fatbin.bin"
        subprocess.run([str(LLVM_BIN / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}",
                        str(lib), str(tmp / "copy.so")], check=True, capture_output=True)
        data = fatbin.read_bytes()
        starts = [m.start() for m in re.finditer(re.escape(BUNDLE_MAGIC), data)] + [len(data)]
        for k in range(len(starts) - 1):
            bundle = tmp / f"b{k}.bin"
            bundle.write_bytes(data[starts[k]:starts[k + 1]])
            co = tmp / f"co{k}.elf"
            subprocess.run([str(LLVM_BIN / "clang-offload-bundler"), "--unbundle", "--type=o",
                            f"--input={bundle}", f"--targets={TARGET}", f"--output={co}"],
                           check=True, capture_output=True)
            if co.stat().st_size == 0:
                continue
            dis = subprocess.run([str(LLVM_BIN / "llvm-objdump"), "-d", "--mcpu=gfx950", str(co)],
                                 check=True, capture_output=True, text=True)
            out.append(dis.stdout)
    return out


def parse(text: str) -> list[list[tuple[str, list[str]]]]:
    """Functions of a disassembly, each a list of (mnemonic, operands) in address order."""
    funcs, cur = [], None
    for line in text.splitlines():
        if _FUNC.match(line.strip()):
            cur = []
            funcs.append(cur)
            continue
        if cur is None:
            continue
        m = _INST.match(line)
        if not m:
            continue
        ops = [o.strip() for o in m.group(2).split(",")] if m.group(2) else []
        cur.append((m.group(1), ops))
    return funcs


def _wait_states(mnemonic: str, ops: list[str]) -> int:
    if mnemonic == "s_nop":
        return int(ops[0], 0) + 1
    return 1


def _vregs(op: str) -> set[int]:
    m = _VREG.match(op.split()[0]) if op else None
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def _is_lds_dma(mnemonic: str, ops: list[str]) -> bool:
    return (mnemonic.startswith(("buffer_load", "global_load"))
            and any(o.split()[-1] == "lds" for o in ops if o))


def m0_dma_violations(func) -> list[int]:
    """Indices of LDS DMA instructions with an M0 write less than the required wait
    states before them."""
    bad = []
    for i, (mn, ops) in enumerate(func):
        if not _is_lds_dma(mn, ops):
            continue
        ws = 0
        for j in range(i - 1, -1, -1):
            pmn, pops = func[j]
            if ws >= M0_DMA_WAIT_STATES:
                break
            if pmn.startswith("s_") and pops and pops[0] == "m0":
                bad.append(i)
                break
            ws += _wait_states(pmn, pops)
    return bad


def store_data_violations(func) -> list[int]:
    """Indices of stores of more than 8 bytes whose data registers a VALU instruction
    writes less than the required wait states after them."""
    bad = []
    for i, (mn, ops) in enumerate(func):
        slot = _WIDE_STORES.get(mn)
        if slot is None or len(ops) <= slot:
            continue
        data = _vregs(ops[slot])
        ws = 0
        for j in range(i + 1, len(func)):
            if ws >= STORE_DATA_WAIT_STATES:
                break
            nmn, nops = func[j]
            if nmn.startswith("v_") and nops and _vregs(nops[0]) & data:
                bad.append(i)
                break
            ws += _wait_states(nmn, nops)
    return bad


def scan(texts: list[str]) -> dict:
    """Counts of LDS DMA instructions and wide stores, and the violations found."""
    res = {"lds_dma": 0, "wide_stores": 0, "m0_dma": [], "store_data": []}
    for text in texts:
        for func in parse(text):
            res["lds_dma"] += sum(1 for mn, ops in func if _is_lds_dma(mn, ops))
            res["wide_stores"] += sum(1 for mn, _ in func if mn in _WIDE_STORES)
            res["m0_dma"] += [func[i] for i in m0_dma_violations(func)]
            res["store_data"] += [func[i] for i in store_data_violations(func)]
    return res
