"""Build libwanmi.so (every HIP kernel of the package) for gfx950 with hipcc.

Each ``csrc/*.hip`` file is compiled to an object under ``_build/`` (in parallel), then linked
into ``libwanmi.so`` next to this file, where :mod:`._lib` loads it. Always rebuilds.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import re
import shutil
import subprocess

PKG_DIR = pathlib.Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libwanmi.so"
INCLUDE_DIR = PKG_DIR.parent / "include"

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Packed-fp32 VALU ops stay disabled: the compiler's scalar/float2 code is used instead.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the gfx950 kernels cannot be built")


_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b|\b(vcc_lo|vcc_hi|vcc)\b")
_VCC = {"vcc_lo": {106}, "vcc_hi": {107}, "vcc": {106, 107}}


def _sgprs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _SREG.finditer(text):
        if m.group(1):
            out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
        elif m.group(3):
            out.add(int(m.group(3)))
        else:
            out |= _VCC[m.group(4)]
    return out


def dma_sgpr_hazards(asm: str, window: int = 5) -> list[str]:
    """Direct-to-LDS loads of `asm` (gfx950 device assembly) that may read an SGPR a vector
    instruction wrote fewer than `window` wait states before (the hardware needs five; the compiler
    does not check inline asm). Conservative: any vector instruction naming one of the load's SGPRs
    counts, and a label or branch inside the window counts as a hazard."""
    lines = [ln.split(";")[0].strip() for ln in asm.splitlines()]
    found = []
    for i, ln in enumerate(lines):
        if not ln.startswith("buffer_load") or " lds" not in ln:
            continue
        used = _sgprs(ln.split(None, 1)[1])
        states, j = 0, i - 1
        while states < window and j >= 0:
            prev = lines[j]
            j -= 1
            if not prev or prev.startswith((".", "#")) and not prev.endswith(":"):
                continue
            if prev.endswith(":") or prev.startswith(("s_branch", "s_cbranch", "s_setpc", "s_swappc")):
                found.append(f"{ln}  (block boundary {window - states} wait states before it)")
                break
            op = prev.split()[0]
            if op == "s_nop":
                states += int(prev.split()[1], 0) + 1
                continue
            if op.startswith("v_") and _sgprs(prev[len(op):]) & used:
                found.append(f"{ln}  (after {prev})")
                break
            states += 1
    return found


_VREG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")


def _vgprs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _VREG.finditer(text):
        if m.group(1):
            out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def store_data_hazards(asm: str, window: int = 2) -> list[str]:
    """Vector stores wider than 64 bits in `asm` (gfx950 device assembly) whose data VGPRs a VALU
    instruction overwrites fewer than `window` wait states later. The store reads its data after it
    issues; overwritten too soon, some lanes store the new value. The compiler's own hazard check has
    missed this (an adaLN store followed directly by a move into one of its data registers), so
    every kernel's generated code is checked."""
    lines = [ln.split(";")[0].strip() for ln in asm.splitlines()]
    labels = {ln[:-1]: k for k, ln in enumerate(lines) if ln.endswith(":") and not ln.startswith(".")
              or ln.startswith(".LBB") and ln.endswith(":")}

    def scan(j: int, states: int, data: set, store: str, found: list, seen: set) -> None:
        # every instruction that may execute within `window` wait states of the store, along each
        # control-flow path: an unconditional branch continues at its target, a conditional one at
        # both its target and the next instruction
        while states < window and j < len(lines):
            if (j, states) in seen:
                return
            seen.add((j, states))
            nxt = lines[j]
            j += 1
            if not nxt or nxt.startswith((".", "#")) and not nxt.endswith(":") or nxt.endswith(":"):
                continue
            nop = nxt.split()[0]
            if nop == "s_nop":
                states += int(nxt.split()[1], 0) + 1
                continue
            if nop.startswith("v_") and _vgprs(nxt[len(nop):].split(",")[0]) & data:
                found.append(f"{store}  (then {nxt}, {states} wait states)")
                return
            if nop in ("s_endpgm", "s_setpc_b64"):
                return
            if nop == "s_branch" or nop.startswith("s_cbranch"):
                target = labels.get(nxt.split()[1])
                if target is None:  # an unknown target: assume the worst (keep scanning linearly)
                    states += 1
                    continue
                scan(target + 1, states + 1, data, store, found, seen)
                if nop == "s_branch":
                    return
            states += 1

    found = []
    for i, ln in enumerate(lines):
        op = ln.split()[0] if ln else ""
        if not op.startswith(("buffer_store", "global_store", "flat_store", "scratch_store")):
            continue
        if not any(w in op for w in ("dwordx3", "dwordx4", "b96", "b128")):
            continue
        operands = [o.strip() for o in ln[len(op):].split(",")]
        data = _vgprs(operands[0] if op.startswith("buffer") else operands[1])
        hits: list = []
        scan(i + 1, 0, data, ln, hits, set())
        found.extend(hits[:1])
    return found


def _compile_once(src: pathlib.Path, obj: pathlib.Path, extra: list[str]) -> None:
    cmd = [_hipcc(), *HIP_FLAGS, *extra, f"-I{INCLUDE_DIR}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")


def _device_asm(src: pathlib.Path, extra: list[str]) -> str:
    out = BUILD_DIR / (src.stem + ".s")
    cmd = [_hipcc(), *HIP_FLAGS, *extra, f"-I{INCLUDE_DIR}", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{res.stderr}")
    return out.read_text()


def _compile(src: pathlib.Path) -> pathlib.Path:
    """Compiles one source and checks its generated code. A source with hot-loop direct-to-LDS loads
    (one wait state) is rebuilt with WANMI_DMA_ALL_WAITS (five wait states everywhere) if any load may
    read an SGPR a vector instruction just wrote. A wide store whose data registers are overwritten
    too soon fails the build."""
    obj = BUILD_DIR / (src.stem + ".o")
    _compile_once(src, obj, [])
    asm = _device_asm(src, [])
    if "lds_dma_b128_hot" in src.read_text() and dma_sgpr_hazards(asm):
        safe = ["-DWANMI_DMA_ALL_WAITS"]
        _compile_once(src, obj, safe)
        asm = _device_asm(src, safe)
        left = dma_sgpr_hazards(asm)
        if left:
            raise RuntimeError(f"{src.name}: direct-to-LDS loads read freshly written SGPRs:\n" + "\n".join(left[:5]))
    bad = store_data_hazards(asm)
    if bad:
        raise RuntimeError(f"{src.name}: store data overwritten before the store read it:\n" + "\n".join(bad[:5]))
    return obj


def build_library(jobs: int | None = None) -> pathlib.Path:
    """Compile and link libwanmi.so; returns its path. Raises on any compiler error."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libwanmi.so failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library())
