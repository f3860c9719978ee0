"""Build libmdlarc_hip.so (the C-ABI kernel library) in-tree with hipcc for gfx950.

    python -m mdlarc_scale_amd.build        # compile every csrc/*.hip, link the shared library

The library is written next to this file so it travels with the source tree; object files go to
``_build/`` beside it.  No CMake: each translation unit is self-contained device + host code.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_NAME = "libmdlarc_hip.so"
LIB_PATH = PKG / LIB_NAME
ARCH = "gfx950"

SOURCES = [
    "norm_embed.hip",
    "rope_cache.hip",
    "swiglu.hip",
    "attn_decode.hip",
    "attn_prefill.hip",
    "attn_f32.hip",
    "head_state.hip",
    "prompt_build.hip",
    "split_gemm.hip",
    "prefill_gemm.hip",
]

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops are kept out of every kernel (they have produced silent wrong results
    # on this hardware pool); hipcc's host pass warns that it does not know the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libmdlarc_hip.so)")


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n"
                           f"{res.stdout}\n{res.stderr}")
    noisy = [ln for ln in res.stderr.splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "remark:" not in ln
             and "'--hip-link'" not in ln]   # hipcc adds it to the device-only assembly pass
    if noisy:
        print("\n".join(noisy), file=sys.stderr)
    return res.stderr


# Kernels that copy global memory straight into LDS by inline assembly (lds_dma.h) wait for those
# copies with their own s_waitcnt; they are only ever run without register spills, so their files
# are compiled with the resource report and any scratch use fails the build.  The copies also
# write M0 behind the compiler's back, so the device assembly of those files is read as well and
# any compiler-generated instruction naming M0 fails the build (check_m0).
DMA_HEADER = "lds_dma.h"
_SCRATCH = re.compile(r"ScratchSize \[bytes/lane\]: (\d+)")
_FUNC = re.compile(r"Function Name: (\S+)")
_M0 = re.compile(r"\bm0\b")
# opcodes that read M0 without naming it (relative register indexing, messages, GWS / ordered
# LDS ops, LDS-address-by-lane ops, LDS copies, interpolation)
_M0_IMPLICIT = re.compile(r"^(v_movrel|s_movrel|s_set_gpr_idx|s_sendmsg|s_ttracedata|ds_gws|"
                          r"ds_append|ds_consume|ds_ordered|ds_\w*addtid|v_interp|"
                          r"global_load_lds|buffer_load\w*.*\blds\b)")


def _uses_dma(src: Path) -> bool:
    return f'#include "{DMA_HEADER}"' in src.read_text()


def check_no_scratch(report: str, src: str) -> None:
    """Raise if the compiler's resource report for ``src`` gives any kernel scratch memory."""
    func = "?"
    for ln in report.splitlines():
        m = _FUNC.search(ln)
        if m:
            func = m.group(1)
            continue
        m = _SCRATCH.search(ln)
        if m and int(m.group(1)) != 0:
            raise RuntimeError(f"{src}: kernel {func} uses {m.group(1)} bytes of scratch per lane; "
                               f"kernels including {DMA_HEADER} must not spill")


def check_m0(asm: str, src: str) -> None:
    """Raise if any instruction of the device assembly ``asm`` outside an inline-asm block names
    M0: the LDS copies of lds_dma.h set M0 without the compiler knowing, which is only safe while
    the compiler keeps nothing of its own there.  Inside the blocks only the copies' own
    ``s_mov_b32 m0, <sgpr>`` may appear."""
    inside = False
    for n, ln in enumerate(asm.splitlines(), 1):
        code = ln.split(";", 1)[0].strip()
        if ln.strip().startswith(";;#ASMSTART"):
            inside = True
            continue
        if ln.strip().startswith(";;#ASMEND"):
            inside = False
            continue
        if not code or code.startswith("."):
            continue
        if inside and (re.fullmatch(r"s_mov_b32\s+m0,\s*s\d+", code) or
                       code.startswith(("s_nop", "global_load_lds_dwordx4"))):
            continue
        if _M0.search(code) or _M0_IMPLICIT.match(code):
            raise RuntimeError(f"{src}: device assembly line {n} uses M0 outside the LDS-copy "
                               f"asm blocks ({code!r}); lds_dma.h's copies would clobber it")


def build(verbose: bool = False) -> Path:
    """Compile all kernels and link ``libmdlarc_hip.so``; returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]

    def compile_one(i: int) -> None:
        src = CSRC / SOURCES[i]
        dma = _uses_dma(src)
        cmd = [hipcc, *FLAGS,
               *(["-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"] if dma else []),
               "-c", str(src), "-o", str(objs[i])]
        if verbose:
            print(" ".join(cmd))
        report = _run(cmd)
        if dma:
            check_no_scratch(report, SOURCES[i])
            asm = BUILD / (Path(SOURCES[i]).stem + ".device.s")
            _run([hipcc, *FLAGS, "-S", "--cuda-device-only", str(src), "-o", str(asm)])
            check_m0(asm.read_text(), SOURCES[i])

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        list(ex.map(compile_one, range(len(SOURCES))))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
