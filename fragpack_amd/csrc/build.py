"""Builds libfragpack_hip.so (gfx950) in-tree: ``python -m fragpack_amd.csrc.build``.

One hipcc invocation over the HIP sources and the C-ABI glue; the library
lands in fragpack_amd/_lib/.  Packed FP32 instruction selection is turned off
(-packed-fp32-ops) for every device compile.
"""

from __future__ import annotations

import os
from pathlib import Path
import subprocess
import sys

CSRC = Path(__file__).resolve().parent
ROOT = CSRC.parent.parent
OUT = CSRC.parent / "_lib" / "libfragpack_hip.so"
SOURCES = ["fp_attn.hip", "fp_store.hip", "fp_prefill.hip", "fp_paged.hip", "fp_capi.cpp"]
ARCH = os.environ.get("FRAGPACK_ARCH", "gfx950")


def command(out: Path = OUT) -> list[str]:
    return [
        os.environ.get("HIPCC", "/opt/rocm/bin/hipcc"),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # the kernels never produce or test for NaN; without this every
        # fmaxf of an MFMA result is preceded by a canonicalising v_max
        "-fno-honor-nans",
        "-Wno-unused-command-line-argument",
        f"-I{ROOT / 'include'}",
        "-o", str(out),
        *[str(CSRC / s) for s in SOURCES],
    ]


def build(out: Path = OUT, verbose: bool = False) -> Path:
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    proc = subprocess.run(command(tmp), capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed ({proc.returncode}) building {out.name}")
    if verbose:
        sys.stderr.write(proc.stderr)
    tmp.replace(out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
