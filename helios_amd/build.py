"""Build the gfx950 shared library ``libhelios_paged.so`` in-tree with hipcc.

The library exports the C ABI declared in ``include/helios_paged.h``. It is built
from the ``.hip`` sources under ``helios_amd/csrc`` for gfx950 only, with packed
FP32 instructions disabled and device code in non-IEEE mode (no NaN operands are
assumed), and written next to this file so that it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = PACKAGE_DIR.parent / "include"
LIBRARY = PACKAGE_DIR / "libhelios_paged.so"
SOURCES = ("kv_ops.hip", "paged_attn.hip", "tick_meta.hip", "qk_rope.hip", "logits.hip")
ARCH = "gfx950"


def hipcc_path() -> str:
    explicit = os.environ.get("HIPCC")
    if explicit:
        return explicit
    found = shutil.which("hipcc")
    return found or "/opt/rocm/bin/hipcc"


def compile_command(output: Path, *, resource_usage: bool = False) -> list[str]:
    cmd = [
        hipcc_path(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # Device code: no NaN operands are assumed and IEEE mode is off, so fmaxf on MFMA
        # results needs no canonicalising pass per element.
        "-Xarch_device", "-fno-honor-nans", "-Xarch_device", "-mno-amdgpu-ieee",
        f"-I{INCLUDE}",
        "-o", str(output),
    ]
    if resource_usage:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    cmd.extend(str(CSRC / name) for name in SOURCES)
    return cmd


def build(*, verbose: bool = False, resource_usage: bool = False) -> Path:
    """Compile every source into ``LIBRARY`` (always recompiles)."""
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = compile_command(tmp, resource_usage=resource_usage)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr, flush=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose=True, resource_usage="--resource-usage" in sys.argv)
    print(path)
