"""Hardware probes behind the kernel's design (microbench/cdna4_probes.hip): build and run.

``python -m trianglemix.microbench`` compiles the probes for gfx950 (when the
binary is missing or older than its source) and runs them on the current GPU:
L2 -> CU bandwidth of LDS DMA and VGPR loads against loads in flight, LDS
read bandwidth while other waves stream DMA, MFMA issue rate with independent
VALU instructions between MFMAs, the attention loop body's time and shader
clock on zero and random K/V, the chip's MFMA rate and clock at full load
on zero and random operands, and the per-launch floor of a near-empty kernel
in the attention kernel's workgroup shape, eager and as a HIP graph.
"""

from __future__ import annotations

import shutil
import subprocess
import sys
from pathlib import Path

SOURCE = Path(__file__).resolve().parents[1] / "microbench" / "cdna4_probes.hip"
BINARY = SOURCE.with_suffix("")


def build() -> Path:
    if BINARY.is_file() and BINARY.stat().st_mtime >= SOURCE.stat().st_mtime:
        return BINARY
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", str(SOURCE), "-o", str(BINARY)], check=True)
    return BINARY


def main() -> int:
    return subprocess.run([str(build())], check=False).returncode


if __name__ == "__main__":
    raise SystemExit(main())
