"""Build the gfx950 HIP library and its PyTorch-ROCm adapter in-tree.

Outputs (next to the Python package, git-ignored, shipped with the tree):

* ``trianglemix/libtrianglemix.so``        -- HIP kernels + C ABI (hipcc, gfx950)
* ``trianglemix/_trianglemix_torch.so``    -- torch.ops registrations (g++),
  linked to the library above through ``$ORIGIN``

Usage: ``python build.py [--hip-only]``.  Each call recompiles.
``python build.py --phase-clocks`` builds the diagnostic phase-clock library
``trianglemix/libtrianglemix_phase_clocks.so`` instead: a diagnostic build whose kernels store
per-wave ``s_memrealtime`` clocks at phase boundaries (exports ``tm_phase_clocks_read`` / ``_clear``).
``python build.py --plan-override`` builds ``trianglemix/libtrianglemix_plan_override.so``: the product
library plus a ``tm_plan_override(kv_parts, tiles_per_split)`` export that forces every call's launch plan,
for the forced-plan sweep the planner's costs are fitted to (``tests/plan_sweep.py``).
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
PKG = HERE / "trianglemix"
INCLUDE = HERE.parent / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIP_LIB = PKG / "libtrianglemix.so"
PHASE_CLOCK_LIB = PKG / "libtrianglemix_phase_clocks.so"  # diagnostic build (--phase-clocks), not loaded by the op
PLAN_OVERRIDE_LIB = PKG / "libtrianglemix_plan_override.so"  # diagnostic build (--plan-override), not loaded by the op
TORCH_LIB = PKG / "_trianglemix_torch.so"

# Disable packed fp32 VALU ops in device code: some of their forms have given
# wrong results on this hardware class, silently.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Keep MFMA accumulators in VGPRs: the softmax rescales them every tile,
    # and VALU cannot operate on AGPRs without copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # Preload the attention kernel's leading scalar arguments (the fields its
    # prologue needs first) into SGPRs at wave launch; 16 dwords is the most
    # the user SGPRs hold, and only scalar arguments qualify.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # Device code only: no NaN operands, so fmaxf needs no quieting
    # canonicalisation of its inputs (which doubled the row-max work).  The
    # kernels never form NaN themselves (masked scores are -inf and an
    # all-masked row's max is taken as 0).  Host code keeps IEEE NaN
    # semantics: the C ABI rejects a NaN scale.
    "-Xarch_device", "-fno-honor-nans",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # The host compilation pass does not know the device-only feature; that
    # warning is expected and filtered.
    lines = [ln for ln in proc.stdout.splitlines() if "is not a recognized feature" not in ln]
    if proc.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd[:3])} ...")
    if lines:
        sys.stdout.write("\n".join(lines) + "\n")


def _atomic_replace(tmp: Path, dst: Path) -> None:
    os.replace(tmp, dst)


def build_hip_library(phase_clocks: bool = False, plan_override: bool = False) -> Path:
    """The kernels + C ABI; ``phase_clocks`` builds the diagnostic variant that records per-wave phase clocks
    (read back through its ``tm_phase_clocks_read`` export), ``plan_override`` the one whose
    ``tm_plan_override`` export forces the launch plan, each into its own file."""
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    dst = PHASE_CLOCK_LIB if phase_clocks else (PLAN_OVERRIDE_LIB if plan_override else HIP_LIB)
    tmp = dst.with_suffix(".so.tmp")
    defines = (["-DTRIANGLEMIX_PHASE_CLOCKS"] if phase_clocks else []) + (["-DTRIANGLEMIX_PLAN_OVERRIDE"] if plan_override else [])
    _run([hipcc, *HIP_FLAGS, *defines, "-shared", f"-I{INCLUDE}",
          str(CSRC / "trianglemix_kernel.hip"), str(CSRC / "trianglemix_cache.hip"), str(CSRC / "trianglemix_capi.cpp"),
          "-o", str(tmp)])
    _atomic_replace(tmp, dst)
    return dst


def build_torch_adapter() -> Path:
    import torch
    from torch.utils import cpp_extension

    cxx = os.environ.get("CXX", "g++")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths()]
    incs += [f"-I{sysconfig.get_paths()['include']}", f"-I{ROCM / 'include'}", f"-I{INCLUDE}"]
    torch_lib = Path(cpp_extension.library_paths()[0])
    tmp = TORCH_LIB.with_suffix(".so.tmp")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared",
          f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
          *incs, str(CSRC / "trianglemix_torch.cpp"),
          f"-L{PKG}", "-ltrianglemix",
          f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-ltorch_python",
          f"-L{ROCM / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}", f"-Wl,-rpath,{ROCM / 'lib'}",
          "-o", str(tmp)])
    _atomic_replace(tmp, TORCH_LIB)
    return TORCH_LIB


def build_all(hip_only: bool = False) -> list[Path]:
    out = [build_hip_library()]
    if not hip_only:
        out.append(build_torch_adapter())
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--hip-only", action="store_true")
    ap.add_argument("--phase-clocks", action="store_true",
                    help="build only the diagnostic phase-clock library (libtrianglemix_phase_clocks.so)")
    ap.add_argument("--plan-override", action="store_true",
                    help="build only the diagnostic plan-override library (libtrianglemix_plan_override.so)")
    args = ap.parse_args()
    if args.phase_clocks:
        print(f"built {build_hip_library(phase_clocks=True)}")
        return 0
    if args.plan_override:
        print(f"built {build_hip_library(plan_override=True)}")
        return 0
    for p in build_all(args.hip_only):
        print(f"built {p}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
