"""Builds the HIP env library (gfx950) and, for tests only, the CPU oracles.

    python -m neurips2026_smart_building_challenge_amd.build

Outputs, in-tree so they travel with the repository snapshot:
    neurips2026_smart_building_challenge_amd/libsbenv.so   product (HIP + C ABI)
    neurips2026_smart_building_challenge_amd/libsbenv_big.so   the same with SB_CONT_BIG
                                                           (320 continuous action heads)
    oracle/liboracle.so, liboracle_big.so                  C restatement (tests)
    oracle/_ref/libcsim_ref.so                             reference csim (tests,
                                                           only where /root/reference exists)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libsbenv.so"
LIB_BIG = PKG / "libsbenv_big.so"   # SB_CONT_BIG: 320 continuous action heads
ARCH = os.environ.get("SBENV_ARCH", "gfx950")
REF_CSIM = Path("/root/reference/complete_port/csim")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# the field step and the field envs' HVAC lanes are bit-exact to the reference
# core only with products rounded before they are added
EXTRA = {"fdm_kernel.hip": ["-ffp-contract=off"], "field_env_kernel.hip": ["-ffp-contract=off"]}


HIP_SOURCES = ["step_kernel.hip", "policy_kernel.hip", "canon_kernel.hip", "fdm_kernel.hip", "field_env_kernel.hip"]
HOST_SOURCES = ["vec.cpp", "plan.cpp", "sbb_reader.cpp", "fdm.cpp", "field_env.cpp"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")


def build_product() -> Path:
    """Both libraries: libsbenv.so (256 + 16 action heads) and libsbenv_big.so
    (-DSB_CONT_BIG: 320 + 16, the reference GPU env's SB_CONT_BIG layout)."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    inc = ["-I", str(ROOT / "include"), "-I", str(CSRC)]
    rocm = Path(hipcc).resolve().parent.parent
    jobs, links = [], []   # (command, object): every translation unit compiles independently
    for lib, tmp, defs in ((LIB, PKG / "_build", []), (LIB_BIG, PKG / "_build_big", ["-DSB_CONT_BIG"])):
        tmp.mkdir(exist_ok=True)
        objs = []
        for src in HIP_SOURCES:
            o = tmp / (Path(src).stem + ".o")
            jobs.append([hipcc, *HIP_FLAGS, *EXTRA.get(src, []), *defs, *inc, "-c", str(CSRC / src), "-o", str(o)])
            objs.append(o)
        for src in HOST_SOURCES:
            # host-only C++ (HIP runtime API calls, no device code)
            o = tmp / (Path(src).stem + ".o")
            jobs.append(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__", *defs,
                         "-I", str(rocm / "include"), *inc, "-c", str(CSRC / src), "-o", str(o)])
            objs.append(o)
        links.append((lib, objs))
    workers = max(1, min(len(jobs), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for f in [pool.submit(_run, cmd) for cmd in jobs]:
            f.result()
    for lib, objs in links:
        out_tmp = lib.with_suffix(".so.tmp")
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(out_tmp)])
        out_tmp.replace(lib)
    return LIB


def build_oracles() -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "oracle"])
    if REF_CSIM.is_dir():
        _run(["make", "-s", "-C", str(ROOT / "oracle"), "ref", f"REF={REF_CSIM}"])


def build() -> None:
    build_product()
    build_oracles()


if __name__ == "__main__":
    build()
    print("built", LIB)
