"""Build step for the ROCm backend plugin: ``compile_rocm`` next to the
reference's ``compile_cpu``/``compile_cuda`` (build_ops.py:164-225).

hipcc compiles every ``mod_amd/csrc/*.hip`` for gfx950 into
``mod_amd/csrc/libtensor_ops_rocm.so`` -- the same ``<backend>/c_src/libtensor_ops_<target>.so``
shape the reference loader resolves (common/utils/lib_loader.py:13-37).
Cross-compiles without a GPU. Run as ``python -m mod_amd.build_ops``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libtensor_ops_rocm.so"
LIB_PATH = CSRC / LIB_NAME
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Never let the compiler form v_pk_{add,mul,fma}_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the ROCm plugin)")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(
            "command failed: " + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    # Surface compiler warnings other than the known host-pass note about the
    # packed-fp32 feature.
    noise = "packed-fp32-ops"
    lines = [l for l in (res.stdout + res.stderr).splitlines()
             if l.strip() and noise not in l and "is not a recognized feature" not in l]
    if lines and os.environ.get("PIO_BUILD_VERBOSE"):
        print("\n".join(lines), file=sys.stderr)


def compile_rocm(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources for gfx950 and link libtensor_ops_rocm.so."""
    cc = hipcc()
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    build_dir = CSRC / "_build"
    build_dir.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for s in srcs:
        o = build_dir / (s.stem + ".o")
        objs.append(o)
        cmds.append([cc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(s), "-o", str(o)])
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 8)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for fut in [ex.submit(_run, c) for c in cmds]:
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def main() -> int:
    compile_rocm(verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
