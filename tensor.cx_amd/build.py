"""Builds the hip device in-tree.

    python tensor.cx_amd/build.py            # HIP library + C++ backend/bindings
    python tensor.cx_amd/build.py --hip-only

Outputs (git-ignored, shipped with the tree to the GPU box):
  tensor.cx_amd/lib/libtensorcx_hip.so   HIP kernels + C ABI (hipcc, gfx950)
  tensor.cx_amd/python/tensorcx/_core*.so  HipBackend (C++20) + pybind11 bindings
"""

from __future__ import annotations

import argparse
import concurrent.futures as futures
import os
import pathlib
import subprocess
import sys
import sysconfig

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}", "-Wall", "-Wno-unused-result",
]
CXX_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-result"]


def run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + result.stdout + result.stderr)
        raise SystemExit(f"build failed: {cmd[0]} {cmd[-1]}")
    noisy = [line for line in (result.stderr or "").splitlines()
             if "packed-fp32-ops" not in line and line.strip()]
    if noisy:
        sys.stderr.write("\n".join(noisy) + "\n")


def build_hip() -> pathlib.Path:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objects = [OBJ / (src.stem + ".o") for src in sources]
    with futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        list(pool.map(lambda so: run([HIPCC, *HIP_FLAGS, "-c", str(so[0]), "-o", str(so[1])]),
                      zip(sources, objects)))
    target = LIB / "libtensorcx_hip.so"
    tmp = LIB / "libtensorcx_hip.so.tmp"
    run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)])
    tmp.replace(target)
    return target


def build_backend() -> pathlib.Path:
    import pybind11

    cpp = PKG / "cpp"
    sources = sorted((cpp / "tensorcx").rglob("*.cpp")) + sorted((PKG / "bindings").glob("*.cpp"))
    include = [f"-I{cpp}", f"-I{ROOT / 'include'}", f"-I{pybind11.get_include()}",
               f"-I{sysconfig.get_paths()['include']}"]
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    target = PKG / "python" / "tensorcx" / f"_core{suffix}"
    objects = []
    OBJ.mkdir(exist_ok=True)
    jobs = []
    for src in sources:
        obj = OBJ / ("cxx_" + "_".join(src.relative_to(PKG).with_suffix(".o").parts))
        objects.append(obj)
        jobs.append(["g++", *CXX_FLAGS, *include, "-c", str(src), "-o", str(obj)])
    with futures.ThreadPoolExecutor(max_workers=8) as pool:
        list(pool.map(run, jobs))
    tmp = target.with_suffix(".tmp")
    run(["g++", "-shared", "-o", str(tmp), *map(str, objects), f"-L{LIB}", "-ltensorcx_hip",
         "-Wl,-rpath,$ORIGIN/../../lib", "-pthread"])
    tmp.replace(target)
    return target


def build_contract() -> pathlib.Path:
    """The backend ABI contract program (tests/cpp/hip_backend_contract.cpp),
    linked against the backend objects of build_backend and the HIP library,
    into tests/cpp/_bin/ (built here, run by the tests on CPU and GPU)."""
    cpp = PKG / "cpp"
    test_dir = ROOT / "tests" / "cpp"
    out_dir = test_dir / "_bin"
    out_dir.mkdir(exist_ok=True)
    objects = sorted(OBJ.glob("cxx_cpp_*.o"))
    if not objects:
        raise SystemExit("build_contract needs build_backend first")
    target = out_dir / "hip_backend_contract"
    tmp = out_dir / "hip_backend_contract.tmp"
    run(["g++", *CXX_FLAGS, f"-I{cpp}", f"-I{ROOT / 'include'}", "-o", str(tmp),
         str(test_dir / "hip_backend_contract.cpp"), *map(str, objects), f"-L{LIB}", "-ltensorcx_hip",
         "-Wl,-rpath,$ORIGIN/../../../tensor.cx_amd/lib", "-pthread"])
    tmp.replace(target)
    return target


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--hip-only", action="store_true")
    args = parser.parse_args()
    print(build_hip())
    if not args.hip_only:
        print(build_backend())
        print(build_contract())


if __name__ == "__main__":
    main()
