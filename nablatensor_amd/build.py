"""In-tree build of the native parts of nablatensor_amd.

Outputs (next to their sources, git-ignored, shipped with the tree):
  nablatensor_amd/libnt_rocm.so        C-ABI engine (include/nablatensor_rocm.h)
  nablatensor_amd/_host*.so            pybind11 module over the C++ host layer
  nablatensor_amd/csrc/skeleton_src.inc the kernel skeleton embedded as a string

The replay kernels themselves are generated per tape and compiled for gfx950
with hipRTC at run time (cached under nablatensor_amd/_kcache/);
`check_offline_hipcc` additionally compiles the skeleton with a generated body
through hipcc --offload-arch=gfx950 as a build check.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
PACKED_FP32_OFF = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    res = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}")


def _newer(target: Path, sources: list[Path]) -> bool:
    if not target.exists():
        return False
    t = target.stat().st_mtime
    return all(s.stat().st_mtime <= t for s in sources)


def embed_skeleton() -> Path:
    src = (CSRC / "nt_skeleton.h").read_text()
    tables = (CSRC / "nt_math_tables.h").read_text()
    out = CSRC / "skeleton_src.inc"
    text = ("// generated from nt_skeleton.h and nt_math_tables.h by nablatensor_amd/build.py; do not edit\n"
            f'static const char NT_SKELETON_SRC[] = R"NTSKEL({src})NTSKEL";\n'
            f'static const char NT_MATH_TABLES_SRC[] = R"NTSKEL({tables})NTSKEL";\n')
    if not out.exists() or out.read_text() != text:
        out.write_text(text)
    return out


def build_engine(force: bool = True) -> Path:
    """libnt_rocm.so: the host C++ (g++) plus nt_noalloc.hip, whose static
    device array needs a hipcc object for gfx950 linked into the library."""
    inc = embed_skeleton()
    out = PKG / "libnt_rocm.so"
    srcs = [CSRC / "nt_rocm.cpp", CSRC / "lower.cpp"]
    hip_src = CSRC / "nt_noalloc.hip"
    deps = srcs + [hip_src, CSRC / "lower.hpp", CSRC / "nt_exec.hpp", CSRC / "nt_testing.h", CSRC / "nt_skeleton.h",
                   CSRC / "nt_math_tables.h", inc, ROOT / "include" / "nablatensor_rocm.h"]
    if not force and _newer(out, deps):
        return out
    incs = [f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    hip_obj = CSRC / "nt_noalloc.o"
    _run([str(ROCM / "bin" / "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", *PACKED_FP32_OFF,
          *incs, "-c", str(hip_src), "-o", str(hip_obj)])
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-D__HIP_PLATFORM_AMD__", *incs, f"-I{ROCM / 'include'}",
           *map(str, srcs), str(hip_obj), "-o", str(out) + ".tmp",
           f"-L{ROCM / 'lib'}", "-lamdhip64", "-lhiprtc", "-lamd_comgr", f"-Wl,-rpath,{ROCM / 'lib'}", "-ldl"]
    _run(cmd)
    os.replace(str(out) + ".tmp", out)
    hip_obj.unlink()
    return out


def host_module_path() -> Path:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return PKG / f"_host{suffix}"


def build_host(force: bool = True) -> Path:
    import pybind11

    out = host_module_path()
    srcs = [HOST / "aad.cpp", HOST / "quant.cpp", HOST / "engine.cpp", HOST / "bindings.cpp"]
    deps = srcs + list(HOST.glob("*.hpp")) + [ROOT / "include" / "nablatensor_rocm.h"]
    if not force and _newer(out, deps):
        return out
    py_inc = sysconfig.get_paths()["include"]
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", "-Wall",
           f"-I{pybind11.get_include()}", f"-I{py_inc}", f"-I{ROOT / 'include'}", f"-I{HOST}",
           *map(str, srcs), "-o", str(out) + ".tmp", "-ldl"]
    _run(cmd)
    os.replace(str(out) + ".tmp", out)
    return out


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "libnt_oracle.so"


def check_offline_hipcc(source: str, name: str = "check") -> Path:
    """Compile a generated kernel source with hipcc for gfx950 (no device needed)."""
    work = PKG / "_kcache"
    work.mkdir(exist_ok=True)
    src = work / f"{name}.hip"
    src.write_text(source)
    out = work / f"{name}.hsaco"
    feats = []
    for line in source.splitlines():
        if line.startswith("// nt-compile:"):
            for f in line.split()[2:]:
                feats += ["-Xclang", "-target-feature", "-Xclang", f]
    cmd = [str(ROCM / "bin" / "hipcc"), "--offload-arch=gfx950", "--cuda-device-only", "-O3", "-std=c++17",
           *PACKED_FP32_OFF, *feats, f"-I{CSRC}", "-c", str(src), "-o", str(out)]
    _run(cmd)
    return out


def build_math_device(force: bool = True) -> Path:
    """Test driver of the skeleton's own fp64 math on the device
    (tests/device_math/nt_math_device.hip -> libnt_math_device.so, loaded by
    tests/test_gpu_math.py)."""
    src = ROOT / "tests" / "device_math" / "nt_math_device.hip"
    out = src.parent / "libnt_math_device.so"
    deps = [src, CSRC / "nt_skeleton.h", CSRC / "nt_math_tables.h"]
    if not force and _newer(out, deps):
        return out
    _run([str(ROCM / "bin" / "hipcc"), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
          *PACKED_FP32_OFF, f"-I{CSRC}", str(src), "-o", str(out) + ".tmp"])
    os.replace(str(out) + ".tmp", out)
    return out


def build_all(force: bool = True) -> None:
    build_engine(force)
    build_host(force)
    build_oracle()
    build_math_device(force)


if __name__ == "__main__":
    build_all(force="--if-stale" not in sys.argv)
    print("built", PKG / "libnt_rocm.so", host_module_path())
