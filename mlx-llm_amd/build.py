"""Build libmlxq.so (gfx950 HIP kernels + C ABI + C++ host API) in-tree.

Usage: python mlx-llm_amd/build.py [--jobs N] [--verbose]

Every HIP source is compiled with hipcc for gfx950 only.  Packed FP32 VALU
ops are disabled (`-Xclang -target-feature -Xclang -packed-fp32-ops`).
Sources whose results must be bit-identical with the CPU restatement
(GGUF dequant, affine quantize) are compiled with -ffp-contract=off.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
OBJ = PKG / "_build"
LIB = PKG / "libmlxq.so"
BIN = PKG / "bin"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
sys.path.insert(0, str(PKG))
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
NO_CONTRACT = {"gguf.hip", "affine.hip", "gguf_requant.hip"}
# MFMA results in ordinary VGPRs (no accumulator-register copies before the
# per-group fold): the batched-decode kernels' results are read by the VALU
# after every group, so the copies were pure overhead there
MFMA_VGPR = {"qmv_tile.hip"}


def sources() -> list[Path]:
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if HOST.is_dir():
        srcs += sorted(HOST.glob("*.cpp"))
    return srcs


def compile_one(src: Path, verbose: bool, src_hash: str = "unknown") -> Path:
    obj = OBJ / (src.parent.name + "_" + src.name + ".o")
    cmd = [HIPCC, *COMMON]
    if src.name == "capi.cpp":  # mlxq_version() reports the sources the library was built from
        cmd.append(f'-DMLXQ_SOURCE_HASH="{src_hash}"')
    if src.name in NO_CONTRACT:
        cmd.append("-ffp-contract=off")
    if src.name in MFMA_VGPR:
        cmd += ["-mllvm", "-amdgpu-mfma-vgpr-form"]
    if src.suffix == ".cpp":
        cmd += ["-x", "hip"]  # host files include hip_runtime for stream types
    cmd += ["-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know packed-fp32-ops: harmless.
    errs = [ln for ln in r.stderr.splitlines() if "warning" in ln and "packed-fp32-ops" not in ln]
    if errs and verbose:
        print("\n".join(errs))
    return obj


def build(jobs: int = 8, verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    from provenance import source_hash

    h = source_hash()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: compile_one(s, verbose, h), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs),
           "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    # a kernel whose host-side stub the compiler dropped (it can, silently,
    # for some builtins in template kernels) would only fail at load time
    nm = subprocess.run(["nm", "-u", str(tmp)], capture_output=True, text=True)
    # (or the kernel symbol itself, when the host pass found the kernel body
    # invalid: any undefined symbol of the library's own namespace)
    missing = [ln.split()[-1] for ln in nm.stdout.splitlines() if "__device_stub__" in ln or "_ZN4mlxq" in ln]
    if missing:
        raise RuntimeError("kernel stubs missing from the library:\n" + "\n".join(missing[:10]))
    os.replace(tmp, LIB)
    build_host_tests(verbose)
    build_cli(verbose)
    return LIB


def build_host_tests(verbose: bool = False) -> Path:
    """The C++ restatement of the reference's tests (tests/cpp/host_tests.cpp)
    against the C++ host API, linked to libmlxq.so (found next to it at run
    time through the rpath)."""
    BIN.mkdir(exist_ok=True)
    out = BIN / "host_tests"
    cmd = [HIPCC, "-O2", "-std=c++17", f"--offload-arch={ARCH}", "-x", "hip", f"-I{ROOT / 'include'}", f"-I{HOST}",
           str(ROOT / "tests" / "cpp" / "host_tests.cpp"), "-x", "none", str(LIB), "-Wl,-rpath,$ORIGIN/..",
           "-o", str(out)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host tests build failed:\n{r.stdout}\n{r.stderr}")
    return out


def build_cli(verbose: bool = False) -> Path:
    """bin/convert_gguf: the GGUF -> MLX snapshot converter (cli/convert_gguf.cpp)."""
    BIN.mkdir(exist_ok=True)
    out = BIN / "convert_gguf"
    cmd = [HIPCC, "-O2", "-std=c++17", f"--offload-arch={ARCH}", "-x", "hip", f"-I{ROOT / 'include'}", f"-I{HOST}",
           str(PKG / "cli" / "convert_gguf.cpp"), "-x", "none", str(LIB), "-Wl,-rpath,$ORIGIN/..", "-o", str(out)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"convert_gguf build failed:\n{r.stdout}\n{r.stderr}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args(argv)
    lib = build(a.jobs, a.verbose)
    print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
