"""Build recipe for the gfx950 library ``libpkv_decode.so`` and the CPU oracle.

The HIP sources are compiled with hipcc for gfx950 only, one object per source
(in parallel), then linked into ``flashatte-hand_amd/lib/libpkv_decode.so``;
the C++ host harness ``flashatte-hand_amd/lib/pkv_harness`` and the torch extension
``flashatte-hand_amd/lib/pkv_torch.so`` link against it.
Packed-fp32 VALU instructions are disabled for all device code
(``-packed-fp32-ops``).  The oracle (test infrastructure) is built with its own
Makefile into ``oracle/libpkv_oracle.so``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent          # flashatte-hand_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
BUILD_DIR = PKG_ROOT / "_build"
LIB_DIR = PKG_ROOT / "lib"
LIB_PATH = LIB_DIR / "libpkv_decode.so"
HARNESS_SRC = PKG_ROOT / "harness" / "pkv_harness.hip"
TORCH_BINDING = "pkv_torch"
TORCH_BINDING_SRC = PKG_ROOT / "binding" / "pkv_torch.cpp"
ORACLE_DIR = REPO_ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "libpkv_oracle.so"

SOURCES = ["pkv_part_d128.hip", "pkv_part_d256.hip", "pkv_part_d64.hip", "pkv_partition.hip",
           "pkv_combine.hip", "pkv_append.hip", "pkv_api.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax rescale touches them with VALU ops,
    # and AGPR accumulators cost a copy each way around every such update.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libpkv_decode.so)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is harmless.
    out = "\n".join(line for line in res.stdout.splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_library(verbose: bool = False, jobs: int = 0) -> Path:
    """Compile every HIP source for gfx950 and link libpkv_decode.so (always rebuilds)."""
    hipcc = _hipcc()
    lib_path = LIB_PATH
    build_dir = BUILD_DIR
    build_dir.mkdir(parents=True, exist_ok=True)
    lib_path.parent.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = build_dir / (src.rsplit(".", 1)[0] + ".o")
        cmds.append([hipcc, *HIPCC_FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    if jobs <= 0:
        jobs = min(len(cmds), max(1, min(16, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = lib_path.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, lib_path)
    return lib_path


def build_harness(verbose: bool = False, lib_path: Path | None = None) -> Path:
    """Compile the C++ host harness (harness/pkv_harness.hip) next to the library it links."""
    lib_path = Path(lib_path) if lib_path else LIB_PATH
    if not lib_path.exists():
        raise RuntimeError(f"{lib_path} is not built; build_library() first")
    exe = lib_path.parent / "pkv_harness"
    tmp = exe.with_name(exe.name + ".tmp")
    _run([_hipcc(), *HIPCC_FLAGS, "-x", "hip", str(HARNESS_SRC), "-o", str(tmp),
          f"-L{lib_path.parent}", "-l" + lib_path.stem[3:], "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, exe)
    return exe


def build_torch_binding(verbose: bool = False) -> Path:
    """Compile the torch extension binding/pkv_torch.cpp (the reference's run_kernel binding and a
    stream-aware decode) against libpkv_decode.so, and place it next to the library as
    lib/pkv_torch*.so, importable with pagedkv.torch_binding()."""
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; build_library() first")
    from torch.utils import cpp_extension

    os.environ.setdefault("PYTORCH_ROCM_ARCH", "gfx950")
    build_dir = BUILD_DIR / "torch_binding"
    if build_dir.exists():
        shutil.rmtree(build_dir)  # always compile (the build check), not ninja's incremental rebuild
    build_dir.mkdir(parents=True)
    # Loaded from the build folder right after building, and from lib/ afterwards.
    cpp_extension.load(name=TORCH_BINDING, sources=[str(TORCH_BINDING_SRC)],
                       extra_include_paths=[str(REPO_ROOT / "include")], extra_cflags=["-O2"],
                       # $ORIGIN escaped for ninja ($$) and for the shell it runs (\\$)
                       extra_ldflags=[f"-L{LIB_DIR}", "-lpkv_decode", "-Wl,-rpath,\\$$ORIGIN:\\$$ORIGIN/../../lib"],
                       build_directory=str(build_dir), with_cuda=True, verbose=verbose)
    built = build_dir / f"{TORCH_BINDING}.so"
    dest = LIB_DIR / built.name
    tmp = dest.with_name(dest.name + ".tmp")
    shutil.copyfile(built, tmp)
    os.replace(tmp, dest)
    return dest


def build_oracle(verbose: bool = False) -> Path:
    """Build the CPU oracle (test infrastructure) with its Makefile."""
    cmd = ["make", "-s", "-B", "-C", str(ORACLE_DIR)]
    _run(cmd, verbose)
    return ORACLE_LIB


if __name__ == "__main__":
    import sys

    v = "-v" in sys.argv
    print(build_library(verbose=v))
    print(build_harness(verbose=v))
    print(build_torch_binding(verbose=v))
    print(build_oracle(verbose=v))
