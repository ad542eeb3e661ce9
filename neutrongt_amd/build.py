"""Builds libngt_attn.so (the HIP kernels + C ABI) for gfx950 with hipcc.

Run as ``python -m neutrongt_amd.build`` or through ``__graft_entry__.build()``.
Objects go to ``neutrongt_amd/_build/``; the shared library is written in-tree
next to this file so that it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
BUILD = PKG / "_build"
LIB_NAME = "libngt_attn.so"
ARCH = os.environ.get("NGT_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 VALU ops stay disabled in every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs (gfx950 has one register file), so
    # the softmax VALU work on score tiles needs no accvgpr copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
]


# Per-source additions.  The dense matrix-core kernels never produce a NaN
# (masked keys are -inf, every tile's running maximum is finite), so they run
# with the IEEE-mode bit off: fmaxf then needs no canonicalising v_max of each
# MFMA result (9 of the forward's 77 VALU instructions per 32 x 32 score tile).
FILE_FLAGS = {
    "ngt_dense_mfma.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, obj: Path, verbose: bool, extra: list[str]) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o",
           str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns about the device-only target feature; keep other output.
    noise = "-packed-fp32-ops"
    msg = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l).strip()
    if msg and verbose:
        print(msg, file=sys.stderr)


def build_library(verbose: bool = False, jobs: int | None = None, out: Path | None = None,
                  extra_flags: list[str] | None = None) -> Path:
    """Compiles every ``csrc/*.hip`` and links ``libngt_attn.so`` (or ``out``);
    returns its path.  ``extra_flags`` (or NGT_HIPCC_EXTRA) are added to every
    compile, e.g. -D tuning macros for an experimental build."""
    extra = list(extra_flags or os.environ.get("NGT_HIPCC_EXTRA", "").split())
    build_dir = BUILD if not extra else BUILD / ("x" + str(abs(hash(tuple(extra))) % 10**8))
    build_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [build_dir / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose, extra) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    out = Path(out) if out else PKG / LIB_NAME
    tmp = out.with_name(out.name + ".tmp")
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build_autograd_ext(verbose: bool = False) -> Path:
    """Compiles csrc/ngt_autograd.cpp (host C++: the sparse attention's
    autograd node, see that file) as a torch extension with g++ and puts
    ngt_autograd.so beside the library; returns its path."""
    import torch
    from torch.utils import cpp_extension

    build_dir = BUILD / "autograd"
    build_dir.mkdir(parents=True, exist_ok=True)
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    cpp_extension.load(
        name="ngt_autograd", sources=[str(CSRC / "ngt_autograd.cpp")],
        extra_include_paths=[str(INCLUDE), str(rocm / "include")],
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"],
        extra_ldflags=[f"-L{torch_lib}", "-lc10_hip", f"-L{rocm / 'lib'}", "-lamdhip64"],
        build_directory=str(build_dir), verbose=verbose, with_cuda=False, is_python_module=True)
    out = PKG / "ngt_autograd.so"
    tmp = out.with_name(out.name + ".tmp")
    shutil.copyfile(build_dir / "ngt_autograd.so", tmp)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
    print(build_autograd_ext(verbose="-v" in sys.argv))
