"""Build libattnres_hip.so in-tree: gfx950 code objects + the C-ABI host library.

Steps (all outputs under ``kotodama_amd/lib/``):

1. ``hipcc --genco --offload-arch=gfx950`` compiles ``csrc/attnres_kernels.hip``
   once per code-object part (``-DATTNRES_PART=0..10``, in parallel).
2. ``gcc`` assembles ``csrc/attnres_blob.S``, which ``.incbin``s the parts.
3. ``hipcc -c -fPIC`` compiles ``csrc/attnres_noalloc.hip`` (the no-alloc
   entry point; its device array needs HIP device code of its own).
4. ``g++`` links ``csrc/attnres_capi.cpp``, the blob and that object into the
   shared library, linked against ROCm's ``libamdhip64.so.7``.  Loaded after ``import torch``,
   the dynamic linker binds that soname to the HIP runtime torch already
   loaded, so streams and device memory are shared with torch.

Run ``python -m kotodama_amd.build`` or call :func:`build`.
"""

from __future__ import annotations

import os
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
INCLUDE = PKG.parent / "include"
LIB_NAME = "libattnres_hip.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"
NUM_PARTS = 11

# Packed-fp32 VALU ops are disabled for every HIP compile (the kernels are
# written with scalar fp32 arithmetic).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "--genco",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False, out_dir: Path | None = None, defines: tuple = ()) -> Path:
    """Compile everything; returns the path of the built shared library.

    ``out_dir`` (default ``kotodama_amd/lib``) and extra ``-D`` ``defines``
    (e.g. ``("ATTNRES_NT_LOADS=0",)``) allow side-by-side variant builds.
    """
    hipcc = str(ROCM / "bin" / "hipcc")
    libdir = Path(out_dir) if out_dir is not None else LIBDIR
    libdir.mkdir(parents=True, exist_ok=True)
    extra = [f"-D{d}" for d in defines]
    with tempfile.TemporaryDirectory(prefix="attnres_build_", dir=libdir) as tmp:
        tmpd = Path(tmp)
        procs = []
        for part in range(NUM_PARTS):
            out = tmpd / f"attnres_gfx950_part{part}.hsaco"
            cmd = [hipcc, *HIP_FLAGS, *extra, f"-DATTNRES_PART={part}", f"-I{CSRC}", str(CSRC / "attnres_kernels.hip"),
                   "-o", str(out)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
        for cmd, p in procs:
            so, se = p.communicate()
            if p.returncode != 0:
                raise RuntimeError(f"hipcc failed ({p.returncode}): {' '.join(cmd)}\n{so}\n{se}")
        blob_o = tmpd / "attnres_blob.o"
        _run(["gcc", "-c", f"-I{tmpd}", str(CSRC / "attnres_blob.S"), "-o", str(blob_o)])
        noalloc_o = tmpd / "attnres_noalloc.o"
        noalloc_cmd = [hipcc, *[f for f in HIP_FLAGS if f != "--genco"], *extra, "-c", "-fPIC", f"-I{INCLUDE}",
                       str(CSRC / "attnres_noalloc.hip"), "-o", str(noalloc_o)]
        if verbose:
            print(" ".join(noalloc_cmd), flush=True)
        _run(noalloc_cmd)
        so_tmp = tmpd / LIB_NAME
        _run(
            [
                "g++",
                "-shared",
                "-fPIC",
                "-O2",
                "-std=c++17",
                "-Wall",
                "-D__HIP_PLATFORM_AMD__",
                *extra,
                f"-I{INCLUDE}",
                f"-I{CSRC}",
                f"-I{ROCM / 'include'}",
                str(CSRC / "attnres_capi.cpp"),
                str(blob_o),
                str(noalloc_o),
                f"-L{ROCM / 'lib'}",
                "-lamdhip64",
                f"-Wl,-rpath,{ROCM / 'lib'}",
                "-o",
                str(so_tmp),
            ]
        )
        final = libdir / LIB_NAME
        os.replace(so_tmp, final)  # atomic: a reader never sees a half-written library
    if verbose:
        print(f"built {final}", flush=True)
    return final


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
