"""Build libprism_mi355x.so (gfx950 HIP kernels + C ABI) in-tree.

    python prism-infer_amd/build_native.py

Compiles every ``csrc/*.hip`` with ``hipcc --offload-arch=gfx950`` and links
the shared library against the HIP runtime that ships with the installed
PyTorch (``torch/lib/libamdhip64.so``), so that a process which has imported
torch holds exactly one HIP runtime and torch's streams are valid handles for
the library.  Packed-fp32 instruction selection is disabled for all device
code.  The output lands in ``prism_infer/_native/libprism_mi355x.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_ROOT / "_build"
OUT_DIR = PKG_ROOT / "prism_infer" / "_native"
LIB_NAME = "libprism_mi355x.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")
    return found


def _torch_lib_dir() -> Path:
    import torch  # noqa: PLC0415

    lib = Path(torch.__file__).resolve().parent / "lib"
    if not (lib / "libamdhip64.so").exists():
        raise RuntimeError(f"torch's HIP runtime not found under {lib}")
    return lib


# Per-source extra flags.  The prefill kernel's max reductions run without the
# IEEE mode's NaN quieting (no operand there is a NaN), which halves their cost.
EXTRA_FLAGS = {
    "paged_prefill.hip": ["-mno-amdgpu-ieee", "-fno-honor-nans"],
}


def _compile(src: Path, build_dir: Path = BUILD_DIR, defines: tuple = ()) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), *(f"-D{d}" for d in defines), f"-I{INCLUDE}",
           f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True, *, out_dir: Path = OUT_DIR, measure: bool = False, defines: tuple = ()) -> Path:
    """Compile all sources and link the shared library; returns its path.

    ``measure=True`` builds the measurement variant (PRISM_DECODE_MEASURE:
    the streaming decode kernel's skip/timestamp switches) into ``out_dir``;
    the product library never has them.
    """

    tag = "measure" if measure else "product"
    if defines:
        tag += "-" + "-".join(d.replace("=", "") for d in defines)
    build_dir = BUILD_DIR / tag
    build_dir.mkdir(parents=True, exist_ok=True)
    out_dir.mkdir(parents=True, exist_ok=True)
    defines = (("PRISM_DECODE_MEASURE",) if measure else ()) + tuple(defines)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(src, build_dir, defines), sources))
    torch_lib = _torch_lib_dir()
    out = out_dir / LIB_NAME
    tmp = out_dir / (LIB_NAME + ".tmp")
    # Link with the host compiler against torch's libamdhip64 (see module doc).
    cmd = [
        "g++", "-shared", "-o", str(tmp), *map(str, objects),
        f"-L{torch_lib}", "-l:libamdhip64.so", f"-Wl,-rpath,{torch_lib}", "-Wl,--no-undefined",
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    try:
        if "--measure" in sys.argv[1:]:
            i = sys.argv.index("--measure")
            build(out_dir=Path(sys.argv[i + 1]).resolve(), measure=True)
        else:
            build()
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
