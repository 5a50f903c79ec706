"""Build the gfx950 C-ABI library ``slipstream_amd/_lib/libslipstream_hip.so``.

One ``hipcc`` compile per ``csrc/*.hip`` source (in parallel), then one link.
Run as ``python -m slipstream_amd.build`` or through ``__graft_entry__.build()``.
The library is built in-tree so it travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libslipstream_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in the device code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build slipstream_amd")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


HOST_EXT = "_host_pairs"


def host_ext_path() -> Path:
    """The CPython extension of host helpers (``csrc/host_pairs.c``), built beside the library."""
    return OUT_DIR / (HOST_EXT + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))


def _build_host_ext() -> Path:
    """``csrc/host_pairs.c`` -> the extension module (gcc, CPython headers; host code only)."""
    src = CSRC / "host_pairs.c"
    target = host_ext_path()
    tmp = target.with_name(target.name + ".tmp")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("gcc not found: needed for the host helper extension")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}", str(src), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, target)
    return target


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library, then the host helper
    extension; returns the library's path."""
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(_compile, srcs, objs))
    target = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, target)
    ext = _build_host_ext()
    if verbose:
        print(f"built {target}")
        print(f"built {ext}")
    return target


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
