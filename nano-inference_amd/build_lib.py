"""Build libnia_attn.so (the gfx950 attention kernels + C ABI) in-tree with hipcc.

Usage: python build_lib.py [-v]   (from any directory)

Every HIP source under csrc/ is compiled for gfx950 only and linked into one
shared library next to this file.  Objects go to _build/ (git-ignored).  The
CPython fast-call module (csrc/fastcall.c, which calls that library's hot entry
points through pointers handed to it at load time) is compiled with the host C
compiler into the same directory.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libnia_attn.so"
FAST_SRC = CSRC / "fastcall.c"
FAST_NAME = "_nia_fast" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the gfx950 attention library cannot be built")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know -packed-fp32-ops; drop that noise.
    err = "\n".join(
        ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err and verbose:
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libnia_attn.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(srcs), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    out = PKG_DIR / LIB_NAME
    tmp = PKG_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    build_fast(verbose)
    return out


def build_fast(verbose: bool = False) -> Path | None:
    """Compile the CPython fast-call module next to the library; returns its path.

    Without a host C compiler or Python's headers it is skipped with a warning: the
    ctypes binding then makes the same calls, at a few microseconds more per call.
    """
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    inc = sysconfig.get_paths().get("include")
    out = PKG_DIR / FAST_NAME
    if not cc or not inc or not (Path(inc) / "Python.h").exists():
        # An earlier build would be bound to the new library without matching it.
        out.unlink(missing_ok=True)
        print(f"warning: {FAST_NAME} not built (no C compiler or Python.h); "
              "the hot calls go through ctypes", file=sys.stderr)
        return None
    tmp = PKG_DIR / (FAST_NAME + ".tmp")
    cmd = [cc, "-O2", "-Wall", "-Wextra", "-shared", "-fPIC", f"-I{inc}",
           str(FAST_SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{FAST_SRC.name} failed to compile:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
