"""Compile csrc/*.hip into libnkilab_hip.so (gfx950), in-tree next to this file.

    python -m nkilab.build          # from nki-kernel-lab_amd/
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
INCLUDE_DIR = os.path.join(os.path.dirname(os.path.dirname(PKG_DIR)), "include")
LIB_NAME = "libnkilab_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

# -packed-fp32-ops: the compiler must not form v_pk_{add,mul,fma}_f32 itself.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def sources() -> list[str]:
    return sorted(os.path.join(SRC_DIR, f) for f in os.listdir(SRC_DIR) if f.endswith(".hip"))


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP kernels cannot be built")


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every csrc/*.hip for gfx950 and link libnkilab_hip.so; return its path."""
    cc = hipcc()
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 16)
    with tempfile.TemporaryDirectory(prefix="nkilab_build_") as tmp:
        objs, procs = [], []
        for s in srcs:
            obj = os.path.join(tmp, os.path.basename(s) + ".o")
            cmd = [cc, *HIP_FLAGS, "-I", INCLUDE_DIR, "-c", s, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
            if len(procs) >= jobs:
                _wait(procs.pop(0), verbose)
        for p in procs:
            _wait(p, verbose)
        tmp_lib = LIB_PATH + ".tmp"
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib]
        if verbose:
            print(" ".join(cmd), flush=True)
        out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if out.returncode != 0:
            raise RuntimeError(f"link failed:\n{out.stdout}")
        missing = undefined_own_symbols(tmp_lib)
        if missing:
            os.remove(tmp_lib)
            raise RuntimeError("the library leaves its own symbols undefined (a kernel whose launch stub the host "
                               "pass did not emit?):\n" + "\n".join(missing))
        os.replace(tmp_lib, LIB_PATH)
    return LIB_PATH


def undefined_own_symbols(lib: str) -> list[str]:
    """Symbols of the library's own namespace (nkl::) that `lib` references
    but does not define: a shared library links with them, and fails only
    when loaded.  Empty when nm is not available."""
    nm = shutil.which("nm")
    if not nm:
        return []
    out = subprocess.run([nm, "-D", "--undefined-only", lib], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                         text=True)
    return [ln.split()[-1] for ln in out.stdout.splitlines() if ln.split() and ln.split()[-1].startswith("_ZN3nkl")]


def _wait(item, verbose):
    src, proc = item
    out, _ = proc.communicate()
    # The host pass does not know the packed-fp32 feature flag; that warning is noise.
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines))


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
