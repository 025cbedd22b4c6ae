"""Build libkdn.so (all HIP kernels + the C ABI) in-tree with hipcc for gfx950.

Every HIP translation unit is compiled with packed fp32 arithmetic disabled (the compiler would
otherwise form v_pk_* fp32 ops from ordinary float code).  Translation units are compiled to objects
in parallel, then linked into the shared library.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
CSRC = os.path.join(PKG_ROOT, "csrc")
SOURCES = ["kdn_api.hip", "kdn_lift.hip", "kdn_prep.hip", "kdn_scan.hip", "kdn_chain.hip", "kdn_serve.hip", "kdn_pool.hip",
           "kdn_bwd.hip", "kdn_general.hip", "kdn_noalloc.hip", "kdn_frep.hip"]
OUT = os.path.join(_HERE, "libkdn.so")
OBJDIR = os.path.join(_HERE, "_build")
ARCH = "gfx950"
HIP_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-source extra flags.  -amdgpu-mfma-vgpr-form puts MFMA results in VGPRs rather than AGPRs, so that
# VALU work on them needs no v_accvgpr_read copies: faster for the prep and backward kernels, which
# post-process nearly every MFMA result (measured); slower for the state kernel, so not global.
SOURCE_FLAGS = {"kdn_prep.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "kdn_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}")


def build_native(verbose: bool = False) -> str:
    """Compile every source into kdn/libkdn.so; returns the library path.  Always recompiles."""
    os.makedirs(OBJDIR, exist_ok=True)
    objs = [os.path.join(OBJDIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[hipcc()] + HIP_FLAGS + SOURCE_FLAGS.get(s, []) + ["-c", "-o", o, os.path.join(CSRC, s)]
            for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = OUT + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, OUT)
    return OUT


# AddressSanitizer + UndefinedBehaviorSanitizer on the host code only (the C ABI, argument checks,
# workspace layouts, the slab pool, the schedules); the device code is built as usual.  Every sanitizer
# flag is behind -Xarch_host: this pool runs no GPU code built with a sanitizer.
SANITIZE_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime() -> str:
    """The shared ASan runtime of hipcc's clang, which a process must preload to load the sanitized
    library (empty if it is not installed)."""
    import glob
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else ""


def build_host_sanitized(out_dir: str, verbose: bool = False) -> str:
    """Compile every source with the host code under ASan + UBSan into out_dir/libkdn_hostsan.so (for the
    host-path tests; not shipped).  Returns the library path."""
    os.makedirs(out_dir, exist_ok=True)
    objs = [os.path.join(out_dir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    flags = [f"--offload-arch={ARCH}", "-O1", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops"] + SANITIZE_FLAGS
    cmds = [[hipcc()] + flags + ["-c", "-o", o, os.path.join(CSRC, s)] for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = os.path.join(out_dir, "libkdn_hostsan.so")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
          "-Xarch_host", "-fsanitize=undefined", "-Xarch_host", "-shared-libasan", "-o", out] + objs, verbose)
    return out


if __name__ == "__main__":
    print(build_native(verbose=True))
