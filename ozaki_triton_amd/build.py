"""Build libozaki_amd.so (HIP kernels + C ABI) in-tree for gfx950.

Every source under csrc/ is compiled with hipcc; the shared library lands next
to this file so that it travels with the source tree.  Flags:

* ``-ffp-contract=off``: no multiply/add is fused where the reference rounds
  the product (the epilogue and the residual update must round like it).
* ``-fno-gpu-flush-denormals-to-zero``: fp32 denormals are kept (scales reach
  2^(-126-alpha), which is subnormal).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 ops.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libozaki_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("OZK_OFFLOAD_ARCH", "gfx950")

# the cross-GEMM kernels are instantiated in one unit per slice dtype (the
# int8 one is the largest), so that they compile in parallel
SOURCES = ["ozk_gemm_i8.hip", "ozk_gemm_f16.hip", "ozk_gemm_bf16.hip", "ozk_gemm_f32.hip",
           "ozk_split.hip", "ozk_api.cpp", "ozk_gemm.hip"]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libozaki_amd.so)")


def build(verbose: bool = False) -> str:
    """Compile all sources (in parallel) and link the shared library.  Always
    rebuilds; returns the library path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmd = [hipcc, *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd.insert(1, "-xhip")
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
        if p.returncode != 0:
            failed.append((src, "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        msg = "\n".join(f"--- {s} ---\n{o}" for s, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}")
    _check_no_undefined_own_symbols(tmp)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _check_no_undefined_own_symbols(lib: str) -> None:
    """A shared library links with undefined symbols, and the loader reports
    them only at run time.  The host pass can leave a kernel's launch stub
    undefined without a diagnostic (a local type it cannot lay out, for
    instance): every symbol of the library's own namespace must be defined."""
    nm = shutil.which("nm") or shutil.which("llvm-nm") or "/opt/rocm/llvm/bin/llvm-nm"
    if not os.path.exists(nm):
        return
    res = subprocess.run([nm, "-D", "--undefined-only", lib], stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True)
    own = [ln.split()[-1] for ln in res.stdout.splitlines() if "_ZN3ozk" in ln]
    if res.returncode != 0 or own:
        os.remove(lib)
        raise RuntimeError("libozaki_amd.so leaves symbols of its own undefined:\n" +
                           ("\n".join(own) if own else res.stdout))


def build_c_example(verbose: bool = False) -> str:
    """Compile tests/c_abi_example.cpp, a plain C++ caller of the C ABI, against
    the in-tree library (rpath to it, relative to the binary)."""
    root = os.path.dirname(HERE)
    src = os.path.join(root, "tests", "c_abi_example.cpp")
    out = os.path.join(root, "tests", "c_abi_example")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-Wall",
           "-I", os.path.join(root, "include"), src, "-o", out, "-L", HERE, "-lozaki_amd",
           "-Wl,-rpath,$ORIGIN/../ozaki_triton_amd"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"c_abi_example build failed:\n{res.stdout}")
    return out


def build_power_probe(verbose: bool = False) -> str:
    """Compile tests/mfma_power_probe.hip, the MFMA rate / clock probe that the
    cross-GEMM's roofline discussion is measured with (test tool, not part of
    the library)."""
    root = os.path.dirname(HERE)
    src = os.path.join(root, "tests", "mfma_power_probe.hip")
    out = os.path.join(root, "tests", "mfma_power_probe")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-Wall",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", src, "-o", out]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"mfma_power_probe build failed:\n{res.stdout}")
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
