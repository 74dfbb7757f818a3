"""Builds localstack_amd/liblstk_moe.so (gfx950) with hipcc, in place.

The library is the product: the MoE kernels (csrc/kernels.hip, grouped.hip, fused.hip), the HBM
expert pool and the MoE C ABI (csrc/pool.cpp, include/lstk_moe.h), the host repacker
(csrc/repack.cpp), the forward pass around the MoE block (csrc/forward.hip, csrc/model.cpp,
include/lstk_qwen3.h) and the GGUF reader (csrc/gguf.cpp, include/lstk_gguf.h).
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "liblstk_moe.so")
SOURCES = ["kernels.hip", "grouped.hip", "fused.hip", "forward.hip", "pool.cpp", "repack.cpp", "model.cpp", "gguf.cpp", "tier.hip"]
ARCH = os.environ.get("LSTK_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


# Per-source extra flags. The grouped MFMA kernels keep their accumulators in VGPRs (the VALU
# epilogue then reads them without v_accvgpr_read moves).
EXTRA = {"grouped.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
COMMON = ["-O3", "-std=c++20", "-fPIC",
          # packed-FP32 instructions off for all device code
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          # every multiply and add rounded on its own, as written: the fused and multi-kernel paths
          # then agree bit for bit whatever the compiler would otherwise contract in each context
          "-ffp-contract=off",
          "-Wall", "-Wno-unused-function"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError("hipcc failed: " + " ".join(cmd))
    if out.strip() and verbose:
        print(out)


OBJ_DIR = os.path.join(HERE, "_build")  # objects of the last build (not shipped; the sanitizer build reuses the kernels')
ASAN_LIB = os.path.join(OBJ_DIR, "liblstk_moe_asan.so")
# host sources checked by the sanitizer build: the pool's bookkeeping, the GGUF reader, the repacker, the model's host side
HOST_SOURCES = ["pool.cpp", "repack.cpp", "model.cpp", "gguf.cpp"]
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer"]


def _compile(sources, objdir, extra, verbose):
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(objdir, exist_ok=True)
    cmds, objs = [], []
    for s in sources:
        o = os.path.join(objdir, s + ".o")
        objs.append(o)
        cmds.append([hipcc(), "-x", "hip", f"--offload-arch={ARCH}"] + COMMON + EXTRA.get(s, []) + extra.get(s, []) +
                    ["-I", os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, s), "-o", o])
    with ThreadPoolExecutor(max_workers=min(len(cmds), 8)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    return objs


def _link(objs, out, extra, verbose):
    tmp = out + ".tmp"
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + extra + objs +
         ["-L", rocm_lib, "-lrocblas", "-Wl,-rpath," + rocm_lib, "-lpthread"], verbose)
    os.replace(tmp, out)


def build(verbose=False):
    """Compiles every source for gfx950 (in parallel) and links the shared library; always rebuilds."""
    objs = _compile(SOURCES, OBJ_DIR, {}, verbose)
    _link(objs, LIB, [], verbose)
    return LIB


def build_sanitized(verbose=False):
    """A copy of the library whose host sources (HOST_SOURCES) are built with AddressSanitizer and
    UndefinedBehaviorSanitizer on the host side only (the device code is unchanged), for the CPU tests of
    the dry pool and the GGUF reader. The kernel sources' objects come from the last build() (compiled
    here if there are none). Load it with the sanitizer runtime preloaded (asan_runtime())."""
    kernels = [s for s in SOURCES if s not in HOST_SOURCES]
    have = all(os.path.exists(os.path.join(OBJ_DIR, s + ".o")) for s in kernels)
    kobjs = [os.path.join(OBJ_DIR, s + ".o") for s in kernels] if have else _compile(kernels, OBJ_DIR, {}, verbose)
    sdir = os.path.join(OBJ_DIR, "asan")
    hobjs = _compile(HOST_SOURCES, sdir, {s: ["-O1", "-g"] + SANITIZE for s in HOST_SOURCES}, verbose)
    _link(kobjs + hobjs, ASAN_LIB, ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                                    "-shared-libsan"], verbose)
    return ASAN_LIB


def asan_runtime():
    """The clang AddressSanitizer runtime that the sanitized library links against, or None."""
    root = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "lib", "clang")
    if not os.path.isdir(root):
        return None
    for v in sorted(os.listdir(root), reverse=True):
        p = os.path.join(root, v, "lib", "linux", "libclang_rt.asan-x86_64.so")
        if os.path.exists(p):
            return p
    return None


if __name__ == "__main__":
    print(build(verbose=True))
