"""Build libkvq.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m kvq_decode_amd.build          # or: python kvq_decode_amd/build.py

Compiles csrc/*.hip and csrc/*.cpp with hipcc (one process per source, in parallel) and
links kvq_decode_amd/libkvq.so. Always recompiles (the build check runs it on every call);
a failed compile raises.
"""
import os
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_PATH = os.path.join(PKG_DIR, "libkvq.so")
OBJ_DIR = os.path.join(PKG_DIR, "_build")  # objects (not committed, not shipped)

ARCH = "gfx950"
SOURCES = ["capi.cpp", "decode.hip", "decode_q.hip", "decode_q_d64.hip", "decode_q_d256.hip",
           "quant.hip", "append.hip", "static_workspace.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops (v_pk_{add,mul,fma}_f32) stay off: hipcc would otherwise form
    # them from ordinary float code. The host pass warns that it does not know the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax rescale works on them with VALU ops, which
    # would otherwise copy them out of and back into AGPRs every chunk.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # No -ffast-math: fp32 division stays correctly rounded (the quantizer's codes must be
    # bit-exact with its float32 spec; quant.hip also turns fp contraction off).
]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.environ.get("HIPCC", os.path.join(rocm, "bin", "hipcc"))


def _compile(src, obj, cmd_base):
    cmd = [*cmd_base, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    return proc, cmd


def _filter(proc):
    noise = ("packed-fp32-ops", "is not a recognized feature")
    return [ln for ln in (proc.stdout + proc.stderr).splitlines()
            if not any(n in ln for n in noise)]


def build(verbose=False):
    """Compiles every source to an object in parallel (one hipcc per source), then links
    libkvq.so. The kernels of different sources call nothing across files, so no
    relocatable device code is needed."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    base = [hipcc(), *flags, f"-I{INCLUDE}", f"-I{CSRC}"]
    t0 = time.time()
    jobs = [(os.path.join(CSRC, s), os.path.join(OBJ_DIR, s + ".o")) for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
        results = list(pool.map(lambda j: _compile(j[0], j[1], base), jobs))
    msgs = []
    for proc, cmd in results:
        msgs += _filter(proc)
        if proc.returncode != 0:
            raise RuntimeError("hipcc failed (%d):\n%s\ncommand: %s"
                               % (proc.returncode, "\n".join(_filter(proc)), " ".join(cmd)))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC",
           *[o for _, o in jobs], "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed (%d):\n%s\ncommand: %s"
                           % (proc.returncode, "\n".join(_filter(proc)), " ".join(cmd)))
    os.replace(tmp, LIB_PATH)
    if verbose:
        for m in msgs:
            print(m)
        print(f"built {LIB_PATH} in {time.time() - t0:.1f}s")
    build_checks(verbose)
    return LIB_PATH


# GPU check programs of the test suite (tests/gpu_checks/*.hip -> executables beside them)
CHECKS_DIR = os.path.join(REPO_DIR, "tests", "gpu_checks")


def build_checks(verbose=False):
    if not os.path.isdir(CHECKS_DIR):
        return
    for name in sorted(os.listdir(CHECKS_DIR)):
        if not name.endswith(".hip"):
            continue
        src = os.path.join(CHECKS_DIR, name)
        out = src[:-len(".hip")]
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", src, "-o", out]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError("hipcc failed (%d) on %s:\n%s"
                               % (proc.returncode, src, proc.stderr[-3000:]))
        if verbose:
            print(f"built {out}")


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
