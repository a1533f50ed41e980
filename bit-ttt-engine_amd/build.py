"""Build libbitlinear_hip.so (gfx950) in-tree.

    python bit-ttt-engine_amd/build.py

Kernels (btl_kernels.hip) are compiled by hipcc for gfx950 only; the C-ABI layer
(btl_api.cpp) is host C++.  The shared library lands next to this file so that
it travels with the source tree to the GPU box.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbitlinear_hip.so")
PROBE = os.path.join(HERE, "probe")
PROBE_LIB = os.path.join(PROBE, "libbtl_probe.so")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# -ffp-contract=off: fp32 results are defined operation by operation (the
# quantiser and the reference-order path must match the CPU restatement bit
# for bit).  -packed-fp32-ops: no v_pk_*_f32 in the device code.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
             "-I" + os.path.join(ROCM, "include")]

KERNEL_SOURCES = ["btl_kernels.hip", "btl_model.hip", "btl_noalloc.hip", "btl_stream.hip"]
HOST_SOURCES = ["btl_api.cpp", "btl_model_api.cpp", "btl_stream_api.cpp"]


# Every kernel must run without scratch memory (register spills or private
# arrays indexed at run time go to scratch, slow and easy to miss): the kernel
# sources are compiled with the compiler's per-kernel resource remarks and the
# build fails on any kernel whose scratch size is not zero.
RESOURCE_REMARKS = ["-Rpass-analysis=kernel-resource-usage"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [l for l in res.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in l]
    remarks = [l for l in lines if "[-Rpass-analysis=kernel-resource-usage]" in l]
    out = "\n".join(l for l in lines if "[-Rpass-analysis=kernel-resource-usage]" not in l)
    if res.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s" % (res.returncode, " ".join(cmd), out))
    if verbose and out.strip():
        print(out)
    return remarks


def scratch_kernels(remarks):
    """(kernel, scratch bytes per lane, spilled VGPRs) of every kernel with scratch,
    from the compiler's kernel-resource-usage remarks."""
    bad, name, spill = [], None, 0
    for line in remarks:
        body = line.split("remark:", 1)[-1].strip()
        if body.startswith("Function Name:"):
            name = body.split(":", 1)[1].split("[")[0].strip()
        elif body.startswith("VGPRs Spill:"):
            spill = int(body.split(":", 1)[1].split("[")[0])
        elif body.startswith("ScratchSize [bytes/lane]:"):
            size = int(body.split(":", 1)[1].split("[")[0])
            if size:
                bad.append((name, size, spill))
    return bad


def build(verbose=False):
    """Compile every source and link libbitlinear_hip.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    inc = ["-I" + INCLUDE, "-I" + CSRC]
    bad = []
    for src in KERNEL_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        remarks = _run([HIPCC] + HIP_FLAGS + RESOURCE_REMARKS + inc + ["-c", os.path.join(CSRC, src), "-o", obj],
                       verbose)
        bad += [(src,) + b for b in scratch_kernels(remarks)]
        objs.append(obj)
    if bad:
        raise RuntimeError("kernels with scratch memory (spills or private arrays):\n" + "\n".join(
            "  %s: %s: %d bytes/lane, %d VGPRs spilled" % b for b in bad))
    cxx = shutil.which("g++") or "g++"
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        _run([cxx] + CXX_FLAGS + inc + ["-c", os.path.join(CSRC, src), "-o", obj], verbose)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp] + objs +
         ["-Wl,-soname,libbitlinear_hip.so"], verbose)
    os.replace(tmp, LIB)
    # the measurement kernels of bench.py --probe, a library of their own
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC] + HIP_FLAGS + ["-shared", os.path.join(PROBE, "btl_probe.hip"), "-o", tmp,
                                "-Wl,-soname,libbtl_probe.so"], verbose)
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
