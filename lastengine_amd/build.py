"""Build recipe for the native parts (run on the CPU build host; hipcc cross-compiles gfx950).

Outputs (git-ignored, shipped with the tree):
  lastengine_amd/lib/le_qmm_<part>.hsaco   gfx950 code objects, one per kernel part
  lastengine_amd/lib/lible_qmm.so          host C-ABI library (include/le_qmm.h, include/le_quant.h)
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", ROCM + "/bin/hipcc")

# Packed FP32 instructions are disabled for all device code (they are not trusted on this pool).
DEVICE_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                "-packed-fp32-ops", "-I" + CSRC]
PARTS = {"deq": ["-DLE_PART_DEQ"], "moe": ["-DLE_PART_MOE"]}
for _ty in (2, 8, 11, 12, 13, 14, 16, 18, 22):
    PARTS["mv%d" % _ty] = ["-DLE_PART_MV=%d" % _ty]
PARTS["gm"] = []
PARTS["gq"] = ["-DLE_GQ_SET=1"]
PARTS["gq2"] = ["-DLE_GQ_SET=2"]
SOURCES = {"gm": "le_gemm_kernels.hip", "gq": "le_gq_kernels.hip", "gq2": "le_gq_kernels.hip"}  # parts not listed here compile le_qmm_kernels.hip

HOST_SOURCES = ["le_qmm.cpp", "le_quant.cpp", "le_gguf.cpp"]
# Host sources that declare device memory (hipcc, host and device passes), linked into the library.
HIP_HOST_SOURCES = ["le_noalloc.hip"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), out))
    return out


def code_object_cmd(part):
    return [HIPCC, "--genco"] + DEVICE_FLAGS + PARTS[part] + [
        os.path.join(CSRC, SOURCES.get(part, "le_qmm_kernels.hip")), "-o", os.path.join(LIB, "le_qmm_%s.hsaco" % part)]


def hip_host_obj(src):
    return os.path.join(LIB, os.path.splitext(src)[0] + ".o")


def hip_host_cmd(src):
    return [HIPCC, "-c", "-fPIC", "-I" + os.path.join(REPO, "include")] + DEVICE_FLAGS + [
        os.path.join(CSRC, src), "-o", hip_host_obj(src)]


def host_lib_cmd():
    # Host C++: the HIP runtime API is used through its C headers; the hipcc-built objects carry
    # the device arrays the host code addresses.
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__",
            "-I" + ROCM + "/include", "-I" + CSRC, "-I" + os.path.join(REPO, "include")] + [
        os.path.join(CSRC, s) for s in HOST_SOURCES] + [hip_host_obj(s) for s in HIP_HOST_SOURCES] + [
        "-o", os.path.join(LIB, "lible_qmm.so"), "-L" + ROCM + "/lib", "-Wl,-rpath," + ROCM + "/lib",
        "-lamdhip64", "-lpthread", "-ldl"]


def oracle_cmd():
    return ["make", "-s", "-C", os.path.join(REPO, "oracle")]


def build(jobs=8, with_oracle=True, parts=None):
    os.makedirs(LIB, exist_ok=True)
    cmds = [code_object_cmd(p) for p in (parts or PARTS)] + [hip_host_cmd(s) for s in HIP_HOST_SOURCES]
    if with_oracle:
        cmds.append(oracle_cmd())
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, cmds):
            if out:
                print(out)
    out = _run(host_lib_cmd())  # links the hipcc objects built above
    if out:
        print(out)


if __name__ == "__main__":
    build(parts=sys.argv[1:] or None)
