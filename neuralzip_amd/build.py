"""Builds libneuralzip_hip.so in-tree: host C++ with g++, the gfx950 kernel
with hipcc, linked by hipcc. Run `python -m neuralzip_amd.build`."""
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OBJ = HERE / "_build"
LIBRARY = HERE / "libneuralzip_hip.so"
ARCH = os.environ.get("NZ_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HOST_SOURCES = ("codebook.cpp", "layout.cpp", "codec.cpp", "capi.cpp", "capi_storage.cpp", "survey.cpp")
DEVICE_SOURCES = ("hip/decode_gfx950.hip", "hip/matvec_gfx950.hip")
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-I", str(CSRC), "-I", str(ROOT / "include")]
# host float arithmetic (the setup's clustering) is evaluated as written: no fused multiply-add
HOST_FLAGS = ["-ffp-contract=off"]
# packed FP32 instructions stay disabled on every HIP translation unit
DEVICE_FLAGS = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build(verbose=False):
    OBJ.mkdir(exist_ok=True)
    jobs, objects = [], []
    for name in HOST_SOURCES:
        obj = OBJ / (Path(name).stem + ".o")
        jobs.append(["g++", *COMMON, *HOST_FLAGS, "-c", str(CSRC / name), "-o", str(obj)])
        objects.append(obj)
    for name in DEVICE_SOURCES:
        obj = OBJ / (Path(name).stem + ".o")
        jobs.append([HIPCC, *COMMON, *DEVICE_FLAGS, "-c", str(CSRC / name), "-o", str(obj)])
        objects.append(obj)
    procs = [subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT) for cmd in jobs]
    failed = []
    for cmd, proc in zip(jobs, procs):
        out = proc.communicate()[0].decode(errors="replace")
        if proc.returncode:
            failed.append(" ".join(cmd) + "\n" + out)
        elif verbose and out.strip():
            print(out)
    if failed:
        raise RuntimeError("neuralzip_amd build failed:\n" + "\n".join(failed))
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [HIPCC, "-shared", "-fPIC", *DEVICE_FLAGS[:1], "-o", str(tmp), *map(str, objects), "-lpthread"]
    result = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if result.returncode:
        raise RuntimeError("neuralzip_amd link failed:\n" + result.stdout.decode(errors="replace"))
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
