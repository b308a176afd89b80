"""Builds a copy of libneuralzip_hip.so whose host C++ runs under
AddressSanitizer and UndefinedBehaviorSanitizer, for the CPU test suite.

The host sources (codebook, layout, codec, survey and the C ABI) are
compiled with g++ and the sanitizers; the gfx950 kernel objects are the
regular build's, unchanged; g++ links both with the HIP runtime. Nothing on
the GPU path loads this copy. Run the CPU tests against it with

    python -m neuralzip_amd.sanitize --run [pytest arguments]

which builds it, then starts pytest with libasan preloaded (Python itself is
not instrumented), leak detection off (the interpreter keeps its own
allocations to the end) and NZ_NATIVE_LIBRARY naming the copy.
"""
import os
import subprocess
import sys
from pathlib import Path

from neuralzip_amd import build as regular

SANITIZED = regular.OBJ / "sanitized" / "libneuralzip_hip_sanitized.so"
OBJ = regular.OBJ / "sanitized"
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"]
ROCM_LIB = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"


def build():
    """Host objects with the sanitizers, the regular kernel objects, one
    shared library; returns its path."""
    kernels = [regular.OBJ / (Path(name).stem + ".o") for name in regular.DEVICE_SOURCES]
    if not all(obj.exists() for obj in kernels):
        regular.build()
    OBJ.mkdir(parents=True, exist_ok=True)
    objects = []
    for name in regular.HOST_SOURCES:
        obj = OBJ / (Path(name).stem + ".o")
        command = ["g++", "-O1", "-g", "-std=c++17", "-fPIC", "-Wall", "-I", str(regular.CSRC),
                   "-I", str(regular.ROOT / "include"), *regular.HOST_FLAGS, *SANITIZE,
                   "-c", str(regular.CSRC / name), "-o", str(obj)]
        subprocess.run(command, check=True)
        objects.append(obj)
    objects += kernels
    link = ["g++", "-shared", *SANITIZE, "-o", str(SANITIZED), *map(str, objects),
            f"-L{ROCM_LIB}", f"-Wl,-rpath,{ROCM_LIB}", "-lamdhip64", "-lpthread"]
    subprocess.run(link, check=True)
    return SANITIZED


def environment(library=SANITIZED):
    """Environment of a Python process that loads the sanitized copy."""
    def runtime(name):
        return subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True,
                              check=True).stdout.strip()
    env = dict(os.environ)
    # libstdc++ right after libasan: its exception interceptor binds to the
    # real __cxa_throw only if libstdc++ is loaded when the runtime starts
    env.update(LD_PRELOAD=f"{runtime('libasan.so')}:{runtime('libstdc++.so')}", NZ_NATIVE_LIBRARY=str(library),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    return env


def run(pytest_args):
    """pytest in a child process against the sanitized copy; returns its
    exit status (also 1 when a sanitizer reported anything)."""
    library = build()
    result = subprocess.run([sys.executable, "-m", "pytest", *pytest_args], env=environment(library),
                            cwd=regular.ROOT, capture_output=True, text=True)
    output = result.stdout + result.stderr
    sys.stdout.write(output)
    reported = "ERROR: AddressSanitizer" in output or "runtime error:" in output
    return 1 if reported and result.returncode == 0 else result.returncode


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--run":
        sys.exit(run(sys.argv[2:] or ["tests", "-q", "-m", "not gpu"]))
    print(build())
