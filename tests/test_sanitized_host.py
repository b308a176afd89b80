"""The host C++ of libneuralzip_hip.so under AddressSanitizer and
UndefinedBehaviorSanitizer: the tests that drive the library's CPU code
(storage codecs and their corrupt inputs, codebooks, the layout encoder and
its emulator, the setup's survey, the fused product's planning, the C ABI)
run in a child process against the sanitized copy that
neuralzip_amd.sanitize builds (host objects instrumented, kernel objects
as built). Any sanitizer report fails the test. No GPU is touched.
"""
import subprocess
import sys

import pytest

HOST_TESTS = ["tests/test_corrupt_inputs.py", "tests/test_codec.py", "tests/test_reference_formats.py",
              "tests/test_abi.py", "tests/test_layout_emulator.py", "tests/test_setup_storage.py",
              "tests/test_export_cpu.py", "tests/test_matvec.py", "tests/test_staging_scheme.py"]


@pytest.fixture(scope="module")
def sanitized():
    from neuralzip_amd import sanitize
    return sanitize, sanitize.build()


def test_the_sanitized_copy_is_the_library_loaded(sanitized):
    sanitize, library = sanitized
    probe = ("from neuralzip_amd import _native; _native.lib(); "
             "print(any(line.rstrip().endswith(str(_native.LIBRARY)) for line in open('/proc/self/maps')))")
    result = subprocess.run([sys.executable, "-c", probe], env=sanitize.environment(library), capture_output=True,
                            text=True, cwd=sanitize.regular.ROOT, timeout=300)
    assert result.returncode == 0, result.stderr[-2000:]
    assert result.stdout.strip() == "True"


def test_host_code_is_clean_under_asan_and_ubsan(sanitized):
    sanitize, library = sanitized
    args = [sys.executable, "-m", "pytest", *HOST_TESTS, "-q", "-m", "not gpu", "-p", "no:cacheprovider"]
    result = subprocess.run(args, env=sanitize.environment(library), capture_output=True, text=True,
                            cwd=sanitize.regular.ROOT, timeout=1200)
    output = result.stdout + result.stderr
    assert "AddressSanitizer" not in output and "runtime error:" not in output, output[-4000:]
    assert result.returncode == 0, output[-4000:]
    assert " passed" in output
