"""The C ABI without a GPU: the library loads, exports every function the
public header declares, reports the header's ABI version, and lays out the
device descriptors as the header and the bindings say."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from neuralzip_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "neuralzip_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(nz_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_documented_entry_points():
    names = declared_functions()
    for expected in ("nz_last_error", "nz_abi_version", "nz_codebook_create", "nz_layout_encode", "nz_layout_pack",
                     "nz_plan_work", "nz_plan_work_interleaved", "nz_decode_slots", "nz_decode_launch", "nz_matvec_plan", "nz_matvec_tiles", "nz_matvec_launch",
                     "nz_matvec_reduce", "nz_storage_compress",
                     "nz_storage_decompress"):
        assert expected in names


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(_native.LIBRARY))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing


def test_abi_version_matches_header_and_bindings():
    version = int(re.search(r"#define NZ_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert ctypes.CDLL(str(_native.LIBRARY)).nz_abi_version() == version == _native.ABI_VERSION
    _native.lib()   # loads with the version check


def test_descriptor_layouts_match_the_format_header(tmp_path):
    probe = tmp_path / "sizes.cpp"
    probe.write_text(
        '#include <cstddef>\n#include <cstdio>\n#include "nz_format.h"\n'
        "int main(void) {\n"
        '  printf("%zu %zu %zu %zu %zu %zu %zu\\n", sizeof(struct nz_frag_desc), sizeof(struct nz_tile),\n'
        "         sizeof(struct nz_work), offsetof(struct nz_frag_desc, bit_length), offsetof(struct nz_frag_desc, numel),\n"
        "         offsetof(struct nz_tile, counts), offsetof(struct nz_work, kind));\n"
        "  return 0;\n}\n")
    exe = tmp_path / "sizes"
    try:
        built = subprocess.run(["g++", "-std=c++17", "-I", str(ROOT / "neuralzip_amd" / "csrc"), str(probe), "-o",
                                str(exe)], capture_output=True, text=True)
    except FileNotFoundError:
        pytest.skip("no C++ compiler for the layout probe")
    assert built.returncode == 0, built.stderr
    sizes = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert sizes == [_native.FRAG_DESC.itemsize, _native.TILE.itemsize, _native.WORK.itemsize,
                     _native.FRAG_DESC.fields["bit_length"][1], _native.FRAG_DESC.fields["numel"][1],
                     _native.TILE.fields["shape"][1], _native.WORK.fields["kind"][1]]


def test_matvec_weight_layout_matches_the_bindings(tmp_path):
    """nz_matvec_weight (public header, plain C) against _native.MatvecWeight."""
    probe = tmp_path / "weight.c"
    probe.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "neuralzip_hip.h"\n'
        "int main(void) {\n"
        '  printf("%zu %zu %zu %zu %zu %d %d\\n", sizeof(nz_matvec_weight), offsetof(nz_matvec_weight, rows),\n'
        "         offsetof(nz_matvec_weight, y), offsetof(nz_matvec_weight, bias), offsetof(nz_matvec_weight, offset),\n"
        "         NZ_MATVEC_MAX_BATCH, NZ_MATVEC_MAX_WEIGHTS);\n"
        "  return 0;\n}\n")
    exe = tmp_path / "weight"
    try:
        built = subprocess.run(["gcc", "-std=c99", "-I", str(ROOT / "include"), str(probe), "-o", str(exe)],
                               capture_output=True, text=True)
    except FileNotFoundError:
        pytest.skip("no C compiler for the layout probe")
    assert built.returncode == 0, built.stderr
    values = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    W = _native.MatvecWeight
    assert values == [ctypes.sizeof(W), W.rows.offset, W.y.offset, W.bias.offset, W.offset.offset,
                      _native.MATVEC_MAX_BATCH, _native.MATVEC_MAX_WEIGHTS]


def test_no_alloc_product_refuses_more_partials_than_its_array():
    """nz_matvec_noalloc checks the product's partial sums against its fixed
    array before touching the device: 2 * n_tiles * batch * 4 bytes over
    NZ_MATVEC_SCRATCH_BYTES fails with NZ_LAYOUT_LIMIT (host-only call)."""
    header = HEADER.read_text()
    limit = int(eval(re.search(r"#define NZ_MATVEC_SCRATCH_BYTES \((.+?)\)", header).group(1).replace("u", "")))
    assert limit == _native.MATVEC_SCRATCH_BYTES
    lib = _native.lib()
    weights = _native.matvec_weights([(0, 8, 1, None)])   # output pointer: never used, the call returns first
    dummy = np.zeros(64, dtype=np.uint8)
    too_many_tiles = limit // (2 * 4 * 4) + 1
    rc = lib.nz_matvec_noalloc(dummy.ctypes.data, dummy.ctypes.data, dummy.ctypes.data, too_many_tiles,
                               dummy.ctypes.data, 1, None, 0, 2, 1, ctypes.addressof(weights), 1, 2048,
                               dummy.ctypes.data, 4, dummy.ctypes.data, None)
    assert rc == -4 and b"no-allocation" in lib.nz_last_error()


def test_decode_args_layout_and_schedule_checks():
    """nz_decode_args is 64 bytes with the header's field order (the ctypes
    mirror is checked against offsets computed from the declaration), and
    nz_decode_schedule rejects missing arrays and events before any HIP
    call; with nothing to do it returns 0 without touching a device."""
    text = re.search(r"typedef struct nz_decode_args \{(.*?)\} nz_decode_args;", HEADER.read_text(), re.S).group(1)
    names = re.findall(r"(\w+);", re.sub(r"/\*.*?\*/", "", text, flags=re.S))
    assert names == [f[0] for f in _native.DecodeArgs._fields_]
    sizes = [8] * 5 + [4] * 6
    offsets = [sum(sizes[:k]) for k in range(len(sizes))]
    assert [getattr(_native.DecodeArgs, n).offset for n in names] == offsets and ctypes.sizeof(_native.DecodeArgs) == 64
    lib = _native.lib()
    one = _native.decode_args([(1, 2, 3, 4, 5, 2, 1, 0, 6, 0)])
    assert lib.nz_decode_schedule(None, 1, None, 0, None, None, None, None, None, None) == -1
    assert lib.nz_decode_schedule(None, 0, one, 1, None, None, None, None, None, None) == -1
    # an ahead launch needs `done` and something for the side stream to wait for (`ready` or `after`)
    token = ctypes.c_void_p(1)
    assert lib.nz_decode_schedule(None, 0, one, 1, None, None, None, token, None, None) == -1
    assert lib.nz_decode_schedule(None, 0, one, 1, None, None, token, None, None, None) == -1
    assert lib.nz_decode_schedule(None, 0, one, 1, None, token, None, None, None, None) == -1
    bad = _native.decode_args([(1, 2, 3, 4, 5, 2, 1, 0, 6, 0)])
    bad[0].reserved = 1
    assert lib.nz_decode_schedule(bad, 1, None, 0, None, None, None, None, None, None) == -1
    assert b"reserved" in lib.nz_last_error()
    assert lib.nz_decode_schedule(None, 0, None, 0, None, None, None, None, None, None) == 0
    # nz_decode_launch_ex: unknown flags, and half-size groups with cached stores, fail before any HIP call
    for flags, message in ((4, b"Unknown decode flags"), (_native.DECODE_CACHED_STORES | _native.DECODE_HALF_GROUPS,
                                                         b"streaming stores only")):
        assert lib.nz_decode_launch_ex(None, None, None, None, 0, 2, 1, 0, None, flags, None) == -1
        assert message in lib.nz_last_error()


def test_numpy_records_match_the_device_structs():
    """The numpy mirrors of the device records (FRAG_DESC, TILE, WORK,
    MATVEC_TILE) have the field names, sizes and offsets of the structs in
    nz_format.h, computed from their declarations (uint64_t / uint32_t /
    uint16_t fields, natural alignment)."""
    text = (ROOT / "neuralzip_amd" / "csrc" / "nz_format.h").read_text()
    width = {"uint64_t": 8, "uint32_t": 4, "uint16_t": 2}

    def layout(name):
        body = re.search(rf"struct {name} \{{(.*?)\}};", text, re.S).group(1)
        fields = re.findall(r"(uint\d+_t)\s+([\w\s,]+);", re.sub(r"//.*", "", body))
        out, offset = [], 0
        for kind, names in fields:
            for n in (x.strip() for x in names.split(",")):
                size = width[kind]
                offset = (offset + size - 1) // size * size
                out.append((n, offset, size))
                offset += size
        return out, (offset + 7) // 8 * 8 if any(s == 8 for _, _, s in out) else offset

    for name, dtype in (("nz_frag_desc", _native.FRAG_DESC), ("nz_work", _native.WORK),
                        ("nz_matvec_tile", _native.MATVEC_TILE)):
        fields, size = layout(name)
        assert dtype.itemsize == size, name
        assert [(n, dtype.fields[n][1], dtype.fields[n][0].itemsize) for n in dtype.names] == fields, name
    # nz_tile's last word is split in two 16-bit halves on the numpy side
    fields, size = layout("nz_tile")
    assert _native.TILE.itemsize == size == 16
    assert [n for n, _, _ in fields] == ["frag", "win0", "out0", "counts"]
    assert _native.TILE.fields["shape"][1] == 12 and _native.TILE.fields["n_out"][1] == 14
