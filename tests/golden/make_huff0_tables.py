"""Writes tests/golden/huff0_tables.json: histograms and the Huffman tree
descriptions that libzstd builds for them.

Run from the repository root: `python tests/golden/make_huff0_tables.py`.
Each case is the literals section of one block of a frame compressed by
pyarrow's bundled libzstd (an implementation independent of this repository).
A literals section carries its own tree description (Zstd's
HUF_buildCTable_wksp then HUF_writeCTable_wksp, the calls the reference
makes in codebooks.h:1-42) and its Huffman streams; decoding the streams with
the oracle gives the literals, whose histogram is what libzstd built the
table from. The table's largest code length is the `max_bits` libzstd passed
(when its tree needed limiting) or the tree's own depth (when it did not),
and either way building with that limit must give the same lengths.

Blocks with sequences are used too: only their literals matter. The sources
cover tied counts (uniform alphabets), trees deeper than the limit
(geometric and Zipf sources), bf16-like exponent bytes, and alphabets from 2
to 256 symbols, so that both FSE-compressed and 4-bit weights appear.
"""
import heapq
import json
import sys
from pathlib import Path

import numpy as np
import pyarrow as pa

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parent.parent))

from zstd_frames import huffman_literal_sections  # noqa: E402
import oracle  # noqa: E402


def unlimited_depth(counts):
    """Depth of one unconstrained Huffman tree (a label only: ties may allow others)."""
    heap = [(int(c), 0, s) for s, c in enumerate(counts) if c]
    heapq.heapify(heap)
    serial = 256
    while len(heap) > 1:
        a, b = heapq.heappop(heap), heapq.heappop(heap)
        heapq.heappush(heap, (a[0] + b[0], max(a[1], b[1]) + 1, serial))
        serial += 1
    return heap[0][1]


def source(rng, kind, size, alphabet, spread):
    if alphabet == 256 or not spread:
        symbols = np.arange(alphabet)   # symbols 0..alphabet-1: short weight lists
    else:
        symbols = (np.arange(alphabet) * 7 + int(rng.integers(0, 256))) % 256
    if kind == "exponents":   # bf16-like exponent bytes with a few outliers
        data = np.clip(np.round(rng.normal(120, 2.5, size)), 0, 255).astype(np.uint8)
        data[rng.integers(0, size, max(1, size // 4000))] = rng.integers(0, 256, max(1, size // 4000))
        return data.tobytes()
    if kind == "uniform":
        p = np.ones(alphabet)
    elif kind == "dirichlet":
        p = rng.dirichlet(np.full(alphabet, 0.4))
    elif kind == "geometric":
        p = float(rng.uniform(0.45, 0.7)) ** np.arange(alphabet)
    else:   # zipf
        p = 1.0 / np.arange(1, alphabet + 1) ** 1.3
    return rng.choice(symbols, size=size, p=p / p.sum()).astype(np.uint8).tobytes()


def main():
    rng = np.random.default_rng(20261202)
    plan = []
    for kind in ("uniform", "dirichlet", "geometric", "zipf"):
        for alphabet in (2, 3, 8, 30, 100, 256):
            for size in (300, 4000, 60000):
                for spread in (False, True):
                    plan.append((kind, alphabet, size, int(rng.choice([1, 3, 9, 19])), spread))
    for kind in ("geometric", "zipf"):   # more trees deeper than the limit
        for alphabet in (40, 64, 128, 256):
            plan.append((kind, alphabet, 120000, 1, True))
    for size in (2000, 30000, 120000):
        plan.append(("exponents", 256, size, 3, False))
    cases, seen = [], set()
    for kind, alphabet, size, level, spread in plan:
        data = source(rng, kind, size, alphabet, spread)
        frame = pa.Codec("zstd", compression_level=level).compress(data, asbytes=True)
        for section in huffman_literal_sections(frame):
            table = oracle.Huff0Table.from_header(section["tree"])
            decode = table.decode4x if section["streams"] == 4 else table.decode1x
            literals = np.frombuffer(decode(section["payload"], section["regenerated"]), np.uint8)
            counts = np.bincount(literals, minlength=256)
            key = (section["tree"], counts.tobytes())
            if key in seen:
                continue
            seen.add(key)
            max_bits = table.codes()[2]
            cases.append({
                "counts": [[int(s), int(c)] for s, c in enumerate(counts) if c],
                "max_bits": int(max_bits),
                "header": section["tree"].hex(),
                "weights": "fse" if section["tree"][0] < 128 else "direct",
                "limited": unlimited_depth(counts) > max_bits,
                "source": {"kind": kind, "alphabet": alphabet, "size": size, "level": level, "spread": spread},
            })
    summary = {
        "cases": len(cases),
        "fse_weights": sum(c["weights"] == "fse" for c in cases),
        "direct_weights": sum(c["weights"] == "direct" for c in cases),
        "limited": sum(c["limited"] for c in cases),
        "max_bits": sorted({c["max_bits"] for c in cases}),
    }
    (HERE / "huff0_tables.json").write_text(json.dumps(
        {"zstd_library": "pyarrow " + pa.__version__, "summary": summary, "cases": cases},
        separators=(",", ":")) + "\n")
    print(json.dumps(summary))


if __name__ == "__main__":
    main()
