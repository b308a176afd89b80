"""Writes tests/golden/huff0_*.zst: Zstd frames of literal-only blocks.

Run from the repository root: `python tests/golden/make_huff0_vectors.py`.
The frames come from pyarrow's bundled libzstd (an implementation independent
of this repository). Inputs are skewed byte sources with large alphabets so
that the compressor finds no matches and every block is Huffman literals.
The manifest records which header kinds (FSE-compressed or direct weights)
and stream counts the vectors cover, plus the SHA-256 of each frame's content.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pyarrow as pa

from zstd_frames import literal_blocks

HERE = Path(__file__).resolve().parent


def source(rng, size, alphabet, low, concentration):
    if concentration < 0:                      # geometric weights with ratio -c
        weights = (-concentration) ** np.arange(alphabet)
        weights /= weights.sum()
    else:
        weights = rng.dirichlet(np.full(alphabet, concentration))
    symbols = np.arange(low, low + alphabet) % 256
    return rng.choice(symbols, size=size, p=weights).astype(np.uint8).tobytes()


def main():
    rng = np.random.default_rng(20261201)
    codec = pa.Codec("zstd", compression_level=1)
    cases = [
        # (size, alphabet, first symbol, dirichlet concentration or -ratio)
        (200, 30, 0, -0.85),        # under 256 literals: one stream
        (400, 48, 100, 0.8),
        (3000, 40, 110, 0.5),
        (20000, 200, 0, 0.3),
        (60000, 90, 30, 0.4),
        (120000, 256, 0, 0.25),     # weights for all 256 symbols: FSE header
        (3000, 40, 0, -0.9),        # geometric: direct 4-bit weights
        (6000, 64, 0, -0.9),
        (6000, 100, 0, -0.9),
        (30000, 64, 64, 1.0),
    ]
    manifest = []
    for index, (size, alphabet, low, concentration) in enumerate(cases):
        for attempt in range(20):
            data = source(rng, size, alphabet, low, concentration)
            frame = codec.compress(data, asbytes=True)
            blocks = list(literal_blocks(frame))
            if all(b is not None for b in blocks) and any(b["kind"] == "huffman" for b in blocks):
                break
        else:
            raise RuntimeError(f"case {index} kept producing sequences")
        name = f"huff0_{index:02d}.zst"
        (HERE / name).write_bytes(frame)
        huffman = [b for b in blocks if b["kind"] == "huffman"]
        manifest.append({
            "file": name,
            "content_bytes": len(data),
            "content_sha256": hashlib.sha256(data).hexdigest(),
            "huffman_blocks": len(huffman),
            "fse_weight_headers": sum(b["tree"][0] < 128 for b in huffman),
            "direct_weight_headers": sum(b["tree"][0] >= 128 for b in huffman),
            "streams": sorted({b["streams"] for b in huffman}),
            "generator": {"size": size, "alphabet": alphabet, "first": low,
                          "concentration": concentration, "attempt": attempt},
        })
    (HERE / "huff0_vectors.json").write_text(json.dumps(
        {"zstd_library": "pyarrow " + pa.__version__, "vectors": manifest}, indent=1) + "\n")
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
