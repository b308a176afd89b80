"""Shared builders for layout/decoder tests (oracle = checker, product = under test)."""
import numpy as np
import torch

import oracle
from neuralzip_amd import _native
from neuralzip_amd.dtypes import DTYPES


def segment_lengths(max_bits):
    """Complete NZM1 lengths with a chain 2..max_bits-8 and token 256 of length 1
    (_experiment_kernel_checks.py:63-69)."""
    chain = max_bits - 8
    remaining = 258 - chain
    lengths = list(range(2, chain + 1))
    lengths += [max_bits - 1] * (256 - remaining) + [max_bits] * (2 * remaining - 256)
    lengths.insert(256, 1)
    return bytes(lengths)


def segment_tensor(dtype, symbols):
    """Words whose selected lane is `symbols` and whose other lanes are arbitrary
    bytes, including non-finite patterns (_experiment_kernel_checks.py:77-85)."""
    spec = DTYPES[dtype]
    stream = spec.selected_stream
    reordered = np.arange(len(symbols) * spec.element_size, dtype=np.uint32).astype(np.uint8)
    reordered[stream::spec.element_size] = symbols
    return np.frombuffer(spec.reorder_bytes(reordered.tobytes(), restore=True), dtype=np.uint8).copy()


def singleton_header(raw, dtype, max_bits=12, prior=1):
    spec = DTYPES[dtype]
    lanes = oracle.split_lanes(raw.tobytes(), spec.element_size, spec.bit_reorder, spec.mantissa_bits,
                               spec.exponent_mask.bit_length())
    counts = np.bincount(lanes[spec.selected_stream], minlength=256).astype(np.uint32) + prior
    return oracle.Huff0Table.from_counts(counts, max_bits).header()


class Encoded:
    """Fragments of several tensors packed into a host image of the device buffer."""

    def __init__(self, tensors, codebooks):
        """tensors: list of (raw uint8 array, dtype, chunk elements, [codebook id or -1 per chunk], workspace offset)."""
        self.codebooks = codebooks
        self.entries = []
        for raw, dtype, step, ids, offset in tensors:
            spec = DTYPES[dtype]
            numel = raw.size // spec.element_size
            frags = []
            for j, start in enumerate(range(0, numel, step)):
                part = raw[start * spec.element_size:min(numel, start + step) * spec.element_size]
                book = codebooks[ids[j]] if ids[j] != -1 else None
                frags.append((part, book, offset + start, spec))
            self.entries.append((_native.Layout(frags), ids, offset, spec, numel))

    def host_image(self):
        luts, cursor = {}, 0
        for i, book in self.codebooks.items():
            luts[i] = (cursor, book.lut())
            cursor += (luts[i][1].nbytes + 15) // 16 * 16
        offsets = []
        for layout, *_ in self.entries:
            offsets.append(cursor)
            cursor += layout.packed_bytes
        base = np.zeros(cursor + 16, dtype=np.uint8)
        for off, img in luts.values():
            base[off:off + img.nbytes] = img.view(np.uint8)
        descs, tiles, frag_base = [], [], 0
        for (layout, ids, offset, spec, numel), off in zip(self.entries, offsets):
            lut_offs = np.array([luts[i][0] if i != -1 else 0 for i in ids], dtype=np.uint64)
            d, t = layout.pack(base[off:], off, lut_offs, frag_base)
            descs.append(d)
            tiles.append(t)
            frag_base += layout.n_fragments
        return base, np.concatenate(descs), np.concatenate(tiles)
