"""Per-dtype byte-lane layout (neuralzip/dtypes.py:7-85).

The selected lane is the exponent byte after moving the sign below the
exponent (bfloat16, float32), or the raw high byte for float16.
"""
from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class DTypeSpec:
    name: str
    torch_dtype: torch.dtype
    numpy: np.dtype
    element_size: int
    bit_reorder: int
    mantissa_bits: int
    exponent_mask: int
    exponent_stream: int | None = None
    global_codebooks: tuple[tuple[int, str], ...] = ()

    @property
    def stream_ids(self):
        return range(self.element_size)

    @property
    def selected_stream(self):
        """The lane the codecs compress (neuralzip/compressor.py:61-64)."""
        return self.exponent_stream if self.exponent_stream is not None else self.element_size - 1

    def reorder_bytes(self, raw_bytes, *, restore=False):
        """The words with the sign bit moved from the top of the word to just
        below the exponent field, or back with `restore` (dtypes.py:23-45).
        A word of size S bits with M mantissa bits is sign:exponent:mantissa
        from the top; reordered it is exponent:sign:mantissa, so the
        exponent of a bfloat16 or float32 word fills its top byte. Layouts
        without the reorder (float16) are returned as they are."""
        if not self.bit_reorder:
            return raw_bytes
        words = np.frombuffer(raw_bytes, dtype=self.numpy)
        m = self.mantissa_bits
        top = 8 * self.element_size - 1                       # the sign bit of the original word
        fraction = words & self.numpy.type((1 << m) - 1)
        if restore:
            sign, exponent = (words >> m) & 1, words >> (m + 1)
            out = (sign << top) | (exponent << m) | fraction
        else:
            sign, exponent = words >> top, (words >> m) & self.exponent_mask
            out = (exponent << (m + 1)) | (sign << m) | fraction
        return out.astype(self.numpy).tobytes()

    def selected_lane(self, raw_bytes):
        """The selected byte lane of the reordered words, without reordering
        the whole buffer. With the sign moved below the exponent, the
        exponent field fills that lane exactly (bfloat16 bits 7-14 land on
        bits 8-15, float32 bits 23-30 on bits 24-31)."""
        if self.bit_reorder:
            return self.extract_exponents(raw_bytes).astype(np.uint8)
        return np.frombuffer(raw_bytes, dtype=np.uint8)[self.selected_stream::self.element_size]

    def extract_exponents(self, raw_bytes):
        """Exponent fields of the original words."""
        values = np.frombuffer(raw_bytes, dtype=self.numpy)
        return (values >> self.mantissa_bits) & self.exponent_mask


bfloat16 = DTypeSpec("bfloat16", torch.bfloat16, np.dtype("<u2"), 2, 1, 7, 0xFF, exponent_stream=1)
float16 = DTypeSpec("float16", torch.float16, np.dtype("<u2"), 2, 0, 10, 0x1F)
float32 = DTypeSpec("float32", torch.float32, np.dtype("<u4"), 4, 1, 23, 0xFF, exponent_stream=3)

DTYPES = {spec.torch_dtype: spec for spec in (float16, bfloat16, float32)}
