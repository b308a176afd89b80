"""Minimal Zstandard frame reader/writer used to pin the Huff0 restatement.

Zstd's literal sections carry exactly the Huff0 format that the reference's
storage uses for singleton chunks (a Huffman tree description followed by one
stream or a 6-byte jump table and four streams, RFC 8878 3.1.1.3.1 and 4.2).
Frames written by an independent Zstd build (pyarrow's bundled libzstd) whose
blocks hold only literals therefore give known-answer vectors for decoding,
and wrapping our own Huff0 output in a frame lets that libzstd check encoding.
"""

MAGIC = b"\x28\xb5\x2f\xfd"


def tree_description_size(data, offset):
    """Byte size of the Huffman tree description at `offset` (RFC 8878 4.2.1)."""
    header = data[offset]
    if header < 128:
        return 1 + header
    return 1 + (header - 127 + 1) // 2


def literal_blocks(frame):
    """Yield one dict per block of a single frame.

    Compressed blocks whose sequence section is empty expose their Huffman
    literals: `tree` (tree description bytes), `payload` (jump table and
    streams, or the single stream), `streams` (1 or 4), `regenerated` and
    `offset` (position of the literals in the decompressed content).
    Parsing stops at the first block whose content size needs sequence
    decoding; such frames are rejected by returning `None` for that block.
    """
    if frame[:4] != MAGIC:
        raise ValueError("not a zstd frame")
    descriptor = frame[4]
    fcs_flag, single = descriptor >> 6, (descriptor >> 5) & 1
    checksum, dict_flag = (descriptor >> 2) & 1, descriptor & 3
    pos = 5 + (0 if single else 1) + (0, 1, 2, 4)[dict_flag]
    pos += (1 if single else 0, 2, 4, 8)[fcs_flag]
    content = 0
    while True:
        header = int.from_bytes(frame[pos:pos + 3], "little")
        pos += 3
        last, kind, size = header & 1, (header >> 1) & 3, header >> 3
        if kind == 0:
            yield {"kind": "raw", "offset": content, "regenerated": size}
            content += size
            pos += size
        elif kind == 1:
            yield {"kind": "rle", "offset": content, "regenerated": size}
            content += size
            pos += 1
        elif kind == 2:
            block = frame[pos:pos + size]
            pos += size
            info = _compressed_block(block, content)
            yield info
            if info is None:
                return
            content += info["regenerated"]
        else:
            raise ValueError("reserved block type")
        if last:
            break
    if checksum:
        pos += 4
    if pos != len(frame):
        raise ValueError("trailing bytes after the frame")


def huffman_literal_sections(frame):
    """Yield the Huffman literals section of every compressed block of one
    frame that carries its own tree description, whether or not the block
    also has sequences: dicts with `tree`, `payload`, `streams` and
    `regenerated` (the literals' count, not the block's content size)."""
    if frame[:4] != MAGIC:
        raise ValueError("not a zstd frame")
    descriptor = frame[4]
    fcs_flag, single = descriptor >> 6, (descriptor >> 5) & 1
    dict_flag = descriptor & 3
    pos = 5 + (0 if single else 1) + (0, 1, 2, 4)[dict_flag]
    pos += (1 if single else 0, 2, 4, 8)[fcs_flag]
    while True:
        header = int.from_bytes(frame[pos:pos + 3], "little")
        pos += 3
        last, kind, size = header & 1, (header >> 1) & 3, header >> 3
        if kind == 1:
            pos += 1
        else:
            if kind == 2 and frame[pos] & 3 == 2:
                section = _literals_section(frame[pos:pos + size])
                if section is not None:
                    yield section
            pos += size
        if last:
            return


def _literals_section(block):
    b0 = block[0]
    size_format = (b0 >> 2) & 3
    if size_format in (0, 1):
        h, head, bits = int.from_bytes(block[:3], "little"), 3, 10
    elif size_format == 2:
        h, head, bits = int.from_bytes(block[:4], "little"), 4, 14
    else:
        h, head, bits = int.from_bytes(block[:5], "little"), 5, 18
    mask = (1 << bits) - 1
    regenerated = (h >> 4) & mask
    compressed = (h >> (4 + bits)) & mask
    literals = block[head:head + compressed]
    tree = tree_description_size(literals, 0)
    return {"tree": bytes(literals[:tree]), "payload": bytes(literals[tree:]),
            "streams": 1 if size_format == 0 else 4, "regenerated": regenerated}


def _compressed_block(block, content):
    b0 = block[0]
    kind, size_format = b0 & 3, (b0 >> 2) & 3
    if kind in (0, 1):
        if size_format in (0, 2):
            regenerated, head = b0 >> 3, 1
        elif size_format == 1:
            regenerated, head = int.from_bytes(block[:2], "little") >> 4, 2
        else:
            regenerated, head = int.from_bytes(block[:3], "little") >> 4, 3
        rest = head + (regenerated if kind == 0 else 1)
        if block[rest] != 0:
            return None
        return {"kind": "raw_literals" if kind == 0 else "rle_literals",
                "offset": content, "regenerated": regenerated}
    if size_format in (0, 1):
        h, head, bits = int.from_bytes(block[:3], "little"), 3, 10
    elif size_format == 2:
        h, head, bits = int.from_bytes(block[:4], "little"), 4, 14
    else:
        h, head, bits = int.from_bytes(block[:5], "little"), 5, 18
    mask = (1 << bits) - 1
    regenerated = (h >> 4) & mask
    compressed = (h >> (4 + bits)) & mask
    literals = block[head:head + compressed]
    sequences = block[head + compressed:]
    if not sequences or sequences[0] != 0:
        return None
    if kind == 3:
        return {"kind": "treeless", "offset": content, "regenerated": regenerated}
    tree = tree_description_size(literals, 0)
    return {
        "kind": "huffman",
        "offset": content,
        "regenerated": regenerated,
        "streams": 1 if size_format == 0 else 4,
        "tree": bytes(literals[:tree]),
        "payload": bytes(literals[tree:]),
    }


def huffman_frame(tree, payload, regenerated, streams=4):
    """One-block frame whose literals are `tree + payload` and no sequences."""
    compressed = len(tree) + len(payload)
    if streams == 1:
        if regenerated > 1023 or compressed > 1023:
            raise ValueError("single-stream literals need 10-bit sizes")
        size_format, head, bits = 0, 3, 10
    elif regenerated <= 1023 and compressed <= 1023:
        size_format, head, bits = 1, 3, 10
    elif regenerated <= 16383 and compressed <= 16383:
        size_format, head, bits = 2, 4, 14
    else:
        size_format, head, bits = 3, 5, 18
    h = 2 | (size_format << 2) | (regenerated << 4) | (compressed << (4 + bits))
    block = h.to_bytes(head, "little") + tree + payload + b"\x00"
    if len(block) >= 1 << 17:
        raise ValueError("block too large")
    descriptor = (2 << 6) | (1 << 5)          # 4-byte content size, single segment
    block_header = (1 | (2 << 1) | (len(block) << 3)).to_bytes(3, "little")
    return MAGIC + bytes([descriptor]) + regenerated.to_bytes(4, "little") + block_header + block
