"""The staging stores of the gfx950 tile decode (stage_tile in
neuralzip_amd/csrc/hip/tile_decode.h), simulated on the CPU in lockstep.

The wavefront clears its staging area; then each lane decodes its window's
bytes, which belong at staging indices [at, at + count). Every LUT step ORs
the step's bytes, shifted to their place, into the dword that holds the
first of them and the dword after it (the LDS atomic OR, so lanes of one
instruction may share a dword). Nothing else is written, so no byte is ever
overwritten; a byte can only receive its own value or zeros. That holds
because the final step of a lane may run past its count, and the bytes it
then emits are the next lane's first bytes: the bitstream is continuous, so
decoding on past a window's last code decodes the codes that start in the
next window. The simulation draws random counts, step sizes and tile
origins, and checks every staged byte; it also checks that each of the
scheme's three conditions is needed.
"""
import random

import pytest


def stage(counts, origin, rng, clear=True, continuation=True, store_or=True):
    """Staging bytes after one tile; returns the indices that came out wrong."""
    starts, pos = [], origin
    for c in counts:
        starts.append(pos)
        pos += c
    stream = [rng.getrandbits(8) for _ in range(pos + 8)]   # the tile's bytes, then what follows it
    size = pos + 16
    staging = bytearray(rng.getrandbits(8) for _ in range(size)) if not clear else bytearray(size)
    lanes = []
    for c, at in zip(counts, starts):
        steps, total = [], 0
        while total < c:                     # LUT steps of 1..4 bytes; the last may run past the count
            n = rng.randint(1, 4)
            if continuation:
                steps.append(stream[at + total:at + total + n])
            else:
                steps.append([b if at + total + k < at + c else rng.getrandbits(8)
                              for k, b in enumerate(stream[at + total:at + total + n])])
            total += n
        lanes.append({"bit": 8 * at, "steps": steps})
    active = [i for i, c in enumerate(counts) if c]
    while active:
        stores = []
        for i in active:
            s = lanes[i]
            step = s["steps"].pop(0)
            y = sum(b << (8 * k) for k, b in enumerate(step))
            fill = s["bit"] & 31
            q = (s["bit"] >> 3) & ~3
            stores.append((q, (y << fill) & 0xFFFFFFFF))
            stores.append((q + 4, (y >> (32 - fill)) if fill else 0))   # ubfe(y, 32 - fill, fill)
            s["bit"] += 8 * len(step)
        for q, word in stores:
            old = int.from_bytes(staging[q:q + 4], "little")
            staging[q:q + 4] = ((old | word) if store_or else word).to_bytes(4, "little")
        active = [i for i in active if lanes[i]["steps"]]
    return [j for j in range(origin, pos) if staging[j] != stream[j]]


def wave_counts(rng):
    return [rng.choice([0, 1, 2, 3, 4, 5, 7, rng.randint(0, 40)]) for _ in range(64)]


def test_every_staged_byte_is_the_lanes_byte():
    rng = random.Random(7)
    for _ in range(1500):
        counts = wave_counts(rng)
        while counts and counts[-1] == 0 and rng.random() < 0.5:   # lanes past the tile's windows
            counts.pop()
        assert not stage(counts, 256 + rng.randint(-200, 40), rng)


@pytest.mark.parametrize("broken", ["no clear", "overrun is not the next lane's bytes", "plain stores"])
def test_each_condition_is_needed(broken):
    """Stale staging bytes, a final step whose extra bytes are not the next
    lane's, or plain stores in place of OR must each leave wrong bytes."""
    rng = random.Random(3)
    options = {"no clear": {"clear": False},
               "overrun is not the next lane's bytes": {"continuation": False},
               "plain stores": {"store_or": False}}[broken]
    assert any(stage(wave_counts(rng), 256, rng, **options) for _ in range(50))
