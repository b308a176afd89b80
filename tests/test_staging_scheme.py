"""The staging stores of the gfx950 tile decode (stage_tile in
neuralzip_amd/csrc/hip/tile_decode.h), simulated on the CPU in lockstep.

Each lane writes its decoded bytes to staging indices [at, at + count): a
register gathers them, every LUT step stores the aligned dword being filled,
and after the loop each lane stores its own bytes of its first and last
dwords one at a time (a neighbour's dword stores may have left stale bytes
there). The simulation runs the same arithmetic as the kernel, applies the
stores of one instruction in either lane order (same-address stores of one
instruction have no defined winner), and checks that every staged byte is
the lane's byte, for random counts, step sizes and overshoots.
"""
import random

import pytest


def stage(counts, origin, rng, reverse, last_from_loop=False):
    """Staging bytes after one tile; returns the indices that came out wrong."""
    starts, pos = [], origin
    for c in counts:
        starts.append(pos)
        pos += c
    staging = bytearray(rng.getrandbits(8) for _ in range(pos + 64))
    expect, streams = {}, []
    for c, at in zip(counts, starts):
        steps, total = [], 0
        while total < c:                      # LUT steps of 1..4 bytes; the last may overshoot
            n = rng.randint(1, 4)
            steps.append([rng.getrandbits(8) for _ in range(n)])
            total += n
        flat = [x for b in steps for x in b]
        expect.update((at + k, flat[k]) for k in range(c))
        streams.append(steps)
    lanes = []
    for c, at in zip(counts, starts):
        q0, q1 = at & ~3, (at + c - 1) & ~3
        lanes.append({"q": q0, "fill": 8 * (at & 3), "pend": 0, "lead": 0, "word": 0, "cap": 0,
                      "q0": q0, "q1": q1, "at": at, "end": at + c, "i": 0})
    active = [i for i, c in enumerate(counts) if c]
    while active:
        stores = []
        for i in active:
            s = lanes[i]
            step = streams[i][s["i"]]
            s["i"] += 1
            y = sum(b << (8 * k) for k, b in enumerate(step))
            word = ((y << s["fill"]) | s["pend"]) & 0xFFFFFFFF
            s["word"] = word
            stores.append((s["q"], word))
            if s["q"] == s["q0"]:
                s["lead"] = word
            if s["q"] == s["q1"]:
                s["cap"] = word
            spill = (y >> (32 - s["fill"])) if s["fill"] else 0
            s["fill"] += 8 * len(step)
            full = s["fill"] >= 32
            s["pend"] = spill if full else word
            s["q"] += 4 if full else 0
            s["fill"] &= 31
        for q, word in (reversed(stores) if reverse else stores):
            staging[q:q + 4] = word.to_bytes(4, "little")
        active = [i for i in active if lanes[i]["q"] * 8 + lanes[i]["fill"] < lanes[i]["end"] * 8]
    for i, c in enumerate(counts):
        if not c:
            continue
        s = lanes[i]
        last = s["cap"] if last_from_loop else (s["pend"] if s["q"] == s["q1"] else s["word"])
        a, b = s["at"] - s["q0"], s["end"] - s["q1"]
        for k in range(4):
            if k >= a and s["q0"] + k < s["end"]:
                staging[s["q0"] + k] = (s["lead"] >> (8 * k)) & 0xFF
            if k < b and s["q1"] + k >= s["at"]:
                staging[s["q1"] + k] = (last >> (8 * k)) & 0xFF
    return [j for j, x in expect.items() if staging[j] != x]


def wave_counts(rng):
    return [rng.choice([0, 1, 2, 3, 4, 5, 7, rng.randint(0, 40)]) for _ in range(64)]


@pytest.mark.parametrize("reverse", [False, True], ids=["low-lane-last", "high-lane-last"])
def test_every_staged_byte_is_the_lanes_byte(reverse):
    rng = random.Random(7 + reverse)
    for _ in range(800):
        assert not stage(wave_counts(rng), 256 + rng.randint(-200, 40), rng, reverse)


def test_taking_the_last_dword_from_inside_the_loop_fails():
    """The last dword is sometimes never stored in the loop (the final step
    fills the dword before it and spills into it); its bytes are then in the
    pending register. Reading them from the loop's last store at that index
    loses them, which the simulation must catch."""
    rng = random.Random(3)
    assert any(stage(wave_counts(rng), 256, rng, False, last_from_loop=True) for _ in range(50))
