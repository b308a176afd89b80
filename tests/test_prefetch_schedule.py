"""The runtime's prefetch schedule, simulated on the CPU.

NeuralZipRuntime._decode_block (the pre-forward hook) issues all of its stream
work through one nz_decode_schedule call. Here that call is replaced by a
model of the two streams: the compute stream is one ordered queue of slot
reads (a block's kernels), inline decodes (slot writes) and event records;
side-stream decodes write their slot once the compute stream waits for their
`done` event. Over random hook sequences (whole forwards, skipped blocks,
stream switches, drains, forwards after a graph capture) two properties must
hold for every slot count:
  * a block reads its slot only when it holds that block's weights and no
    side-stream decode into it may still be running;
  * a side-stream decode starts after the event it waits for (`after`, or
    `ready` recorded in the same call), and nothing queued on the compute
    stream after that event reads or writes the slot it overwrites.
A planted mistake (the side stream always waiting for the previous hook's
record, whatever the slots) must break the second property.
"""
import random

import pytest
import torch

from neuralzip_amd import _native
from neuralzip_amd.gpu import inference
from neuralzip_amd.gpu.inference import NeuralZipRuntime, _unit_slots


class StreamModel:
    def __init__(self, runtime):
        self.runtime = runtime
        self.queue = []          # compute-stream ops in issue order: (kind, value)
        self.records = {}        # event -> index into queue of its latest record
        self.side = []           # side-stream decodes not yet waited for: (unit, done event)
        self.content = {}        # slot -> unit whose weights it holds (writes applied)
        self.after_used = 0

    def slot(self, unit):
        return self.runtime.block_slot[unit]

    def wait(self, event):
        """The compute stream waits for a side-stream `done`: that decode and
        every earlier one on the in-order side stream have completed."""
        for k, (unit, done) in enumerate(self.side):
            if done == event:
                for u, _ in self.side[:k + 1]:
                    self.content[self.slot(u)] = u
                del self.side[:k + 1]
                return
        raise AssertionError(f"wait for {event}, which no pending decode records")

    def schedule(self, inline, ahead, wait, ready, done, stream, side, after=None):
        if wait is not None:
            self.wait(wait)
        if inline is not None:
            unit = inline[1]
            assert all(self.slot(u) != self.slot(unit) for u, _ in self.side), "inline decode races a side decode"
            self.queue.append(("write", self.slot(unit)))
            self.content[self.slot(unit)] = unit
        if ahead is not None:
            unit = ahead[1]
            assert done is not None and (ready is not None or after is not None)
            if ready is not None:
                self.queue.append(("record", ready))
                self.records[ready] = len(self.queue) - 1
            target = after if after is not None else ready
            if after is not None:
                self.after_used += 1
            assert target in self.records, "the side stream waits for an event never recorded"
            since = self.queue[self.records[target] + 1:]
            clash = [op for op in since if op[0] in ("read", "write") and op[1] == self.slot(unit)]
            assert not clash, f"decode of {unit} into slot {self.slot(unit)} overlaps {clash}"
            self.side.append((unit, done))

    def block_runs(self, unit):
        """The block's kernels after its hook: they read its slot."""
        slot = self.slot(unit)
        assert all(self.slot(u) != slot for u, _ in self.side), f"{unit} reads a slot a side decode may write"
        assert self.content.get(slot) == unit, f"{unit} reads slot {slot} holding {self.content.get(slot)}"
        self.queue.append(("read", slot))


def fake_runtime(n_units, cycle, monkeypatch):
    order = tuple(f"blocks.{i}" for i in range(n_units))
    rt = object.__new__(NeuralZipRuntime)
    rt.units = order
    rt.block_slot = _unit_slots(order, cycle)
    rt._following = {name: order[(i + 1) % len(order)] for i, name in enumerate(order)}
    rt._segmenting, rt._eager_decodes, rt._matvec_blocks, rt._fused = None, False, frozenset(), set()
    rt._pending, rt._markers, rt._wrap, rt._side_off = None, [], True, False
    rt._schedule_args = {u: ("args", u) for u in order}
    rt._ahead_args = rt._schedule_args
    rt._events = {u: (("ready", u), ("done", u)) for u in order}
    rt.side_stream, rt._side_handle, rt.device, rt.workspaces = object(), "side", None, {}
    model = StreamModel(rt)
    current = {"stream": "A"}
    monkeypatch.setattr(_native, "decode_schedule", model.schedule)
    monkeypatch.setattr(inference, "_current_stream_handle", lambda device: current["stream"])
    return rt, model, current


def drive(rt, model, current, rng, forwards=12):
    order = rt.units
    for f in range(forwards):
        if rng.random() < 0.15:
            rt.drain()
        if rng.random() < 0.2:
            current["stream"] = "B" if current["stream"] == "A" else "A"
        if f == forwards // 2 and rng.random() < 0.5:
            rt.drain()
            rt._wrap = False   # after a graph capture: the last block no longer prefetches the first
        units = [u for u in order if rng.random() > 0.1] or [order[0]]
        for unit in units:
            rt._decode_block(unit)
            model.block_runs(unit)


@pytest.mark.parametrize("cycle", [2, 3, 4, 5])
@pytest.mark.parametrize("n_units", [2, 3, 4, 5, 7, 8, 33])
def test_hooks_never_overwrite_a_slot_in_use(cycle, n_units, monkeypatch):
    rt, model, current = fake_runtime(n_units, cycle, monkeypatch)
    with torch.no_grad():
        for seed in range(6):
            drive(rt, model, current, random.Random(seed * 100 + n_units))
    slots = len(set(rt.block_slot.values()))
    if slots >= 3 and n_units >= 3:
        assert model.after_used > 0   # the earlier record is used where the slots allow it


def test_three_slots_use_the_previous_record_for_every_hook_after_the_first(monkeypatch):
    rt, model, current = fake_runtime(33, 3, monkeypatch)
    with torch.no_grad():
        for _ in range(3):
            for unit in rt.units:
                rt._decode_block(unit)
                model.block_runs(unit)
    assert model.after_used == 3 * 33 - 1


@pytest.mark.parametrize("cycle", [3, 4, 5, 6])
def test_more_slots_wait_for_older_records(cycle, monkeypatch):
    """With `cycle` slots, a hook in the middle of a forward has the side
    stream wait for the record made cycle - 2 hooks earlier: the oldest after
    which no queued block holds the slot being refilled."""
    rt, model, current = fake_runtime(33, cycle, monkeypatch)
    calls = []
    schedule = model.schedule

    def spy(inline, ahead, wait, ready, done, stream, side, after=None):
        calls.append(after)
        schedule(inline, ahead, wait, ready, done, stream, side, after)
    monkeypatch.setattr(_native, "decode_schedule", spy)
    order = rt.units
    with torch.no_grad():
        for _ in range(2):
            for unit in order:
                rt._decode_block(unit)
                model.block_runs(unit)
    for i in range(cycle, len(order) - cycle):
        # hook w records ("ready", unit w + 1)
        assert calls[len(order) + i] == ("ready", order[i - (cycle - 2) + 1]), i


def test_two_slots_wait_for_a_record_made_in_the_same_call(monkeypatch):
    """Units 0..31 alternate two slots and the last takes a third: only the
    hooks next to the last unit may use the earlier record."""
    rt, model, current = fake_runtime(33, 2, monkeypatch)
    with torch.no_grad():
        for _ in range(2):
            for unit in rt.units:
                rt._decode_block(unit)
                model.block_runs(unit)
    assert model.after_used == 2 * 3 - 1


@pytest.mark.parametrize("cycle, careless", [
    (2, lambda self, following, stream: self._markers[-1][1] if self._markers else None),   # previous record
    (4, lambda self, following, stream: self._markers[0][1] if self._markers else None),    # oldest record
])
def test_a_planted_rule_that_ignores_the_slots_is_caught(cycle, careless, monkeypatch):
    rt, model, current = fake_runtime(9, cycle, monkeypatch)
    monkeypatch.setattr(NeuralZipRuntime, "_earlier_marker", careless)
    with torch.no_grad(), pytest.raises(AssertionError, match="overlaps"):
        for unit in rt.units * 2:
            rt._decode_block(unit)
            model.block_runs(unit)


def test_unit_slots():
    order = tuple("abcdefg")
    for cycle in range(2, 6):
        slots = _unit_slots(order, cycle)
        assert all(slots[a] != slots[b] for a, b in zip(order, order[1:] + order[:1]))
        assert max(slots.values()) <= cycle
    assert set(_unit_slots(order, 1).values()) == {0}
    assert _unit_slots(("a",), 3) == {"a": 0}
    assert _unit_slots(tuple("abcde"), 3) == {"a": 0, "b": 1, "c": 2, "d": 0, "e": 1}
    assert _unit_slots(tuple("abcde"), 2) == {"a": 0, "b": 1, "c": 0, "d": 1, "e": 2}
