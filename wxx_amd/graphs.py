"""Step graphs: one call of a step function recorded from the library's
stream as a HIP graph and replayed with a single launch.

The reference encodes every dispatch of every step again on the host
(reference src/wxx/backend/device.py:15-16 notes that this host cost
dominates small models).  Here a step that has run eagerly at least once is
recorded once with :class:`StepGraph` and then replayed: every kernel,
device copy and upload of the step runs again, in the same order, with one
``hipGraphLaunch`` and no Python dispatch.

What a replay repeats, and what it does not:

* device work: exactly the recorded sequence, on the same device addresses.
  Tensors the step reads (parameters, optimizer moments, inputs) must stay
  alive while the graph does; new input data goes into the same tensors
  before a replay (``functional.assign(x, from_numpy(batch))``).  Blocks the recording
  allocated belong to the graph until :meth:`StepGraph.close`, so outputs the
  step returned (a loss) are rewritten by every replay;
* uploads made while recording (position ids, descriptor tables) are
  replayed with the bytes recorded;
* host state that a step advances is advanced before each launch by hooks
  the recording registered, in recording order: the optimizer's step count
  and bias corrections, the scheduler's learning rate, each dropout call's
  seed from the host RNG.  Values a kernel needs from them live in a block of
  per-replay device words (:func:`per_replay`) uploaded once per replay, so a
  replayed step computes what the eager step would have;
* checks that the eager step makes by reading the device (cross-entropy
  target range) run after the launch, once the replay has finished.

While recording, nothing runs on the device; a call that would wait for the
device (reading a tensor back, synchronising) raises ``HIPError`` and the
recording is abandoned.
"""

import ctypes as C

import numpy as np

from .backend import lib as _lib
from .backend.device import ensure_device, get_buffer_pool

MAX_REPLAY_WORDS = 4096
"""32-bit per-replay device words one graph can hold."""

_state = {"recording": None}


class _Recording:
    def __init__(self):
        self.hooks = []   # (offset, count, fill) in recording order
        self.checks = []  # run after each replay, once it has finished
        self.keep = []    # objects whose device memory the graph uses
        self.used = 0
        self.words = np.zeros(MAX_REPLAY_WORDS, np.uint32)
        self.block = get_buffer_pool().create_buffer(4 * MAX_REPLAY_WORDS,
                                                     label="step graph words")


def capturing():
    """True while a step graph is being recorded."""
    return _state["recording"] is not None


def _recording(what):
    rec = _state["recording"]
    if rec is None:
        raise RuntimeError(f"{what} is only available while a step graph is being recorded")
    return rec


def per_replay(count, fill):
    """Reserve ``count`` 32-bit device words whose values ``fill(words)``
    writes (into a numpy uint32 array of that length) before every replay;
    returns their device address for the recorded kernels to read."""
    rec = _recording("per_replay")
    if rec.used + count > MAX_REPLAY_WORDS:
        raise RuntimeError(f"a step graph holds at most {MAX_REPLAY_WORDS} per-replay words")
    off = rec.used
    rec.used += count
    rec.hooks.append((off, count, fill))
    return rec.block.ptr + 4 * off


def on_replay(fn):
    """Run ``fn()`` on the host before every replay (host state the eager
    step would advance)."""
    _recording("on_replay").hooks.append((0, 0, lambda words: fn()))


def after_replay(check):
    """Run ``check()`` after every replay has finished on the device."""
    _recording("after_replay").checks.append(check)


def keep_alive(*objs):
    """Hold ``objs`` for as long as the graph lives."""
    _recording("keep_alive").keep.extend(objs)


class StepGraph:
    """``fn`` (a callable taking no arguments) recorded once and replayed.

    ``capture()`` records one call of ``fn`` and runs nothing on the device;
    each ``replay()`` (or call of the object) then performs one step.  ``fn``
    should have run eagerly at least once first, so lazily created state
    (optimizer moments, cached masks, FFT tables) exists and the allocator's
    cache holds blocks of every size the step uses.  ``result`` is what
    ``fn`` returned during the recording; device tensors in it hold each
    replay's values once that replay has finished.
    """

    def __init__(self, fn):
        self.fn = fn
        self.result = None
        self.nodes = 0
        self._handle = None
        self._rec = None

    def capture(self):
        if self._handle is not None:
            raise RuntimeError("this step graph has already been recorded")
        if capturing():
            raise RuntimeError("another step graph is being recorded")
        ensure_device()
        rec = _Recording()
        _lib.call("wxx_graph_begin")
        _state["recording"] = rec
        try:
            result = self.fn()
        except BaseException:
            _state["recording"] = None
            _lib.load().wxx_graph_abort()
            raise
        _state["recording"] = None
        handle = C.c_void_p()
        nodes = C.c_int64(0)
        _lib.call("wxx_graph_end", C.byref(handle), C.byref(nodes))
        self._handle = handle
        self._rec = rec
        self.result = result
        self.nodes = int(nodes.value)
        return self

    def replay(self):
        """Advance the host state the step advances, upload the per-replay
        words, launch the recording, then run the recorded checks."""
        if self._handle is None:
            raise RuntimeError("capture() the step graph before replaying it")
        rec = self._rec
        for off, count, fill in rec.hooks:
            fill(rec.words[off:off + count])
        if rec.used:
            _lib.call("wxx_h2d", C.c_void_p(rec.block.ptr),
                      rec.words.ctypes.data_as(C.c_void_p), 4 * rec.used)
        _lib.call("wxx_graph_launch", self._handle)
        if rec.checks:
            _lib.call("wxx_sync")
            for check in rec.checks:
                check()
        return self.result

    __call__ = replay

    def close(self):
        """Release the graph and the device blocks it owns (waits for a
        replay in flight)."""
        if self._handle is not None:
            handle, self._handle = self._handle, None
            try:
                _lib.call("wxx_graph_destroy", handle)
            finally:
                self._rec = None
                self.result = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass


__all__ = ["StepGraph", "capturing", "per_replay", "on_replay", "after_replay", "keep_alive",
           "MAX_REPLAY_WORDS"]
