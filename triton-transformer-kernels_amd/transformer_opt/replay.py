"""hipGraph replay of the encoder forward.

The model resolves, once per call, every tensor and scalar its forward reads
(``submission._Operands``) and fingerprints that read set.  This module keeps
what outlives a call:

* ``PackedQKV`` - the Q, K and V projection weights concatenated into one
  ``[3d, d]`` GEMM operand, valid while its six source tensors are the same
  objects with the same storage and version counters;
* ``CapturedForward`` - one forward captured as a ``torch.cuda.CUDAGraph``
  (a hipGraph on ROCm) over static input buffers, replayed with fresh inputs
  copied in and a clone of the static output returned;
* ``ReplayCache`` - the captures of one model fingerprint, least recently
  used first, keyed by input geometry, plus the packed projections and the
  lock that serialises capture and replay.

The contract follows the reference's replay (transformer_opt/submission.py:
527-723): any change to what a capture baked in makes it stale, every replay
returns a tensor the caller owns, replays on different caller streams are
ordered by an event, warm-up and capture are not counted as forwards, and a
device or dtype move drops every capture.
"""

from __future__ import annotations

import gc
import threading
from collections import OrderedDict
from typing import Callable, Dict, Hashable, Optional, Sequence

import torch


class CallTally:
    """Kernel launches one forward performs, by kind."""

    __slots__ = ("attention", "fused_norms")

    def __init__(self) -> None:
        self.attention: Dict[str, int] = {}
        self.fused_norms = 0

    def count_attention(self, selected: str) -> None:
        self.attention[selected] = self.attention.get(selected, 0) + 1

    def count_fused_norm(self) -> None:
        self.fused_norms += 1


def tensor_stamp(t: torch.Tensor) -> tuple:
    """Identity, storage and in-place version of a tensor.

    Any of these changing means a GEMM operand or a captured kernel argument
    may differ: a replaced parameter object, a ``.data`` swap or a device or
    dtype move (new storage), or an in-place update (``add_``, ``copy_``,
    ``load_state_dict``; version counter).
    """
    return (id(t), t.data_ptr(), t._version)


class PackedQKV:
    """``cat(Wq, Wk, Wv)`` and ``cat(bq, bk, bv)`` for one packed projection GEMM.

    The reference keeps the same derived operand outside the state dict and
    rebuilds it whenever a source changes (transformer_opt/submission.py:
    145-217).  Sources that are inference tensors have no version counter,
    so such a pack is never reused.
    """

    __slots__ = ("sources", "stamp", "weight", "bias")

    def __init__(self, weights: Sequence[torch.Tensor], biases: Sequence[Optional[torch.Tensor]]):
        filled = [b if b is not None else w.new_zeros(w.shape[0]) for w, b in zip(weights, biases)]
        self.sources = tuple(weights) + tuple(biases)
        self.stamp = PackedQKV.stamp_of(self.sources)
        with torch.no_grad():
            self.weight = torch.cat(tuple(weights), dim=0).detach()
            self.bias = torch.cat(filled, dim=0).detach()

    @staticmethod
    def stamp_of(sources: Sequence[Optional[torch.Tensor]]) -> Optional[tuple]:
        if any(t is not None and t.is_inference() for t in sources):
            return None
        return tuple(None if t is None else tensor_stamp(t) for t in sources)

    def serves(self, weights, biases) -> bool:
        if self.stamp is None:
            return False
        return self.stamp == PackedQKV.stamp_of(tuple(weights) + tuple(biases))


class PackedOut:
    """The attention output projection's weight in the MFMA fragment order of
    the fused projection + residual + LayerNorm kernel, rebuilt whenever the
    weight changes (same rule as ``PackedQKV``).  ``packed`` is None when that
    kernel cannot take the weight (not a 16-bit [1024, K] ROCm tensor with K a
    multiple of 128)."""

    __slots__ = ("sources", "stamp", "packed")

    def __init__(self, weight: torch.Tensor):
        from .kernels.linear_ln import WIDTH, pack_weight

        self.sources = (weight,)
        self.stamp = PackedQKV.stamp_of(self.sources)
        self.packed = None
        if (weight.is_cuda and weight.dtype in (torch.bfloat16, torch.float16) and weight.ndim == 2
                and weight.shape[0] == WIDTH and weight.shape[1] % 128 == 0):
            with torch.no_grad():
                self.packed = pack_weight(weight.detach())

    def serves(self, weight: torch.Tensor) -> bool:
        return self.stamp is not None and self.stamp == PackedQKV.stamp_of((weight,))


_CAPTURE_STREAMS: Dict[int, torch.cuda.Stream] = {}
_CAPTURE_STREAMS_LOCK = threading.Lock()


def capture_stream(device: torch.device) -> torch.cuda.Stream:
    """One side stream per device for warm-up and capture.

    Reusing it keeps the library GEMM workspace that torch creates per stream
    from multiplying with every capture.  Default priority.
    """
    index = device.index if device.index is not None else torch.cuda.current_device()
    with _CAPTURE_STREAMS_LOCK:
        stream = _CAPTURE_STREAMS.get(index)
        if stream is None:
            stream = torch.cuda.Stream(device=index)
            _CAPTURE_STREAMS[index] = stream
        return stream


class CapturedForward:
    """One forward captured over static buffers, replayable with new inputs.

    ``run(x, mask, tally)`` is the eager forward with its operands already
    resolved; it runs once on the capture stream to create every lazily
    allocated library resource outside the graph pool, then once under
    capture.  ``tally`` holds the launches of one forward, added to the
    model's counters per replay.  ``keepalive`` pins the tensors the graph
    reads by address for as long as the capture exists.
    """

    def __init__(self, run: Callable, x: torch.Tensor, mask: Optional[torch.Tensor],
                 keepalive: tuple) -> None:
        self.keepalive = keepalive
        caller = torch.cuda.current_stream(x.device)
        side = capture_stream(x.device)
        # Capture outside inference mode: torch creates the generator's
        # graph-safe RNG state at the first capture of a process and updates
        # it at every later one, so it must not be an inference tensor.  The
        # replay clones the output in the caller's mode.
        with torch.inference_mode(False), torch.no_grad():
            self.x = x.clone()
            self.mask = None if mask is None else mask.clone()
            side.wait_stream(caller)
            with torch.cuda.stream(side):
                run(self.x, self.mask, CallTally())
                self.tally = CallTally()
                self.graph = torch.cuda.CUDAGraph()
                # No cyclic garbage collection during the capture: garbage
                # that holds another capture (a dropped model in a reference
                # cycle) would destroy its graph and release its memory pool
                # while this stream captures, which HIP does not allow; the
                # error inside that destructor aborts the process.  torch
                # does not collect before a capture by default.
                collecting = gc.isenabled()
                gc.disable()
                try:
                    with torch.cuda.graph(self.graph, stream=side):
                        self.out = run(self.x, self.mask, self.tally)
                finally:
                    if collecting:
                        gc.enable()
            caller.wait_stream(side)
        # Recorded on the stream of the most recent replay; the next replay,
        # on whatever stream, waits for it before touching the static buffers.
        self.released = torch.cuda.Event()
        self.released.record(caller)

    def replay(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
        stream = torch.cuda.current_stream(x.device)
        stream.wait_event(self.released)
        self.x.copy_(x)
        if self.mask is not None:
            self.mask.copy_(mask)
        self.graph.replay()
        result = self.out.clone()
        self.released.record(stream)
        return result


class ReplayCache:
    """Captures of one model fingerprint (LRU by geometry) and packed projections.

    Not copied with the model: ``copy.deepcopy`` and pickling give an empty
    cache of the same capacity, since captures hold device graphs and static
    buffers that belong to the original.
    """

    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.lock = threading.RLock()
        self.fingerprint: Optional[Hashable] = None
        self.entries: "OrderedDict[Hashable, CapturedForward]" = OrderedDict()
        self.last: Optional[CapturedForward] = None
        self.packs: Dict[int, PackedQKV] = {}
        self.out_packs: Dict[int, PackedOut] = {}
        # The model's module-tree layout and the operands resolved from it,
        # with the (layout epoch, tensor stamps, scalars) key they were
        # resolved under; owned by the model, cached here so copies start
        # empty.
        self.layout = None
        self.layout_epoch = 0
        self.operands = None
        self.operands_key = None

    def __deepcopy__(self, memo) -> "ReplayCache":
        return ReplayCache(self.capacity)

    def __reduce__(self):
        return (ReplayCache, (self.capacity,))

    def drop_captures(self) -> None:
        self.entries.clear()
        self.last = None
        self.fingerprint = None

    def reset(self) -> None:
        """Forget every capture and packed projection (device/dtype moves)."""
        with self.lock:
            self.drop_captures()
            self.packs.clear()
            self.out_packs.clear()
            self.layout = None
            self.operands = None
            self.operands_key = None

    def pack_for(self, slot: int, weights, biases) -> PackedQKV:
        pack = self.packs.get(slot)
        if pack is None or not pack.serves(weights, biases):
            pack = PackedQKV(weights, biases)
            self.packs[slot] = pack
        return pack

    def out_pack_for(self, slot: int, weight: torch.Tensor) -> PackedOut:
        pack = self.out_packs.get(slot)
        if pack is None or not pack.serves(weight):
            pack = PackedOut(weight)
            self.out_packs[slot] = pack
        return pack

    def entry(self, fingerprint: Hashable, geometry: Hashable,
              build: Callable[[], CapturedForward]) -> CapturedForward:
        """The capture for ``geometry`` under ``fingerprint``, built if absent.

        A new fingerprint means the model changed since the cached captures
        were made: all of them are dropped (they would also pin the old
        storage).  Call with ``lock`` held.
        """
        if fingerprint != self.fingerprint:
            self.drop_captures()
            self.fingerprint = fingerprint
        captured = self.entries.get(geometry)
        if captured is None:
            captured = build()
            self.entries[geometry] = captured
            while len(self.entries) > self.capacity:
                self.entries.popitem(last=False)
        else:
            self.entries.move_to_end(geometry)
        self.last = captured
        return captured
