"""Frozen weights streamed through a bounded device window — borch's scale primitives on
this surface (``borch_amd.streaming``; the reference puts them under ``torch.streaming``).

* ``window(byte_size)`` / ``Window``: one device buffer that holds many weights end to end,
  each in an aligned slot (borch-ts/src/device.ts:2990-3165). A slot is reserved first fit
  from the regions that evictions freed, else at the growing cursor; past the capacity
  ``place`` raises ``WindowFull`` with the reference's text. Every offset carries a
  generation, bumped when the offset is (re)written or evicted.
* ``in_window`` / ``in_window_f16`` / ``in_window_int8(win, data, shape)``: a frozen weight
  placed in a slot as f32, f16 or per-output-channel int8 (tensor.ts:1620-1705), returned as
  ``(weight, evict)``. The int8 form quantizes on the host (``bq_quantize_weight_host``: the
  bytes of ``bq_quantize_weight_per_channel``, or with ``rounding="reference"`` the bytes of
  borch-ts's own packer, quant.ts:35-41), copies only the int8 bytes into the slot (a quarter
  of the f32 bytes) and keeps the per-channel scales in a small resident tensor.
  ``F.linear`` reads the int8 slot in place with the weight-only kernel
  (``bq_linear_w8a32``: the reference's int8 read, kernels.ts:2695-2708); ``matmul`` and
  ``conv2d`` unpack it to f32 first (``bq_dequant_i8``; the reference's other weight funnels
  dequantize to f32 scratch, tensor.ts:1330-1350). A use after the slot was evicted raises
  the reference's "evicted" error (tensor.ts:1692-1699); any other op on a windowed weight
  raises (it is a weight operand only).
* ``stream_sequential(win, input, blocks, int8=..., f16=...)``: a no-grad forward over
  blocks whose weights pass through the window: place a block's weights, run it, evict them
  (stream.ts:36-68; borch_webgpu/_stream.py:61-66).

MI355X-first, where the reference serializes: every host-to-device copy runs on the
window's own copy stream, from pinned host memory, and ``stream_sequential`` places block
k+1 while block k runs (when the window has room for both), so the copies overlap the
compute. Ordering is by events, never by a host wait: a slot's first use waits (on the
using stream) for the copy that filled it, and a copy into a reused region waits for the
event its eviction recorded on the stream that last used it. ``pack_int8_host`` packs a
weight once into pinned memory, so a weight streamed many times is not re-quantized on
every placement (the bytes are the same either way).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, NamedTuple, Sequence

import numpy as np
import torch

from . import _lib
from . import int8 as _i8
from ._lib import check, lib, require_device

__all__ = ["ALIGN", "Window", "WindowFull", "window", "Slot", "WindowedWeight", "Placed", "HostInt8Weight",
           "pack_int8_host", "in_window", "in_window_f16", "in_window_int8", "StreamBlock", "stream_sequential",
           "EVICTED_MESSAGE"]

ALIGN = 256  # slot alignment in bytes (every slot offset is a multiple; 16-byte loads need 16)

EVICTED_MESSAGE = ("this windowed weight was evicted — its slot holds another weight now. "
                   "Re-place it in the window before using it.")

_ROUNDING = {"exact": _lib.ROUND_EXACT, "reference": _lib.ROUND_REFERENCE,
             "reference_conv": _lib.ROUND_REFERENCE_CONV}


class WindowFull(RuntimeError):
    """No freed region fits and the cursor would pass the window's capacity."""


class Regions:
    """The window's host-side bookkeeping, with no device state (device.ts:3015-3165):
    the cursor (high-water mark), the freed regions (first fit, each taken whole, no
    coalescing: the streaming case is equal-sized blocks), the reserved size of each live
    slot, and the generation of each offset. ``token`` is whatever the caller attaches to a
    freed region (the window: the event its eviction recorded) and gets back on reuse."""

    def __init__(self, capacity: int, align: int = ALIGN):
        self.capacity = int(capacity)
        self.align = int(align)
        self.cursor = 0
        self.freed: list[tuple[int, int, object]] = []
        self.reserved: dict[int, int] = {}
        self.gens: dict[int, int] = {}
        self.tick = 0

    def need(self, nbytes: int) -> int:
        return max(1, -(-int(nbytes) // self.align)) * self.align

    def reserve(self, nbytes: int):
        """(offset, generation, token of the freed region reused or None)."""
        need = self.need(nbytes)
        hit = next((i for i, (_, size, _) in enumerate(self.freed) if size >= need), None)
        if hit is not None:
            offset, size, token = self.freed.pop(hit)
        else:
            offset, size, token = self.cursor, need, None
            if offset + need > self.capacity:
                raise WindowFull(
                    f"window is full: {offset} + {need} > {self.capacity} bytes, and no freed region fits. "
                    "Evict a slot, or size the window larger.")
            self.cursor = offset + need
        self.reserved[offset] = size
        self.tick += 1
        self.gens[offset] = self.tick
        return offset, self.tick, token

    def release(self, offset: int, token=None) -> None:
        """Evicts the slot at ``offset``: its generation moves on (a stale use is loud) and
        its region returns to the free list with ``token``."""
        self.tick += 1
        self.gens[offset] = self.tick
        size = self.reserved.pop(offset, None)
        if size is not None:
            self.freed.append((offset, size, token))

    def gen_of(self, offset: int) -> int:
        return self.gens.get(offset, -1)

    @property
    def used(self) -> int:
        return self.cursor

    @property
    def live(self) -> int:
        return sum(self.reserved.values())


@dataclass
class Slot:
    """One placed weight's bytes: ``[offset, offset + size)`` of the window buffer, the
    generation it was placed at, and the event recorded after the copy that filled it."""
    window: "Window"
    offset: int
    size: int
    gen: int
    ready: torch.cuda.Event | None
    _waited: set | None = None

    def live(self) -> bool:
        return self.window._open and self.window.regions.gen_of(self.offset) == self.gen

    def check_live(self) -> None:
        if not self.window._open:
            raise RuntimeError("this windowed weight's window was freed")
        if self.window.regions.gen_of(self.offset) != self.gen:
            raise RuntimeError(EVICTED_MESSAGE)

    def ensure_ready(self, stream: torch.cuda.Stream) -> None:
        """The using stream waits for the slot's copy (once per stream)."""
        if self.ready is None:
            return
        if self._waited is None:
            self._waited = set()
        if stream.cuda_stream not in self._waited:
            stream.wait_event(self.ready)
            self._waited.add(stream.cuda_stream)

    def view(self, dtype: torch.dtype, shape) -> torch.Tensor:
        t = self.window.buffer[self.offset:self.offset + self.size]
        return t.view(dtype).view(tuple(shape))


class Window:
    """A bounded slice of device memory the frozen weights stream through (device.ts:2990-3165).
    ``free()`` releases it; the slots of a freed window refuse every use."""

    def __init__(self, byte_size: int, device=None):
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        require_device(dev)
        if int(byte_size) <= 0:
            raise ValueError(f"a window needs a positive size, got {byte_size}")
        self.device = dev
        self.capacity = int(byte_size)
        self.buffer = torch.empty(self.capacity, dtype=torch.uint8, device=dev)
        self.regions = Regions(self.capacity, ALIGN)
        self.copy_stream = torch.cuda.Stream(device=dev)  # default priority
        self.buffer.record_stream(self.copy_stream)  # the allocator sees the copies as uses
        self._open = True

    @property
    def used(self) -> int:
        """The high-water mark of the cursor, in bytes (stays near the resident set)."""
        return self.regions.used

    @property
    def live(self) -> int:
        """Bytes currently placed and not evicted."""
        return self.regions.live

    def place(self, data) -> Slot:
        """Copies host ``data`` (a numpy array or a CPU tensor, any dtype; pinned memory is
        copied from directly, anything else staged through a pinned buffer) into the next
        slot, on the window's copy stream. Returns at once; the copy is ordered after the
        eviction that freed a reused region, and every use of the slot waits for it."""
        if not self._open:
            raise RuntimeError("this window was freed")
        src = _host_bytes(data)
        offset, gen, freed_evt = self.regions.reserve(src.numel())
        ready = None
        if src.numel():
            with torch.cuda.stream(self.copy_stream):
                if freed_evt is not None:
                    self.copy_stream.wait_event(freed_evt)
                self.buffer[offset:offset + src.numel()].copy_(src, non_blocking=True)
                ready = torch.cuda.Event()
                ready.record(self.copy_stream)
        return Slot(self, offset, src.numel(), gen, ready)

    def evict(self, slot: Slot) -> None:
        """Frees ``slot`` for the next placement; a later use of its weight raises. The
        region is reused only after the work enqueued so far on the current stream (the
        slot's last readers) has run: the next copy into it waits for this point."""
        if not self._open or slot.window is not self:
            return
        if self.regions.gen_of(slot.offset) != slot.gen:
            return  # already evicted
        evt = torch.cuda.Event()
        evt.record(torch.cuda.current_stream(self.device))
        self.regions.release(slot.offset, evt)

    def free(self) -> None:
        """Returns the window's memory; every slot's weight refuses use after this."""
        if self._open:
            self._open = False
            torch.cuda.current_stream(self.device).wait_stream(self.copy_stream)
            self.buffer = None


def window(byte_size: int, device=None) -> Window:
    """A window of ``byte_size`` bytes on ``device`` (borch_webgpu/_stream.py:30-32)."""
    return Window(byte_size, device)


def _host_bytes(data) -> torch.Tensor:
    """``data`` as a flat uint8 CPU tensor in pinned memory (a pinned tensor is used as is)."""
    t = torch.from_numpy(np.ascontiguousarray(data)) if isinstance(data, np.ndarray) else data
    if not isinstance(t, torch.Tensor) or t.device.type != "cpu":
        raise TypeError("a window is filled from host memory (a numpy array or a CPU tensor)")
    t = t.contiguous().reshape(-1).view(torch.uint8)
    if t.is_pinned():
        return t
    pinned = torch.empty(t.numel(), dtype=torch.uint8, pin_memory=True)
    pinned.copy_(t)
    return pinned


# ------------------------------------------------------------------ host int8 packing

@dataclass
class HostInt8Weight:
    """A weight packed on the host for an int8 window slot: ``q int8 [N, Kpad]`` (K padded
    to a multiple of 16 with zeros) and ``s f32 [N]``, both in pinned memory when a GPU is
    present; ``shape`` is the weight's own shape (``N = shape[0]``, ``K`` the rest)."""
    q: torch.Tensor
    s: torch.Tensor
    shape: tuple

    @property
    def out_features(self) -> int:
        return int(self.shape[0])

    @property
    def in_features(self) -> int:
        return int(np.prod(self.shape[1:], dtype=np.int64)) if len(self.shape) > 1 else 1


def pack_int8_host(data, shape=None, rounding: str = "exact", threads: int = 0) -> HostInt8Weight:
    """Per-output-channel int8 of a host f32 weight (quantizeInt8PerChannel,
    borch-ts/src/quant.ts:23-53, ``shape[0]`` output channels) into pinned memory.

    ``rounding="exact"``: the library's rule, the bytes ``bq_quantize_weight_per_channel``
    writes on the device. ``"reference"``: the bytes of borch-ts's Linear packer
    (quant.ts:35-41: a double scale, ``Math.round(w * (1/scale))``), which differ on some
    near-ties. ``"reference_conv"``: its conv packer's rounding (quant.ts:88-96)."""
    if rounding not in _ROUNDING:
        raise ValueError(f"rounding must be one of {sorted(_ROUNDING)}, got {rounding!r}")
    w = data.detach().cpu().numpy() if isinstance(data, torch.Tensor) else np.asarray(data)
    w = np.ascontiguousarray(w, dtype=np.float32)
    shape = tuple(int(d) for d in (w.shape if shape is None else shape))
    count = int(np.prod(shape, dtype=np.int64))
    if w.size != count:
        raise ValueError(f"a weight of {w.size} values does not have the shape {list(shape)}")
    N = shape[0] if shape else 1
    K = count // N if N else 0
    kpad = _i8.round_up(max(K, 16), 16)
    pin = torch.cuda.is_available()
    q = torch.empty((N, kpad), dtype=torch.int8, pin_memory=pin)
    s = torch.empty((N,), dtype=torch.float32, pin_memory=pin)
    check(lib().bq_quantize_weight_host(w.ctypes.data, N, K, kpad, _ROUNDING[rounding], q.data_ptr(),
                                         s.data_ptr(), int(threads)))
    return HostInt8Weight(q, s, shape)


# ------------------------------------------------------------------ windowed weights

_LINEAR_FUNCS = {torch.nn.functional.linear}
_MATMUL_FUNCS = {torch.matmul, torch.Tensor.matmul, torch.Tensor.__matmul__, torch.mm, torch.Tensor.mm}
_CONV_FUNCS = {torch.nn.functional.conv2d}


class WindowedWeight:
    """A frozen weight whose bytes live in a window slot (a weight operand only).

    ``kind`` is "f32", "f16" or "int8". ``F.linear(x, w, b)``, ``x @ w`` / ``torch.matmul(x,
    w)`` and ``F.conv2d(x, w, ...)`` take it as the weight; each use checks the slot's
    generation first and raises the reference's "evicted" error once the slot was evicted
    (tensor.ts:1692-1699). Any other torch op on it raises: a windowed weight is not a
    general tensor (window_probe.html's "refuses a generic op")."""

    def __init__(self, slot: Slot, shape, kind: str, scales: torch.Tensor | None = None, kpad: int = 0):
        self.slot = slot
        self.shape = torch.Size(int(d) for d in shape)
        self.kind = kind
        self.scales = scales
        self.kpad = kpad
        self.requires_grad = False

    def __repr__(self):
        state = "live" if self.slot.live() else "evicted"
        return f"WindowedWeight({self.kind}, shape={list(self.shape)}, offset={self.slot.offset}, {state})"

    @property
    def device(self):
        return self.slot.window.device

    @property
    def out_features(self) -> int:
        return int(self.shape[0])

    @property
    def in_features(self) -> int:
        return int(np.prod(self.shape[1:], dtype=np.int64)) if len(self.shape) > 1 else 1

    def evict(self) -> None:
        self.slot.window.evict(self.slot)

    def _ready(self, stream=None) -> None:
        self.slot.check_live()
        st = stream if stream is not None else torch.cuda.current_stream(self.device)
        self.slot.ensure_ready(st)
        if self.scales is not None:
            self.scales.record_stream(st)

    def int8_weight(self) -> _i8.Int8Weight:
        """The slot as the weight-only packing the W8A32 kernel reads in place."""
        if self.kind != "int8":
            raise TypeError(f"a {self.kind} windowed weight has no int8 packing")
        self._ready()
        q = self.slot.view(torch.int8, (self.out_features, self.kpad))
        return _i8.Int8Weight(q, self.scales, self.in_features, self.out_features, weight_only=True)

    def tensor(self) -> torch.Tensor:
        """The weight's values as an f32 tensor of its shape: the slot itself (f32), its f16
        values widened, or the int8 values unpacked, f32(q) * s (bq_dequant_i8)."""
        self._ready()
        if self.kind == "f32":
            return self.slot.view(torch.float32, self.shape)
        if self.kind == "f16":
            return self.slot.view(torch.float16, self.shape).float()
        w = _i8.dequant_weight(self.int8_weight())
        return w[:, :self.in_features].reshape(self.shape)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = dict(kwargs or {})
        if func in _LINEAR_FUNCS:
            return _linear(*args, **kwargs)
        if func in _MATMUL_FUNCS and len(args) == 2 and not isinstance(args[0], WindowedWeight):
            return torch.matmul(args[0], args[1].tensor())
        if func in _CONV_FUNCS and len(args) >= 2 and not isinstance(args[0], WindowedWeight):
            a = list(args)
            a[1] = a[1].tensor()
            return func(*a, **kwargs)
        name = getattr(func, "__name__", str(func))
        raise RuntimeError(f"a windowed weight is a weight operand only (linear, matmul, conv2d): "
                           f"{name} cannot read the window")


def _linear(input, weight, bias=None):  # noqa: A002
    if not isinstance(weight, WindowedWeight) or isinstance(input, WindowedWeight) or isinstance(bias, WindowedWeight):
        raise RuntimeError("a windowed weight is a weight operand only: linear takes it as the weight")
    if weight.kind == "int8":
        return _i8.linear_w8a32(input, weight.int8_weight(), bias)
    return torch.nn.functional.linear(input, weight.tensor(), bias)


class Placed(NamedTuple):
    """``{weight, evict}`` of tensor.ts:1704: the windowed weight and its slot's eviction."""
    weight: WindowedWeight
    evict: Callable[[], None]


def _host_f32(data, shape):
    w = data.detach().cpu() if isinstance(data, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(data))
    w = w.contiguous()
    shape = tuple(int(d) for d in (w.shape if shape is None else shape))
    if w.numel() != int(np.prod(shape, dtype=np.int64)):
        raise ValueError(f"a weight of {w.numel()} values does not have the shape {list(shape)}")
    return w, shape


def in_window(win: Window, data, shape=None) -> Placed:
    """A frozen f32 weight placed in ``win`` (Tensor.inWindow, tensor.ts:1620-1650)."""
    w, shape = _host_f32(data, shape)
    slot = win.place(w.float())
    ww = WindowedWeight(slot, shape, "f32")
    return Placed(ww, ww.evict)


def in_window_f16(win: Window, data, shape=None) -> Placed:
    """A frozen weight placed as f16 (half the bytes, widened on use; Tensor.inWindowF16,
    tensor.ts:1652-1673). The values are the f16-rounded ones."""
    w, shape = _host_f32(data, shape)
    slot = win.place(w.float().half())
    ww = WindowedWeight(slot, shape, "f16")
    return Placed(ww, ww.evict)


def in_window_int8(win: Window, data, shape=None, rounding: str = "exact") -> Placed:
    """A frozen weight placed as per-output-channel int8 (Tensor.inWindowInt8,
    tensor.ts:1675-1705): quantized on the host (``shape[0]`` output channels; or already
    packed, a ``HostInt8Weight``), the int8 bytes copied into the slot (a quarter of the
    f32 bytes; K padded to a multiple of 16), the scales into a small resident tensor."""
    hw = data if isinstance(data, HostInt8Weight) else pack_int8_host(data, shape, rounding)
    if shape is not None and tuple(int(d) for d in shape) != tuple(hw.shape):
        raise ValueError(f"a packed weight of shape {list(hw.shape)} placed as {list(shape)}")
    slot = win.place(hw.q)
    with torch.cuda.stream(win.copy_stream):
        s = torch.empty(hw.s.shape, dtype=torch.float32, device=win.device)
        s.copy_(hw.s if hw.s.is_pinned() else hw.s.pin_memory(), non_blocking=True)
        evt = torch.cuda.Event()
        evt.record(win.copy_stream)
    slot.ready = evt  # recorded after both copies
    ww = WindowedWeight(slot, hw.shape, "int8", scales=s, kpad=int(hw.q.shape[1]))
    return Placed(ww, ww.evict)


# ------------------------------------------------------------------ the scheduler

@dataclass
class StreamBlock:
    """One block of a streamed stack (stream.ts:21-28): its frozen weights in the order
    ``run`` consumes them (host f32 arrays or tensors, or ``HostInt8Weight`` packings for
    ``int8=True``), their shapes, and the forward ``run(h, weights) -> h``."""
    weights: Sequence
    shapes: Sequence
    run: Callable


def _place_block(win: Window, blk: StreamBlock, int8: bool, f16: bool, rounding: str) -> list[Placed]:
    placed: list[Placed] = []
    try:
        for data, shape in zip(blk.weights, blk.shapes):
            if data is None or shape is None:
                continue
            if int8:
                placed.append(in_window_int8(win, data, shape, rounding))
            elif f16:
                placed.append(in_window_f16(win, data, shape))
            else:
                placed.append(in_window(win, data, shape))
    except BaseException:
        for p in placed:
            p.evict()
        raise
    return placed


def stream_sequential(win: Window, input, blocks: Sequence[StreamBlock], *, int8: bool = False,  # noqa: A002
                      f16: bool = False, rounding: str = "exact", prefetch: bool = True):
    """Runs ``blocks`` in order over ``input``, each block's weights placed in ``win`` just
    before it runs and evicted just after (stream.ts:36-68), as a no-grad forward.
    ``int8`` / ``f16`` store each weight quantized (a quarter / half of the window bytes;
    borch_webgpu/_stream.py:61-66). With ``prefetch`` block k+1 is placed while block k runs
    whenever the window holds both: its copies run on the window's copy stream under block
    k's kernels. The result is the same either way."""
    if int8 and f16:
        raise ValueError("int8 and f16 are two storage choices: pick one")
    blocks = list(blocks)
    h = input
    if not blocks:
        return h
    nxt = _place_block(win, blocks[0], int8, f16, rounding)
    with torch.no_grad():
        for i, blk in enumerate(blocks):
            cur, nxt = nxt, None
            try:
                if prefetch and i + 1 < len(blocks):
                    try:
                        nxt = _place_block(win, blocks[i + 1], int8, f16, rounding)
                    except WindowFull:
                        nxt = None  # no room for two blocks: place it after this one's eviction
                out = blk.run(h, [p.weight for p in cur])
            except BaseException:
                for p in nxt or []:
                    p.evict()
                raise
            finally:
                for p in cur:
                    p.evict()
            if nxt is None and i + 1 < len(blocks):
                nxt = _place_block(win, blocks[i + 1], int8, f16, rounding)
            h = out
    return h
