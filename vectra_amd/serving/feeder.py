"""Host-to-device staging that keeps the GPU busy between batches.

The reference gateway hands each batch to the model as pageable host
tensors (serving/predict.py:236-249 into compile_entry.ServingModel.predict,
models/export/compile_entry.py:301-316), so every batch's copy to the GPU,
the model and the copy of the result back run one after another.  At the
serving batch (1024 subjects x 64 comparables) the inputs are ~38 MB, which
crosses PCIe in about as long as the compiled model takes to run, so that
order leaves the GPU idle for half of every cycle.

`DeviceFeeder` gives every batch in flight a slot: one pinned host buffer
holding every input field of the compiled batch shape (filled in place) and
one device buffer with the same layout, so a batch crosses PCIe as a single
copy.  `launch` enqueues that copy on a copy stream, the model on the
compute stream once the copy has landed, and the copy of the [B] result
into pinned memory; it returns without waiting.  `finish` waits for one
slot's result.  With two slots the copy of batch n + 1 overlaps the model
on batch n.  With `graph=True` each slot's model call is captured once as a
HIP graph on that slot's buffers, so a launch costs one graph replay on the
host instead of one launch per kernel.  A short batch is padded with copies
of its last request (the compiled shape is static) and the padding rows are
dropped from the result, as ServingModel.predict does.  Streams keep the
default priority.
"""

import dataclasses

import torch

from vectra_amd.price_transformer import model as model_lib


# Field offsets inside a slot's buffers are multiples of this (bytes).
_ALIGN = 256


def _layout(example) -> tuple[list[tuple[int, torch.dtype, tuple]], int]:
    """(offset, dtype, shape) of every field in one contiguous buffer, and its size."""
    fields, offset = [], 0
    for t in example:
        offset = -(-offset // _ALIGN) * _ALIGN
        fields.append((offset, t.dtype, tuple(t.shape)))
        offset += t.numel() * t.element_size()
    return fields, -(-offset // _ALIGN) * _ALIGN


def _views(buffer: torch.Tensor, fields) -> model_lib.PricingInputs:
    """Typed views of a uint8 buffer, one per field."""
    out = []
    for offset, dtype, shape in fields:
        size = torch.Size(shape).numel() * torch.empty((), dtype=dtype).element_size()
        out.append(buffer[offset:offset + size].view(dtype).view(shape))
    return model_lib.PricingInputs(*out)


@dataclasses.dataclass
class _Slot:
    host_bytes: torch.Tensor  # pinned uint8, every field
    device_bytes: torch.Tensor  # uint8 on the GPU, same layout
    host: model_lib.PricingInputs  # views of host_bytes, [B, ...]
    device: model_lib.PricingInputs  # views of device_bytes
    result: torch.Tensor  # pinned fp32 [B]
    copied: torch.cuda.Event  # host-to-device copy done (copy stream)
    consumed: torch.cuda.Event  # the model no longer needs `device` (compute stream)
    done: torch.cuda.Event  # result in pinned memory (compute stream)
    graph: torch.cuda.CUDAGraph | None = None
    graph_out: torch.Tensor | None = None  # the captured call's fp32 output
    rows: int = 0
    in_flight: bool = False


@dataclasses.dataclass(frozen=True)
class Handle:
    """A launched batch: its slot and its number of real rows."""

    slot: int
    rows: int


class DeviceFeeder:
    """Pinned, multi-slot staging of PricingInputs for a compiled model.

    Args:
      model: the compiled model, called as model(*inputs) on device tensors
        of the batch shape; returns [B] predictions.
      example: a PricingInputs batch (any device) giving every field's
        shape (leading dimension = the compiled batch size) and dtype.
      device: the GPU.
      slots: batches in flight (2: the copy of the next batch overlaps the
        model on the current one).
      graph: capture each slot's model call as a HIP graph (the model must
        be capturable: no host synchronisation inside).
    """

    def __init__(self, model, example: model_lib.PricingInputs, device='cuda', slots: int = 2,
                 graph: bool = False):
        if slots < 1:
            raise ValueError('need at least one slot')
        self.device = torch.device(device)
        if self.device.type != 'cuda':
            raise ValueError('DeviceFeeder stages batches for a GPU')
        self.batch_size = int(example[0].shape[0])
        self._model = model
        self._compute = torch.cuda.current_stream(self.device)
        self._copy = torch.cuda.Stream(self.device)
        fields, size = _layout(example)
        self.bytes_per_batch = size
        self._slots = []
        for _ in range(slots):
            host_bytes = torch.empty(size, dtype=torch.uint8, pin_memory=True)
            device_bytes = torch.empty(size, dtype=torch.uint8, device=self.device)
            consumed = torch.cuda.Event()
            consumed.record(self._compute)  # the device buffers start free
            self._slots.append(_Slot(host_bytes, device_bytes, _views(host_bytes, fields),
                                     _views(device_bytes, fields),
                                     torch.empty(self.batch_size, dtype=torch.float32, pin_memory=True),
                                     torch.cuda.Event(), consumed, torch.cuda.Event()))
        if graph:
            self._capture(example)
        self._next = 0

    def _capture(self, example) -> None:
        """Captures the model call of every slot as a HIP graph on the
        slot's device buffers (warmed up eagerly first, on a side stream)."""
        for s in self._slots:
            for dst, src in zip(s.device, example):
                dst.copy_(src)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(self._compute)
        with torch.cuda.stream(side), torch.no_grad():
            for s in self._slots:
                for _ in range(2):
                    self._model(*s.device)
        self._compute.wait_stream(side)
        torch.cuda.synchronize(self.device)
        for s in self._slots:  # a memory pool per graph: nothing shared between slots
            s.graph = torch.cuda.CUDAGraph()
            with torch.no_grad(), torch.cuda.graph(s.graph):
                s.graph_out = self._model(*s.device).float()
        torch.cuda.synchronize(self.device)

    @property
    def slots(self) -> int:
        return len(self._slots)

    def next_slot(self) -> tuple[int, model_lib.PricingInputs]:
        """The slot the next launch uses and its pinned host buffers [B, ...],
        to be filled in place (rows 0 .. n - 1) before `launch(slot, n)`.

        Raises RuntimeError if that slot's previous batch was not finished.
        """
        slot = self._slots[self._next]
        if slot.in_flight:
            raise RuntimeError(f'slot {self._next} is still in flight: finish() its batch first')
        return self._next, slot.host

    def stage(self, batch: model_lib.PricingInputs) -> tuple[int, int]:
        """Copies a host batch of n <= B rows into the next slot's pinned
        buffers; returns (slot, n) for `launch`."""
        index, host = self.next_slot()
        rows = int(batch[0].shape[0])
        if not 1 <= rows <= self.batch_size:
            raise ValueError(f'a batch holds 1 .. {self.batch_size} requests, not {rows}')
        for dst, src in zip(host, batch):
            dst[:rows].copy_(src)
        return index, rows

    def launch(self, slot: int, rows: int) -> Handle:
        """Enqueues slot `slot` (rows 0 .. rows - 1 filled): pads it to the
        compiled batch, copies it to the GPU, runs the model and copies the
        result back.  Returns without waiting."""
        if slot != self._next:
            raise ValueError(f'slots are launched in order: expected {self._next}, got {slot}')
        s = self._slots[slot]
        if s.in_flight:
            raise RuntimeError(f'slot {slot} is still in flight')
        if not 1 <= rows <= self.batch_size:
            raise ValueError(f'a batch holds 1 .. {self.batch_size} requests, not {rows}')
        if rows < self.batch_size:
            for t in s.host:
                t[rows:].copy_(t[rows - 1:rows].expand(self.batch_size - rows, *t.shape[1:]))
        with torch.cuda.stream(self._copy):
            # The device buffer is rewritten only after the model's last read
            # of it from this slot's previous batch.
            self._copy.wait_event(s.consumed)
            s.device_bytes.copy_(s.host_bytes, non_blocking=True)
            s.copied.record(self._copy)
        with torch.cuda.stream(self._compute):
            self._compute.wait_event(s.copied)
            if s.graph is not None:
                s.graph.replay()
                out = s.graph_out
            else:
                with torch.no_grad():
                    out = self._model(*s.device).float()
            s.consumed.record(self._compute)
            s.result.copy_(out, non_blocking=True)
            s.done.record(self._compute)
        s.rows, s.in_flight = rows, True
        self._next = (self._next + 1) % len(self._slots)
        return Handle(slot, rows)

    def finish(self, handle: Handle) -> torch.Tensor:
        """Waits for a launched batch; returns its [rows] fp32 predictions
        (a host tensor of its own)."""
        s = self._slots[handle.slot]
        if not s.in_flight:
            raise RuntimeError(f'slot {handle.slot} has no batch in flight')
        s.done.synchronize()
        s.in_flight = False
        return s.result[:handle.rows].clone()

    def run(self, batch: model_lib.PricingInputs) -> torch.Tensor:
        """One batch, staged, launched and finished."""
        return self.finish(self.launch(*self.stage(batch)))
