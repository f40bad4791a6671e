"""Offload of the tensors a packed-attention layer keeps for its backward to pinned host memory.

Keeps the contract the reference's PackedAttention relies on (solution/offload.py:71-73, 86-95,
153-170; used at solution/attention.py:266-274 and 283):

    OFFLOADER.begin(device) / OFFLOADER.end()   bracket a forward pass (the caller does this)
    OFFLOADER.wants(*tensors)  -> bool           offload these tensors?
    OFFLOADER.save(*tensors)   -> item           start their device-to-host copy
    OFFLOADER.load(item)       -> tensors        bring them back (bit for bit) on the device

Design for a 288 GB device: the newest `keep_bytes` of saved tensors stay on the GPU (the
backward needs them first); older items are copied to pinned host memory on a side stream at the
default priority, and the compute stream waits for a copy before the GPU memory is released. In
the backward, `load` copies an item back on the side stream and makes the compute stream wait for
that copy only. Outside begin()/end() nothing is offloaded.
"""

import torch

KEEP_BYTES = 1 << 30  # newest bytes left on the GPU at the end of the forward


class _Item:
    __slots__ = ("tensors", "host", "nbytes", "copied")

    def __init__(self, tensors):
        self.tensors = tensors
        self.host = None
        self.copied = None
        self.nbytes = sum(t.numel() * t.element_size() for t in tensors)


class Offloader:
    def __init__(self):
        self.active = False
        self.items = []
        self.stream = None
        self.resident = 0
        self.evict_next = 0

    def begin(self, device):
        self.items, self.resident, self.evict_next = [], 0, 0
        if self.stream is None or self.stream.device != torch.device(device):
            self.stream = torch.cuda.Stream(device=device)  # default priority
        self.active = True

    def end(self):
        self.active = False

    def wants(self, *tensors):
        return self.active and torch.is_grad_enabled() and all(t.is_cuda for t in tensors)

    def save(self, *tensors):
        item = _Item(tensors)
        self.items.append(item)
        self.resident += item.nbytes
        while self.resident > KEEP_BYTES and self.evict_next < len(self.items) - 1:
            old = self.items[self.evict_next]
            self.evict_next += 1
            self.resident -= old.nbytes
            self._to_host(old)
        return item

    def _to_host(self, item):
        compute = torch.cuda.current_stream()
        produced = compute.record_event()
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(produced)
            item.host = []
            for t in item.tensors:
                buf = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
                buf.copy_(t, non_blocking=True)
                item.host.append(buf)
            done = self.stream.record_event()
        compute.wait_event(done)  # the GPU copy is freed in compute-stream order after this
        item.tensors = None

    def load(self, item):
        if item.tensors is not None:
            tensors, item.tensors = item.tensors, None
            return tensors
        compute = torch.cuda.current_stream()
        restored = [torch.empty(h.shape, dtype=h.dtype, device=compute.device) for h in item.host]
        free = compute.record_event()
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(free)
            for gpu, host in zip(restored, item.host):
                gpu.copy_(host, non_blocking=True)
            ready = self.stream.record_event()
        compute.wait_event(ready)
        item.host = None
        return restored


OFFLOADER = Offloader()
