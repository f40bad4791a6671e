"""Host offload of what a packed-attention layer keeps for its backward.

The interface is the one the reference's PackedAttention calls (solution/offload.py:71-73, 86-95,
153-170; used at solution/attention.py:266-274 and 283):

    OFFLOADER.begin(device) / OFFLOADER.end()   bracket a forward pass (the caller does this)
    OFFLOADER.wants(*tensors)  -> bool           should these tensors be offloaded?
    OFFLOADER.save(*tensors)   -> handle         hand them over (they may leave the GPU)
    OFFLOADER.load(handle)     -> tensors        get them back on the GPU, bit for bit

How this one works. Saved layers form a queue in forward order. While the saved bytes still on
the GPU exceed KEEP_BYTES, the oldest layer (never the newest: the backward needs that one first)
is copied to pinned host memory on a side stream that first waits for the compute stream's work
so far. The device tensors are marked as in use by the side stream (`record_stream`), so the
caching allocator does not reuse their memory before the copy has read them; the compute stream
never waits for an eviction. `load` brings a layer back on the side stream into memory allocated
there, marks it as used by the compute stream, and makes only the compute stream wait for that
copy. Because the backward visits the layers in reverse, each load also starts bringing back the
previous evicted layer, so its copy overlaps the current layer's backward. All streams have the
default priority. Pinned buffers are released through torch's caching host allocator, which holds
a block until the copies queued on it have finished.
"""

import torch

KEEP_BYTES = 1 << 30  # saved bytes allowed to stay on the GPU at the end of a forward pass


class _Layer:
    """One save() call: where its tensors are (device list, host list, or a copy on its way back)
    and the events that order the copies."""

    __slots__ = ("index", "peers", "on_device", "on_host", "returning", "nbytes", "host_ready",
                 "device_ready")

    def __init__(self, index, peers, tensors):
        self.index = index
        self.peers = peers  # the layers saved in the same forward pass, in order
        self.on_device = list(tensors)
        self.on_host = None
        self.returning = None
        self.nbytes = sum(t.numel() * t.element_size() for t in tensors)
        self.host_ready = None
        self.device_ready = None


class Offloader:
    def __init__(self):
        self._active = False
        self._layers = []
        self._oldest_on_device = 0
        self._device_bytes = 0
        self._side = None

    def begin(self, device):
        device = torch.device(device)
        if self._side is None or self._side.device != device:
            self._side = torch.cuda.Stream(device=device)
        self._layers, self._oldest_on_device, self._device_bytes = [], 0, 0
        self._active = True

    def end(self):
        self._active = False

    def wants(self, *tensors):
        return self._active and torch.is_grad_enabled() and all(t.is_cuda for t in tensors)

    def save(self, *tensors):
        layer = _Layer(len(self._layers), self._layers, tensors)
        self._layers.append(layer)
        self._device_bytes += layer.nbytes
        while (self._device_bytes > KEEP_BYTES
               and self._oldest_on_device < len(self._layers) - 1):
            self._evict(self._layers[self._oldest_on_device])
            self._oldest_on_device += 1
        return layer

    def _evict(self, layer):
        compute = torch.cuda.current_stream(self._side.device)
        self._side.wait_stream(compute)
        with torch.cuda.stream(self._side):
            host = []
            for t in layer.on_device:
                h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
                h.copy_(t, non_blocking=True)
                t.record_stream(self._side)
                host.append(h)
            layer.host_ready = self._side.record_event()
        layer.on_host, layer.on_device = host, None
        self._device_bytes -= layer.nbytes

    def _bring_back(self, layer):
        """Queue the host-to-device copy of an evicted layer on the side stream."""
        compute = torch.cuda.current_stream(self._side.device)
        with torch.cuda.stream(self._side):
            self._side.wait_event(layer.host_ready)
            back = []
            for h in layer.on_host:
                d = torch.empty(h.shape, dtype=h.dtype, device=self._side.device)
                d.copy_(h, non_blocking=True)
                d.record_stream(compute)
                back.append(d)
            layer.device_ready = self._side.record_event()
        layer.returning = back

    def load(self, layer):
        if layer.on_device is not None:  # never left the GPU
            tensors, layer.on_device = layer.on_device, None
            return tensors
        if layer.returning is None:
            self._bring_back(layer)
        torch.cuda.current_stream(self._side.device).wait_event(layer.device_ready)
        tensors, layer.returning, layer.on_host = layer.returning, None, None
        # the backward runs in reverse: start bringing back the layer saved before this one
        if layer.index > 0:
            earlier = layer.peers[layer.index - 1]
            if earlier.on_host is not None and earlier.returning is None:
                self._bring_back(earlier)
        return tensors


OFFLOADER = Offloader()
