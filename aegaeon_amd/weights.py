"""Weight loads of a model switch.

The reference keeps each cached model's weights in pinned host memory, one
storage per tensors content of each sharding content
(QuickLoader.model_contents, aegaeon/loader/quick_loader.py:297-323), and on
a switch copies every content into a device slice of its arena with one
`slice_storage.copy_(tensors_content.tensors_storage, non_blocking=True)`
each (:325-340), inside Worker.switch (aegaeon/worker.py:455-551), over the
same host link the KV swaps use. Here a model's contents share one pinned
pool (HostWeights) and a switch loads all of them with one aegkv_load_slices
call (ops.load_slices).
"""

from __future__ import annotations

from typing import List, Sequence

import torch

from . import ops

_ALIGN = 256


def _aligned(n: int) -> int:
    return -(-n // _ALIGN) * _ALIGN


class HostWeights:
    """A model's weight contents in one pinned host pool, each content at a
    256-byte aligned offset (`slices`, uint8 views)."""

    def __init__(self, content_bytes: Sequence[int], uncached: bool = False):
        if not content_bytes or any(b <= 0 for b in content_bytes):
            raise ValueError("content sizes must be positive")
        self.content_bytes = [int(b) for b in content_bytes]
        self.offsets = []
        off = 0
        for b in self.content_bytes:
            self.offsets.append(off)
            off += _aligned(b)
        self.pool = ops.PinnedHostPool(off, uncached=uncached)
        self.slices: List[torch.Tensor] = [
            self.pool.tensor.narrow(0, o, b) for o, b in zip(self.offsets, self.content_bytes)]

    @property
    def total_bytes(self) -> int:
        return sum(self.content_bytes)

    def free(self) -> None:
        self.slices = []
        self.pool.free()


class DeviceWeights:
    """The device arena slices a model's contents load into, one per
    content, 256-byte aligned inside one allocation."""

    def __init__(self, content_bytes: Sequence[int], device: torch.device):
        self.content_bytes = [int(b) for b in content_bytes]
        total = sum(_aligned(b) for b in self.content_bytes)
        self.arena = torch.empty(total, dtype=torch.uint8, device=device)
        self.slices: List[torch.Tensor] = []
        off = 0
        for b in self.content_bytes:
            self.slices.append(self.arena.narrow(0, off, b))
            off += _aligned(b)


def load_model(target: DeviceWeights, source: HostWeights, *, mode="auto",
               stream: torch.cuda.Stream | None = None) -> None:
    """Load every content of `source` into `target` (same content sizes) in
    one call (load_model_to_tensors' loop of per-content copies,
    quick_loader.py:297-340)."""
    if target.content_bytes != source.content_bytes:
        raise ValueError("device and host weights differ in their content sizes")
    ops.load_slices(target.slices, source.slices, mode=mode, stream=stream)


def qwen2_content_bytes(layers: int = 28, hidden: int = 3584, intermediate: int = 18944,
                        kv_dim: int = 512, vocab: int = 152064, dtype_bytes: int = 2
                        ) -> List[int]:
    """Per-content byte sizes of a Qwen2-style decoder (the default is
    Qwen2.5-7B: 7.6 B parameters, bf16): the embedding, one content per
    layer (attention q/k/v/o with biases, the MLP, two norms) and the
    output head."""
    per_layer = (hidden * hidden + 2 * kv_dim * hidden + hidden * hidden   # q, k, v, o
                 + hidden + 2 * kv_dim                                     # q/k/v biases
                 + 3 * hidden * intermediate                                # gate, up, down
                 + 2 * hidden)                                              # two RMS norms
    embed = vocab * hidden
    return ([embed * dtype_bytes] + [per_layer * dtype_bytes] * layers
            + [(embed + hidden) * dtype_bytes])
