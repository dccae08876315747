"""Composite KV-cache layout: backing tensors on the device, composite
pages on the host.

Mirrors aegaeon/vllm_cache.py:28-154 without vLLM. Each backing tensor is a
*segment*: on the device it is viewed as [num_blocks, page_size_bytes]; on
the host every block id owns one composite page in which segment s occupies
[cpu_offset_s, cpu_offset_s + page_size_bytes_s), segments packed in order
(vllm_cache.py:75-101). With tensor parallelism the host page is tp_size
composite pages and rank r writes the r-th (aegaeon/worker.py:1419-1432,
2304-2309).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Sequence, Tuple

import torch


@dataclass(frozen=True)
class CacheSegment:
    """One backing tensor's bytes inside a composite block (vllm_cache.py:28-41)."""

    layer_name: str
    shared_by: Tuple[str, ...]
    cpu_offset: int
    page_size_bytes: int


@dataclass(frozen=True)
class KVCacheTensorSpec:
    """The fields of vLLM's KVCacheTensor that the layout reads: total bytes,
    the layers bound to the tensor, and vLLM's packed-layout stride."""

    size: int
    shared_by: Tuple[str, ...]
    block_stride: int = 0


def make_composite_layout(tensor_specs: Sequence[KVCacheTensorSpec], num_blocks: int
                          ) -> Tuple[List[CacheSegment], int]:
    """Segments in tensor order and the composite page size
    (vllm_cache.py:75-101, including its three rejections)."""
    if num_blocks <= 0:
        raise MemoryError(f"a cache of {num_blocks} blocks holds no block")
    segments: List[CacheSegment] = []
    offset = 0
    for spec in tensor_specs:
        if spec.block_stride > 0:
            raise NotImplementedError(
                "a backing tensor with a block stride (packed K/V) has no per-block page "
                "for the swaps"
            )
        if spec.size % num_blocks:
            raise ValueError(
                f"a {spec.size}-byte backing tensor does not split into {num_blocks} "
                "equal block pages"
            )
        if not spec.shared_by:
            raise ValueError("a backing tensor with no layer names")
        page = spec.size // num_blocks
        segments.append(CacheSegment(spec.shared_by[0], tuple(spec.shared_by), offset, page))
        offset += page
    return segments, offset


def kv_tensor_specs(num_layers: int, num_blocks: int, block_size: int, kv_heads: int,
                    head_dim: int, dtype_bytes: int) -> List[KVCacheTensorSpec]:
    """One K and one V tensor [num_blocks, block_size, kv_heads, head_dim] per
    layer, in order layer0.K, layer0.V, layer1.K, ... ."""
    size = num_blocks * block_size * kv_heads * head_dim * dtype_bytes
    specs = []
    for layer in range(num_layers):
        for kv in ("k", "v"):
            specs.append(KVCacheTensorSpec(size, (f"layers.{layer}.{kv}",)))
    return specs


@dataclass
class CompositeCache:
    """Device backing tensors plus their composite layout (vllm_cache.py:43-51)."""

    segments: List[CacheSegment]
    raw_tensors: Dict[str, torch.Tensor]
    page_size_bytes: int
    num_blocks: int
    backing: List[torch.Tensor] = field(default_factory=list)

    def segment_tensor(self, index: int) -> torch.Tensor:
        return self.raw_tensors[self.segments[index].layer_name]

    def segment_pages(self, index: int) -> torch.Tensor:
        """Segment `index` as uint8 [num_blocks, page] (worker.py:2273-2277)."""
        seg = self.segments[index]
        return self.segment_tensor(index).view(torch.uint8).view(
            self.num_blocks, seg.page_size_bytes)


def allocate_composite_cache(tensor_specs: Sequence[KVCacheTensorSpec], num_blocks: int,
                             device: torch.device | str, zero: bool = True) -> CompositeCache:
    """Allocate one int8 backing tensor per spec and alias its layers
    (vllm_cache.py:104-154). zero=True matches the reference's zero-fill."""
    segments, page = make_composite_layout(tensor_specs, num_blocks)
    raw: Dict[str, torch.Tensor] = {}
    backing = []
    for spec in tensor_specs:
        t = torch.empty((spec.size,), dtype=torch.int8, device=device)
        if zero:
            t.zero_()
        backing.append(t)
        for name in spec.shared_by:
            raw[name] = t
    if torch.device(device).type == "cuda":
        torch.cuda.current_stream(torch.device(device)).synchronize()
    return CompositeCache(segments, raw, page, num_blocks, backing)


def wrap_composite_cache(tensor_specs: Sequence[KVCacheTensorSpec], num_blocks: int,
                         backing: Sequence[torch.Tensor]) -> CompositeCache:
    """A CompositeCache over backing tensors that already exist, one per
    spec in spec order: another process's cache opened through HIP IPC
    memory handles (what the reference's worker exports for migration,
    worker.py:2439-2445), or tensors allocated elsewhere. Sizes are checked;
    nothing is copied or zeroed."""
    if len(backing) != len(tensor_specs):
        raise ValueError(f"{len(backing)} backing tensors for {len(tensor_specs)} specs")
    segments, page = make_composite_layout(tensor_specs, num_blocks)
    raw: Dict[str, torch.Tensor] = {}
    for spec, t in zip(tensor_specs, backing):
        if t.numel() * t.element_size() < spec.size:
            raise ValueError(f"backing tensor of {t.numel() * t.element_size()} bytes is "
                             f"smaller than its spec ({spec.size})")
        for name in spec.shared_by:
            raw[name] = t
    return CompositeCache(segments, raw, page, num_blocks, list(backing))


def host_page_geometry(composite_page_bytes: int, tp_size: int, element_size: int = 2
                       ) -> int:
    """Host bytes per block id: one composite page per TP rank
    (worker.py:1419-1426, which also requires element alignment)."""
    total = composite_page_bytes * tp_size
    if total % element_size:
        raise ValueError(
            f"a {total}-byte host page is not a whole number of {element_size}-byte "
            "host elements"
        )
    return total
