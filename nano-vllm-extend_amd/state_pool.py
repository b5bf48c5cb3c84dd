"""Slot bookkeeping for the GDN recurrent / conv state pools.

Restates the reference's pool contract (the layout the HIP kernels index):
  * LinearStatePool -- CPU free list of slot ids
    (nanovllm/engine/linear_state_pool.py:12-27);
  * allocate_state_pools -- s_pool [slots+1, L, H, K, V] fp32 and
    conv_pool [slots+1, L, conv_dim, K-1] bf16 with one dummy slot for
    graph pad rows, per-layer views [:, l]
    (nanovllm/engine/model_runner.py:265-303);
  * reset_linear_states -- fresh-prefill zeroing of a slot
    (model_runner.py:305-322);
  * varlen_meta -- per-step cu_seqlens / lens tensors shared by the layers
    of a step (nanovllm/models/qwen3_5.py:486-502).
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass

import torch


class LinearStatePool:
    """CPU free list of state slots.  Slots are assigned on first scheduling
    and freed when a sequence finishes; a preempted sequence keeps its slot
    and is re-prefilled with the slot zeroed."""

    def __init__(self, num_slots: int):
        self.num_slots = num_slots
        self.free_slots: deque[int] = deque(range(num_slots))

    def alloc(self) -> int:
        assert self.free_slots, "no free linear-state slots"
        return self.free_slots.popleft()

    def free(self, slot: int) -> None:
        self.free_slots.append(slot)

    @property
    def num_free(self) -> int:
        return len(self.free_slots)


@dataclass
class StatePools:
    s_pool: torch.Tensor       # [slots + 1, L, H, K, V] fp32
    conv_pool: torch.Tensor    # [slots + 1, L, conv_dim, K - 1] bf16
    num_slots: int

    @property
    def dummy_slot(self) -> int:
        """Graph pad rows point here so in-place updates never touch a live slot."""
        return self.num_slots

    def layer(self, l: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-layer views (s_cache [slots+1, H, K, V], conv_cache [slots+1, conv_dim, K-1])."""
        return self.s_pool[:, l], self.conv_pool[:, l]


def slot_bytes(L: int, H: int, K: int, V: int, conv_dim: int, conv_states: int) -> int:
    """Bytes per slot across the GDN layers (fp32 state + bf16 conv state)."""
    return L * (H * K * V * 4 + conv_dim * conv_states * 2)


def allocate_state_pools(num_slots: int, L: int, H: int, K: int, V: int, conv_dim: int,
                         conv_kernel: int, device, conv_dtype=torch.bfloat16) -> StatePools:
    s_pool = torch.zeros(num_slots + 1, L, H, K, V, dtype=torch.float32, device=device)
    conv_pool = torch.zeros(num_slots + 1, L, conv_dim, conv_kernel - 1, dtype=conv_dtype, device=device)
    return StatePools(s_pool, conv_pool, num_slots)


def reset_linear_states(pools: StatePools, slot_ids: torch.Tensor) -> None:
    """Zero the recurrent and conv state of fresh-prefill slots."""
    pools.s_pool[slot_ids] = 0
    pools.conv_pool[slot_ids] = 0


_VARLEN_META: tuple | None = None


def varlen_meta(lens_q: list[int], device):
    """(cu int32 [n+1], lens int32 [n], cu64 host [n+1], cu64 device [n+1]),
    built once per distinct length tuple and reused by every GDN layer of
    the step."""
    global _VARLEN_META
    key = (tuple(lens_q), str(device))
    if _VARLEN_META is not None and _VARLEN_META[0] == key:
        return _VARLEN_META[1]
    cu = [0]
    for l in lens_q:
        cu.append(cu[-1] + l)
    pin = torch.device(device).type == "cuda"
    cu_cpu = torch.tensor(cu, dtype=torch.int32, pin_memory=pin)
    lens_cpu = torch.tensor(lens_q, dtype=torch.int32, pin_memory=pin)
    cu64_cpu = cu_cpu.to(torch.int64)
    meta = (cu_cpu.to(device, non_blocking=True), lens_cpu.to(device, non_blocking=True), cu64_cpu,
            cu64_cpu.to(device, non_blocking=True))
    _VARLEN_META = (key, meta)
    return meta
