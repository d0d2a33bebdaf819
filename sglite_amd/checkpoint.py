"""AWQ checkpoint ingestion: tensor-parallel shard rules, fused-projection
merges and expert stacking for checkpoint streams.

Follows python/sglite/srt/model_executor/model_loader/weight_loader.py:
  shard rules        _shard_tensor (weight_loader.py:40-69)
  merge groups       _MERGE_GROUPS / _get_merge_info (:17-30, :72-77)
  expert stacking    _get_expert_stack_info (:80-89), load_weight (:121-142)
  dtype              floating tensors cast to the engine dtype, integer
                     (packed) tensors passed through (engine.py:168-174)

AWQ tensors keep the checkpoint layout here -- ``qweight`` int32
``[K, N/8]``, ``qzeros`` int32 ``[K/G, N/8]``, ``scales`` ``[K/G, N]`` -- so:
  * column-parallel projections (q/k/v, gate/up) shard along dim 1 (the packed
    output columns; N/8 words hold 8 columns each, so a chunk of words is a
    chunk of columns);
  * row-parallel projections (o, down) shard along dim 0 (input rows, and the
    group rows of qzeros/scales);
  * fused projections concatenate their parts along dim 1 in slot order
    (q, k, v) and (gate, up);
  * expert tensors ``<prefix>.experts.<i>.<name>`` are stacked on dim 0 into
    ``<prefix>.<name>`` once all experts have arrived.
The repack into the CDNA4 tile layout happens afterwards, per layer, in the
linear method's post-load step (or ``moe.process_awq_moe_weights`` for expert
stacks).
"""

from __future__ import annotations

import glob
import os
import re
from typing import Dict, Iterable, Iterator, Optional, Tuple

import torch

_SPLIT_DIM_0 = (".q_proj", ".k_proj", ".v_proj", ".gate_proj", ".up_proj")
_SPLIT_DIM_1 = (".o_proj", ".down_proj")

MERGE_GROUPS = {
    ".q_proj": (".qkv_proj", ("q", "k", "v")),
    ".k_proj": (".qkv_proj", ("q", "k", "v")),
    ".v_proj": (".qkv_proj", ("q", "k", "v")),
    ".gate_proj": (".gate_up_proj", ("gate", "up")),
    ".up_proj": (".gate_up_proj", ("gate", "up")),
}
_SLOT_NAMES = {".q_proj": "q", ".k_proj": "k", ".v_proj": "v", ".gate_proj": "gate", ".up_proj": "up"}
_EXPERT_PATTERN = re.compile(r"^(?P<prefix>.+\.experts)\.(?P<idx>\d+)\.(?P<name>.+)$")
AWQ_SUFFIXES = (".qweight", ".qzeros", ".scales")


def is_awq_tensor(key: str) -> bool:
    """Whether a checkpoint key names AWQ-packed storage (weight_loader.py:35-37)."""
    return key.endswith(AWQ_SUFFIXES)


def shard_tensor(key: str, value: torch.Tensor, rank: int, world: int,
                 num_kv_heads: Optional[int] = None) -> torch.Tensor:
    """Rank ``rank``'s shard of one checkpoint tensor (weight_loader.py:40-69)."""
    awq = is_awq_tensor(key)
    if any(s in key for s in _SPLIT_DIM_0):
        if awq:  # packed output columns live on dim 1
            return value.chunk(world, dim=1)[rank].clone()
        is_kv = any(s in key for s in (".k_proj", ".v_proj"))
        if is_kv and num_kv_heads is not None and num_kv_heads < world:
            head_dim = value.shape[0] // num_kv_heads
            head = rank * num_kv_heads // world
            return value[head * head_dim:(head + 1) * head_dim].clone()
        return value.chunk(world, dim=0)[rank].clone()
    if any(s in key for s in _SPLIT_DIM_1):
        if awq:  # input rows (and group rows) live on dim 0
            return value.chunk(world, dim=0)[rank].clone()
        return value.chunk(world, dim=1)[rank].clone()
    if "lm_head" in key or "embed_tokens" in key:
        per = -(-value.shape[0] // world)
        return value[rank * per:min((rank + 1) * per, value.shape[0]), :].clone()
    return value


def merge_info(key: str) -> Optional[Tuple[str, str, Tuple[str, ...]]]:
    """(fused key, slot, slots in order) for a projection that is fused at run time."""
    for suffix, (fused, slots) in MERGE_GROUPS.items():
        if suffix in key:
            return key.replace(suffix, fused), _SLOT_NAMES[suffix], slots
    return None


def expert_stack_info(key: str) -> Optional[Tuple[str, int]]:
    """(stacked key, expert index) for ``<prefix>.experts.<i>.<name>`` keys."""
    m = _EXPERT_PATTERN.match(key)
    if m is None:
        return None
    name = m.group("name")
    if name.endswith(".weight"):
        name = name[: -len(".weight")]
    return f"{m.group('prefix')}.{name}", int(m.group("idx"))


def ingest(tensors: Iterable[Tuple[str, torch.Tensor]], rank: int = 0, world: int = 1,
           num_kv_heads: Optional[int] = None, num_experts: Optional[int] = None,
           dtype: Optional[torch.dtype] = None) -> Iterator[Tuple[str, torch.Tensor]]:
    """Shard, merge and stack a stream of checkpoint tensors (load_weight,
    weight_loader.py:92-145).  Merged tensors are yielded once every slot has
    arrived; with ``num_experts`` set, expert tensors are yielded stacked once
    all experts have arrived.  Floating tensors are cast to ``dtype``.
    Raises ValueError if the stream ends with an incomplete merge or stack."""
    merge_buf: Dict[str, Dict[str, torch.Tensor]] = {}
    expert_buf: Dict[str, Dict[int, torch.Tensor]] = {}
    for name, raw in tensors:
        if name.startswith(("vision_tower.", "multi_modal_projector.")):
            continue
        name = name[len("language_model."):] if name.startswith("language_model.") else name
        t = shard_tensor(name, raw, rank, world, num_kv_heads)
        info = merge_info(name)
        if info is None:
            out = (name, t)
        else:
            fused, slot, slots = info
            buf = merge_buf.setdefault(fused, {})
            if slot in buf:
                raise ValueError(f"duplicate {slot} part for {fused}")
            buf[slot] = t
            if not all(s in buf for s in slots):
                continue
            parts = [buf[s] for s in slots]
            del merge_buf[fused]
            out = (fused, torch.cat(parts, dim=1 if is_awq_tensor(fused) else 0))
        if dtype is not None and out[1].is_floating_point():
            out = (out[0], out[1].to(dtype))
        if num_experts is not None and (ex := expert_stack_info(out[0])) is not None:
            key, idx = ex
            slots_e = expert_buf.setdefault(key, {})
            slots_e[idx] = out[1]
            if len(slots_e) != num_experts:
                continue
            del expert_buf[key]
            yield key, torch.stack([slots_e[i] for i in range(num_experts)], dim=0)
        else:
            yield out
    if merge_buf:
        raise ValueError(f"incomplete merge groups in checkpoint: {sorted(merge_buf)}")
    if expert_buf:
        raise ValueError(f"incomplete expert tensors in checkpoint: {sorted(expert_buf)}")


def iter_safetensors(model_dir: str, device: str = "cpu") -> Iterator[Tuple[str, torch.Tensor]]:
    """(name, tensor) pairs of every ``*.safetensors`` file in a directory (the
    file selection of weight_loader.py:104-105), read with safetensors only."""
    import safetensors

    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    files = [f for f in files if not f.endswith("consolidated.safetensors")] or files
    for path in files:
        with safetensors.safe_open(path, framework="pt", device=device) as f:
            for name in f.keys():
                yield name, f.get_tensor(name)
