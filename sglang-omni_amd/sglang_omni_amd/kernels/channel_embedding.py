"""MOSS-TTS's fused multi-channel embedding sum on the HIP kernel.

``ChannelEmbeddingTables`` has the reference's two calls (sglang_omni/models/moss_tts/
channel_embedding.py:53-126): ``refresh(weights)`` binds the channels' tables and returns False
when the kernel cannot take them together, and ``embed(token_ids, weights)`` returns
sum_c weights[c][token_ids[:, c]] in channel order, rounded to the tables' dtype after every add,
ids outside a table's vocabulary adding nothing.

The kernel reads the tables through a device array of their addresses and vocabulary sizes.
Building it copies host memory to the device, which a graph capture must not record, so the
array is built once per set of tables and a capture may only reuse a binding made before it.
"""

from __future__ import annotations

import torch

from .. import _native as N

_TABLE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _binding_key(weights: list[torch.Tensor]) -> tuple | None:
    """What identifies a set of tables to the kernel (device, dtype, width and each table's
    address and rows), or None when the kernel cannot read them as one set: on different GPUs
    or the CPU, of mixed dtypes or widths, a dtype other than bf16 / f16 / f32, not contiguous
    [rows, width] tables."""
    if not weights:
        return None
    head = weights[0]
    if head.device.type != "cuda" or head.dtype not in _TABLE_DTYPES or head.dim() != 2:
        return None
    width = head.shape[1]
    for table in weights:
        if (table.device != head.device or table.dtype != head.dtype or table.dim() != 2
                or table.shape[1] != width or not table.is_contiguous()):
            return None
    return (head.device, head.dtype, int(width),
            tuple((table.data_ptr(), int(table.shape[0])) for table in weights))


class ChannelEmbeddingTables:
    """The bound tables' device array: row 0 their addresses, row 1 their vocabulary sizes."""

    def __init__(self) -> None:
        self._key: tuple | None = None
        self._table_info: torch.Tensor | None = None  # int64 [2, channels] on the tables' GPU
        # the bound tables and their addresses: embed's per-call check (identity and address of
        # each table, a few microseconds) before the full binding key (tens of microseconds)
        self._bound: tuple[tuple[torch.Tensor, int, int], ...] = ()

    def refresh(self, weights: list[torch.Tensor]) -> bool:
        """Bind `weights` (one [vocabulary, hidden] table per channel). True when they are bound
        (already, or now); False when the kernel cannot take them, or when binding them anew
        would copy to the device inside a graph capture."""
        if self._same_tables(weights):
            return True
        key = _binding_key(weights)
        if key is None:
            return False
        if key == self._key:
            self._bound = tuple((table, table.data_ptr(), table.shape[0]) for table in weights)
            return True
        if torch.cuda.is_current_stream_capturing():
            return False
        entries = key[3]
        info = torch.tensor([[address for address, _ in entries], [rows for _, rows in entries]],
                            dtype=torch.int64)
        self._table_info = info.to(key[0])
        self._key = key
        self._bound = tuple((table, table.data_ptr(), table.shape[0]) for table in weights)
        return True

    def _same_tables(self, weights: list[torch.Tensor]) -> bool:
        """The bound tensors themselves, at the addresses and sizes they were bound with."""
        bound = self._bound
        return len(weights) == len(bound) and all(
            table is held and table.data_ptr() == address and table.shape[0] == rows
            for table, (held, address, rows) in zip(weights, bound))

    def _is_bound(self, weights: list[torch.Tensor]) -> bool:
        if self._same_tables(weights):
            return True
        return self._key is not None and _binding_key(weights) == self._key

    def embed(self, token_ids: torch.Tensor, weights: list[torch.Tensor]) -> torch.Tensor:
        """token_ids [rows, channels] int32 / int64 -> [rows, hidden] in the tables' dtype."""
        head = weights[0]
        out = torch.empty(token_ids.shape[0], head.shape[1], dtype=head.dtype, device=head.device)
        if token_ids.shape[0] == 0:
            return out
        if not self._is_bound(weights):
            raise N.OmniCodecError("embed needs the same tables a successful refresh bound")
        N.require_device(token_ids)
        if token_ids.device != head.device:
            raise ValueError(f"token_ids are on {token_ids.device}, the tables on {head.device}")
        if token_ids.dim() != 2 or token_ids.shape[1] != len(weights):
            raise ValueError("token_ids must be [rows, channels], one column per table")
        info = self._table_info
        lib = N.load_library()
        N.check(lib.omni_channel_embedding_sum(
            token_ids.data_ptr(), N.omni_dtype(token_ids.dtype), token_ids.shape[0], len(weights),
            token_ids.stride(0), token_ids.stride(1), info[0].data_ptr(), info[1].data_ptr(),
            N.omni_dtype(head.dtype), head.shape[1], out.data_ptr(), N.stream_handle(head.device)),
            "omni_channel_embedding_sum")
        return out


__all__ = ["ChannelEmbeddingTables"]
