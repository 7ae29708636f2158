"""MOSS-TTS's fused multi-channel embedding sum on the HIP kernel.

``ChannelEmbeddingTables`` keeps the reference's API (sglang_omni/models/moss_tts/
channel_embedding.py:53-126): ``refresh(weights)`` points the kernel at the channels' tables
(False when they cannot be fused: not all on one GPU, mixed dtypes or widths, non-contiguous, a
dtype other than bf16 / f16 / f32, or a capture in progress when the address array would have to
be rebuilt) and ``embed(token_ids,
weights)`` returns sum_c weights[c][token_ids[:, c]] in channel order, rounded to the tables'
dtype after every add, ids outside a table's vocabulary adding nothing.
"""

from __future__ import annotations

import torch

from .. import _native as N


class ChannelEmbeddingTables:
    """The channels' table addresses and vocabulary sizes on the device, rebuilt only when the
    tables' storage changes."""

    def __init__(self) -> None:
        self.weight_pointers: tuple[int, ...] = ()
        self.weight_pointer_tensor: torch.Tensor | None = None
        self.vocab_size_tensor: torch.Tensor | None = None

    def refresh(self, weights: list[torch.Tensor]) -> bool:
        first = weights[0]
        hidden = int(first.shape[1])
        if not all(w.is_cuda and w.device == first.device and w.dtype == first.dtype
                   and w.ndim == 2 and int(w.shape[1]) == hidden and w.is_contiguous()
                   for w in weights):
            return False
        if first.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            return False
        pointers = tuple(w.data_ptr() for w in weights)
        if pointers == self.weight_pointers:
            return True
        if torch.cuda.is_current_stream_capturing():
            return False
        self.weight_pointer_tensor = torch.tensor(pointers, dtype=torch.int64, device=first.device)
        self.vocab_size_tensor = torch.tensor([int(w.shape[0]) for w in weights], dtype=torch.int64,
                                              device=first.device)
        self.weight_pointers = pointers
        return True

    def embed(self, token_ids: torch.Tensor, weights: list[torch.Tensor]) -> torch.Tensor:
        """token_ids [rows, channels] int32 / int64 -> [rows, hidden] in the tables' dtype."""
        first = weights[0]
        rows, hidden = int(token_ids.shape[0]), int(first.shape[1])
        output = torch.empty((rows, hidden), device=first.device, dtype=first.dtype)
        if rows == 0:
            return output
        if self.weight_pointer_tensor is None or tuple(w.data_ptr() for w in weights) != self.weight_pointers:
            raise N.OmniCodecError("refresh(weights) must succeed before embed(token_ids, weights)")
        N.require_device(token_ids)
        if token_ids.dim() != 2 or token_ids.shape[1] != len(weights):
            raise ValueError("token_ids must be [rows, channels], one column per table")
        lib = N.load_library()
        N.check(lib.omni_channel_embedding_sum(
            token_ids.data_ptr(), N.omni_dtype(token_ids.dtype), rows, len(weights),
            token_ids.stride(0), token_ids.stride(1), self.weight_pointer_tensor.data_ptr(),
            self.vocab_size_tensor.data_ptr(), N.omni_dtype(first.dtype), hidden,
            output.data_ptr(), N.stream_handle(first.device)), "omni_channel_embedding_sum")
        return output


__all__ = ["ChannelEmbeddingTables"]
