"""In-place exchanges of per-slot codec state, with the reference kernels' signatures and exact
semantics (sglang_omni/kernels/codec_state.py:150-210): a causal conv's history in front of its
new samples, and a transposed conv's overlap added into its output.

The fused decode path does not call these: its convs read and write slot histories themselves
(see ``fused_conv``). They serve callers written against the reference's kernel API.
"""

from __future__ import annotations

import torch

from .. import _native as N


def history_exchange(
    padded: torch.Tensor,
    history_pool: torch.Tensor,
    slot_index: torch.Tensor,
    new_samples: int,
    is_cold: bool,
) -> None:
    """In place on ``padded`` (rows, H + new_samples + tail, channels), whose middle
    ``new_samples`` positions a producer has written: positions [0, H) receive the row's slot
    history (zeros when ``is_cold``), the tail positions become zero, and the slot's history
    becomes the last H positions of the row's [history, new samples] sequence, read before this
    call changed anything. ``history_pool`` is (slots, H, channels); ``slot_index`` holds one
    distinct slot per row."""
    N.require_device(padded, history_pool, slot_index)
    if padded.dtype != history_pool.dtype:
        raise ValueError("padded and history_pool must share a dtype")
    rows, padded_samples, channels = padded.shape
    history_samples = int(history_pool.shape[1])
    if padded_samples - history_samples - new_samples < 0:
        raise ValueError("padded is shorter than history + new samples")
    index = slot_index.to(torch.int64)
    lib = N.load_library()
    N.check(
        lib.omni_history_exchange(
            padded.data_ptr(), N.omni_dtype(padded.dtype), rows, padded_samples, channels,
            *padded.stride(), history_pool.data_ptr(), history_pool.shape[0], history_samples,
            *history_pool.stride(),
            index.data_ptr(), new_samples, int(is_cold), N.stream_handle(padded.device),
        ),
        "omni_history_exchange",
    )


def overlap_exchange(
    output: torch.Tensor,
    overlap_pool: torch.Tensor,
    slot_index: torch.Tensor,
    emitted_samples: int,
    is_cold: bool,
) -> None:
    """In place on a transposed conv's ``output`` (rows, emitted + O, channels): unless
    ``is_cold``, the first O positions of each row gain the row's slot overlap (summed in float32,
    rounded once); the slot's overlap then becomes the row's positions [emitted, emitted + O) as
    they were before the add. The two ranges are disjoint, which needs emitted_samples >= O."""
    N.require_device(output, overlap_pool, slot_index)
    if output.dtype != overlap_pool.dtype:
        raise ValueError("output and overlap_pool must share a dtype")
    rows, _, channels = output.shape
    overlap_samples = int(overlap_pool.shape[1])
    if emitted_samples < overlap_samples:
        raise ValueError("emitted_samples must be at least the overlap")
    index = slot_index.to(torch.int64)
    lib = N.load_library()
    N.check(
        lib.omni_overlap_exchange(
            output.data_ptr(), N.omni_dtype(output.dtype), rows, channels, *output.stride(),
            overlap_pool.data_ptr(), overlap_pool.shape[0], overlap_samples, *overlap_pool.stride(),
            index.data_ptr(),
            emitted_samples, int(is_cold), N.stream_handle(output.device),
        ),
        "omni_overlap_exchange",
    )
