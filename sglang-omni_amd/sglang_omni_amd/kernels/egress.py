"""Waveform egress on the HIP kernel: a decode step's rows packed for one device-to-host copy.

``waveform_egress`` packs the rows of a float32 waveform (B, 1, samples) or (B, samples) into a
(B, samples) buffer as float32 (the relay payload's samples, sglang_omni/utils/audio_payload.py:
40-55) or as signed 16-bit PCM with the realtime bridge's encoding
(sglang_omni/serve/realtime/session_bridge.py:86-88: clip to [-1, 1], times 32767, truncated).
"""

from __future__ import annotations

import torch

from .. import _native as N

FORMATS = {"f32": (N.EGRESS_F32, torch.float32), "pcm16": (N.EGRESS_PCM16, torch.int16)}


def _rows(wave: torch.Tensor) -> torch.Tensor:
    if wave.dim() == 3:
        if wave.shape[1] != 1:
            raise ValueError(f"a (B, 1, samples) waveform is mono; got {tuple(wave.shape)}")
        wave = wave[:, 0]
    if wave.dim() != 2:
        raise ValueError(f"the waveform must be (B, samples) or (B, 1, samples); got "
                         f"{tuple(wave.shape)}")
    if wave.dtype != torch.float32:
        raise ValueError(f"the waveform must be float32; got {wave.dtype}")
    if wave.stride(-1) != 1:
        raise ValueError("the waveform's samples must be contiguous")
    return wave


def waveform_egress(wave: torch.Tensor, *, format: str = "f32",
                    row_samples: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Pack wave's rows into out (B, >= samples) of float32 (format "f32") or int16 ("pcm16").
    row_samples (int64 [B] on the device) stops row r after row_samples[r] samples; the rest of
    that row of out is left as it was. Returns out."""
    if format not in FORMATS:
        raise ValueError(f"format must be one of {sorted(FORMATS)}; got {format!r}")
    code, dtype = FORMATS[format]
    rows = _rows(wave)
    N.require_device(rows, row_samples, out)
    batch, samples = rows.shape
    if out is None:
        out = torch.empty(batch, samples, dtype=dtype, device=rows.device)
    if out.dtype != dtype or out.dim() != 2 or out.shape[0] != batch or out.shape[1] < samples \
            or out.stride(1) != 1:
        raise ValueError(f"out must be {dtype} (B, >= {samples}) with contiguous rows")
    if row_samples is not None and (row_samples.dtype != torch.int64 or row_samples.shape != (batch,)
                                    or not row_samples.is_contiguous()):
        raise ValueError("row_samples must be a contiguous int64 tensor of one count per row")
    lib = N.load_library()
    N.check(lib.omni_waveform_egress(rows.data_ptr(), batch, samples, rows.stride(0),
                                     N.ptr(row_samples), code, out.data_ptr(), out.stride(0),
                                     N.stream_handle(rows.device)),
            "omni_waveform_egress")
    return out
