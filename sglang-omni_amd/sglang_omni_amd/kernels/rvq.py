"""RVQ dequantize (gather-and-sum of code embeddings) on the GPU.

Replaces the per-codebook ``F.embedding`` + add of the reference's quantizer decodes
(DAC ``from_codes`` via sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/rvq.py:374-388;
sglang_omni/models/personaplex/components/mimi.py:275-280;
sglang_omni/models/higgs_tts/audio_codec.py:60-78) and the mean form of
sglang_omni/models/qwen3_omni/components/code2wav.py:443.
"""

from __future__ import annotations

import torch

from .. import _native as N


def rvq_gather_sum(
    codes: torch.Tensor,
    codebooks: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
    mean: bool = False,
    clamp: bool = True,
    channels_last: bool = True,
) -> torch.Tensor:
    """out[b, t, :] (channels_last) or out[b, :, t] = sum_k codebooks[k, codes[b, k, t]], summed
    k = 0 .. K-1 in float32 and rounded once. codes [B, K, T] int32/int64 (any strides);
    codebooks [K, V, D] float32 or bf16, contiguous. ``clamp`` reads codes above V-1 as V-1, as
    the DAC quantizer decode does; negative codes (and, without clamp, codes >= V) add nothing.
    """
    N.require_device(codes, codebooks)
    if codes.dim() != 3:
        raise ValueError(f"codes must be [B, K, T], got {tuple(codes.shape)}")
    if codebooks.dim() != 3 or not codebooks.is_contiguous():
        raise ValueError("codebooks must be a contiguous [K, V, D] tensor")
    batch, k, frames = codes.shape
    if codebooks.shape[0] != k:
        raise ValueError(f"{k} codebooks in codes, {codebooks.shape[0]} tables")
    dim = codebooks.shape[2]
    if out is None:
        dtype = out_dtype or codebooks.dtype
        shape = (batch, frames, dim) if channels_last else (batch, dim, frames)
        out = torch.empty(shape, dtype=dtype, device=codes.device)
    if channels_last:
        os_b, os_t, os_d = out.stride(0), out.stride(1), out.stride(2)
    else:
        os_b, os_d, os_t = out.stride(0), out.stride(1), out.stride(2)
    flags = (N.RVQ_MEAN if mean else 0) | (N.RVQ_CLAMP if clamp else 0)
    lib = N.load_library()
    N.check(
        lib.omni_rvq_gather_sum(
            codes.data_ptr(), N.omni_dtype(codes.dtype), batch, k, frames, codes.stride(0),
            codes.stride(1), codes.stride(2), codebooks.data_ptr(), N.omni_dtype(codebooks.dtype),
            codebooks.shape[1], dim, out.data_ptr(), N.omni_dtype(out.dtype), os_b, os_t, os_d,
            flags, N.stream_handle(codes.device),
        ),
        "omni_rvq_gather_sum",
    )
    return out
