"""The weight tree and configuration of ``DacCodecDecoder`` from the reference's DAC codec module.

``dac_weight_tree(dac)`` walks the causal decoder the reference builds
(sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/modded_dac.py:790-835):

    decoder.model = [CausalConvNet(latent -> C, k 7),
                     DecoderBlock.block = [Snake1d, CausalTransConvNet(k 2s, stride s),
                                           ResidualUnit.block = [Snake1d, CausalConvNet(k 7, d),
                                                                 Snake1d, CausalConvNet(k 1)]
                                           x 3] x len(rates),
                     Snake1d, CausalConvNet(C_last -> 1, k 7), Tanh]

reading each conv's weight with weight norm folded (g * v / |v| per output slice, the value
``DAC.fold_weight_norm`` writes, modded_dac.py:994-1002) and each Snake1d's alpha.

The quantizer (``DownsampleResidualVectorQuantize.decode``, rvq.py:374-388) sums, per frame, the
semantic quantizer's and the residual quantizers' ``out_proj(codebook[code])`` (each code clamped
to its own codebook). Every term is a fixed row of a [V, D] table out_proj(codebook) + bias, so
the tree's ``codebooks`` are those tables stacked in quantizer order (semantic first), the
decoder's gather-sum adding them in that order. Codebooks of different sizes are padded to the
largest with copies of their own last row, so the gather's clamp to the largest size reads
exactly the row each quantizer's own clamp reads. A quantizer whose decode continues past the
sum (a ``post_module`` or ``upsample`` that is not the identity) cannot be folded: the tree then
holds no codebooks and the decoder is driven from latents (``DacCodecDecoder.decode``).
"""

from __future__ import annotations

from typing import Any

import torch

from .configs import DacDecoderConfig


def _folded_weight(conv: torch.nn.Module) -> torch.Tensor:
    """A Conv1d / ConvTranspose1d weight with weight norm folded in: the parametrized weight
    (torch.nn.utils.parametrizations.weight_norm) evaluates g * v / |v|; the older hook form
    (weight_g / weight_v) is folded here the same way (dim 0)."""
    if hasattr(conv, "weight_g") and hasattr(conv, "weight_v"):
        return torch._weight_norm(conv.weight_v, conv.weight_g, 0).detach()
    return conv.weight.detach()


def _conv_of(module: torch.nn.Module, kind: type) -> torch.nn.Module:
    """The torch conv inside a CausalConvNet / CausalTransConvNet (its ``conv``)."""
    conv = getattr(module, "conv", None)
    if not isinstance(conv, kind):
        raise ValueError(f"{type(module).__name__} is not a causal {kind.__name__} wrapper: the "
                         "decoder on these kernels is the causal DAC decoder")
    return conv


def _conv_entry(conv: torch.nn.Module) -> dict[str, torch.Tensor]:
    bias = conv.bias.detach().float().clone() if conv.bias is not None else None
    return {"weight": _folded_weight(conv).float().clone(), "bias": bias}


def _alpha(snake: torch.nn.Module) -> torch.Tensor:
    alpha = getattr(snake, "alpha", None)
    if alpha is None:
        raise ValueError(f"expected a Snake1d, found {type(snake).__name__}")
    return alpha.detach().float().reshape(-1).clone()


def _children(module: torch.nn.Module, attr: str = "block") -> list[torch.nn.Module]:
    seq = getattr(module, attr, None)
    if seq is None:
        raise ValueError(f"{type(module).__name__} has no {attr!r} sequence")
    return [m for m in seq if not isinstance(m, torch.nn.Identity)]


def _unit(module: torch.nn.Module) -> dict[str, Any]:
    snake1, conv1, snake2, conv2 = _children(module)
    c1 = _conv_of(conv1, torch.nn.Conv1d)
    c2 = _conv_of(conv2, torch.nn.Conv1d)
    if c1.kernel_size[0] != 7 or c2.kernel_size[0] != 1 or c1.stride[0] != 1 or c1.groups != 1:
        raise ValueError("a residual unit is a k = 7 dilated conv and a k = 1 conv")
    return {"dilation": c1.dilation[0], "alpha1": _alpha(snake1), "conv1": _conv_entry(c1),
            "alpha2": _alpha(snake2), "conv2": _conv_entry(c2)}


def _block(module: torch.nn.Module) -> dict[str, Any]:
    parts = _children(module)
    snake, up, units = parts[0], parts[1], parts[2:]
    t = _conv_of(up, torch.nn.ConvTranspose1d)
    stride = t.stride[0]
    if t.kernel_size[0] != 2 * stride or t.dilation[0] != 1 or t.groups != 1:
        raise ValueError("a decoder block upsamples by a k = 2s transposed conv")
    return {"stride": stride, "alpha": _alpha(snake), "up": _conv_entry(t),
            "units": [_unit(u) for u in units]}


def _gather_tables(quantizers: list[torch.nn.Module]) -> torch.Tensor:
    """out_proj(codebook) + bias of each vector quantizer, [K, V_max, D] float32, smaller
    codebooks padded with copies of their last row."""
    tables = []
    for vq in quantizers:
        book = vq.codebook.weight.detach().double()  # [V, d]
        proj = _folded_weight(vq.out_proj).double()[:, :, 0]  # [D, d]
        table = book @ proj.t()
        if vq.out_proj.bias is not None:
            table = table + vq.out_proj.bias.detach().double()
        tables.append(table.float())
    size = max(t.shape[0] for t in tables)
    padded = [torch.cat([t, t[-1:].expand(size - t.shape[0], -1)]) if t.shape[0] < size else t
              for t in tables]
    return torch.stack(padded)


def _quantizers(quantizer: torch.nn.Module) -> list[torch.nn.Module] | None:
    """The vector quantizers whose projected codebook rows sum to the decoder's input, in the
    order the decode adds them; None when the decode does more than sum them."""
    for name in ("post_module", "upsample"):
        extra = getattr(quantizer, name, None)
        if extra is None or isinstance(extra, torch.nn.Identity):
            continue
        if isinstance(extra, torch.nn.Sequential) and len(extra) == 0:
            continue
        return None
    groups = []
    for name in ("semantic_quantizer", "quantizer"):
        rvq = getattr(quantizer, name, None)
        if rvq is not None:
            groups.extend(rvq.quantizers)
    if not groups and hasattr(quantizer, "quantizers"):
        groups = list(quantizer.quantizers)
    return groups or None


def dac_weight_tree(dac: torch.nn.Module, *, sample_rate: int | None = None,
                    ) -> tuple[dict[str, Any], DacDecoderConfig]:
    """(weights, config) for ``DacCodecDecoder`` from the reference's ``DAC`` (its ``decoder``
    and, when foldable, its ``quantizer``) or from a bare ``Decoder``. Weights are float32 CPU
    tensors in the reference's layouts; the module is left as it is."""
    decoder = getattr(dac, "decoder", dac)
    layers = [m for m in decoder.model if not isinstance(m, torch.nn.Identity)]
    if len(layers) < 4 or not isinstance(layers[-1], torch.nn.Tanh):
        raise ValueError("the decoder's model must end in Snake1d, conv to one channel, Tanh")
    in_conv = _conv_of(layers[0], torch.nn.Conv1d)
    final_conv = _conv_of(layers[-2], torch.nn.Conv1d)
    blocks = [_block(m) for m in layers[1:-3]]
    weights: dict[str, Any] = {
        "in_conv": _conv_entry(in_conv),
        "blocks": blocks,
        "final": {"alpha": _alpha(layers[-3]), "conv": _conv_entry(final_conv)},
    }
    quantizer = getattr(dac, "quantizer", None)
    vqs = _quantizers(quantizer) if quantizer is not None else None
    if vqs is not None:
        weights["codebooks"] = _gather_tables(vqs)
    dilations = tuple(u["dilation"] for u in blocks[0]["units"]) if blocks else (1, 3, 9)
    for b in blocks:
        if tuple(u["dilation"] for u in b["units"]) != dilations:
            raise ValueError("every block's residual units share one dilation pattern")
    config = DacDecoderConfig(
        n_codebooks=0 if vqs is None else len(vqs),
        codebook_size=0 if vqs is None else int(weights["codebooks"].shape[1]),
        latent_dim=in_conv.in_channels,
        channels=in_conv.out_channels,
        rates=tuple(b["stride"] for b in blocks),
        dilations=dilations,
        kernel_size=in_conv.kernel_size[0],
        sample_rate=int(sample_rate if sample_rate is not None
                        else getattr(dac, "sample_rate", 44100)),
    )
    return weights, config


__all__ = ["dac_weight_tree"]
