"""HiFiGAN-style mel -> wave vocoder body on HIP kernels.

Layer order of the HiFT generator's ``decode_body`` up to its output conv
(sglang_omni/models/minicpm_o/components/token2wav/hift.py:255-281, ResBlock
hift_layers.py:57-110) with LeakyReLU activations: conv_pre k=7 -> per stage LeakyReLU(0.1) ->
ConvTranspose1d(k, u, padding (k-u)//2) -> mean of the multi-receptive-field ResBlocks ->
LeakyReLU(0.01) -> conv_post to one channel k=7 -> tanh.

Every conv is one ``omni_conv1d_fused`` launch whose epilogue applies the following LeakyReLU
(so no activation kernel runs on its own); each ResBlock keeps its running sum as a residual
stream (float16 by default: stored in half precision between launches, widened exactly and
added in float32; ``residual_dtype=torch.float32`` keeps it in float32) and the last conv of the
last ResBlock folds in the mean of the three blocks.
"""

from __future__ import annotations

from typing import Any

import torch

from .. import _native as N
from ..kernels.conv import (PackedConv, fused_conv, pack_conv1d, pack_conv_transpose1d,
                            resblock_pair, resblock_pair_supported)
from ..kernels.single_output_conv import single_output_conv
from ..quantization import reference_weights
from .configs import HifiGanConfig


class HifiGanVocoder:
    """mel [B, n_mels, T] -> waveform [B, 1, T * prod(rates)] float32."""

    def __init__(self, weights: dict[str, Any], config: HifiGanConfig, *,
                 device: torch.device | str = "cuda", weight_format: str = "bf16",
                 residual_dtype: torch.dtype = torch.float16, resblock_pairs: bool = True):
        if residual_dtype not in (torch.float16, torch.float32):
            raise ValueError("the residual streams are float16 or float32")
        self.config = config
        self.device = torch.device(device)
        self.residual_dtype = residual_dtype
        # the 32-channel stage's ResBlock pairs as one launch each (omni_resblock_pair)
        self.pairs = resblock_pairs
        fp8 = weight_format == "fp8"
        ref = reference_weights(weights, weight_format)
        dev = self.device
        self.slope = float(weights["slope"])
        self.final_slope = float(weights["final_slope"])
        self.sample_rate = config.sample_rate
        self.hop_length = config.hop_length

        def conv(src: dict, rsrc: dict, dilation: int = 1) -> PackedConv:
            w = src["weight"] if fp8 else rsrc["weight"]
            return pack_conv1d(w, rsrc["bias"], dilation=dilation, causal=False, fp8=fp8).to(dev)

        self.conv_pre = conv(weights["conv_pre"], ref["conv_pre"])
        self.stages = []
        for sw, sr in zip(weights["stages"], ref["stages"]):
            k = sw["up"]["weight"].shape[-1]
            w = sw["up"]["weight"] if fp8 else sr["up"]["weight"]
            up = pack_conv_transpose1d(w, sr["up"]["bias"], stride=sr["rate"],
                                       padding=(k - sr["rate"]) // 2, fp8=fp8).to(dev)
            blocks = []
            for bw, br in zip(sw["resblocks"], sr["resblocks"]):
                pairs = [
                    (conv(c1w, c1r, d), conv(c2w, c2r, 1))
                    for c1w, c1r, c2w, c2r, d in zip(bw["convs1"], br["convs1"], bw["convs2"],
                                                     br["convs2"], br["dilations"])
                ]
                blocks.append(pairs)
            self.stages.append({"rate": sr["rate"], "up": up, "blocks": blocks})
        post = ref["conv_post"]
        self.post_weight = post["weight"][0].t().contiguous().float().to(dev)  # [k, C]
        self.post_bias = post["bias"].float().to(dev).contiguous()
        self.post_taps = post["weight"].shape[-1]
        if len(self.stages[0]["blocks"]) != 3:
            raise ValueError("the MRF mean is fused for three ResBlocks per stage")

    def _workspace(self, elements: int) -> tuple[torch.Tensor, ...]:
        """The intermediate activations of a call: four bf16 buffers and three residual streams
        (``residual_dtype``), flat, of at least ``elements`` each, kept between calls and grown
        (never shrunk) when a call needs more. Calls on one vocoder share them, so they must not
        overlap (one stream, or calls ordered between streams)."""
        ws = getattr(self, "_ws", None)
        if ws is None or ws[0].numel() < elements:
            bf, rd = torch.bfloat16, self.residual_dtype
            ws = tuple(torch.empty(elements, dtype=dt, device=self.device)
                       for dt in (bf, bf, bf, bf, rd, rd, rd))
            self._ws = ws
        return ws

    @torch.no_grad()
    def forward(self, mel: torch.Tensor) -> torch.Tensor:
        N.require_device(mel)
        batch, _, frames = mel.shape
        dev = self.device
        # layout/dtype plumbing of the input: [B, n_mels, T] -> channels-last bf16
        x = mel.transpose(1, 2).to(torch.bfloat16).contiguous()
        length = frames
        c = self.conv_pre.n_cols
        sizes = [length * c]
        ll, cc = length, c
        for st in self.stages:
            ll *= st["rate"]
            cc = st["up"].c_out
            sizes.append(ll * cc)
        act_p, act_q, h, run, xs, xb0, xb1 = self._workspace(batch * max(sizes))
        xb = [xb0, xb1]

        def view(flat: torch.Tensor, length: int, ch: int) -> torch.Tensor:
            return flat[: batch * length * ch].view(batch, length, ch)

        lrelu = N.ACT_LEAKY_RELU
        p = view(act_p, length, c)
        fused_conv(x, self.conv_pre, p, activation=lrelu, slope=self.slope)
        for si, st in enumerate(self.stages):
            up: PackedConv = st["up"]
            out_len = length * st["rate"]
            cout = up.c_out
            q = view(act_q, out_len, cout)
            xstage = view(xs, out_len, cout)
            fused_conv(p, up, q.view(batch, length, up.n_cols), activation=lrelu, slope=self.slope,
                       sum_out=xstage.view(batch, length, up.n_cols))
            length = out_len
            hv = view(h, length, cout)
            rv = view(run, length, cout)
            last_stage = si + 1 == len(self.stages)
            pn = view(act_p, length, cout)
            for j, pairs in enumerate(st["blocks"]):
                xj = view(xb[j], length, cout) if j < 2 else None
                src = q
                for m, (c1, c2) in enumerate(pairs):
                    # (k = 11 pairs measured slower as one launch: 540-610 against 435 us for
                    # the two launches at 16 x 240 000 samples, the tile's 2 x 30-row x halo)
                    paired = self.pairs and c1.taps < 11 and resblock_pair_supported(c1, c2)
                    last_m = m + 1 == len(pairs)
                    resid = xstage if m == 0 else (xj if j < 2 else xstage)
                    if not last_m:
                        # running sum of this block; block 2 reuses the stage buffer in place.
                        # A pair reads its operand's neighbours' halo rows, so it writes the next
                        # operand into the other buffer (h stays on chip, so hv is free)
                        target = xj if j < 2 else xstage
                        nxt = (hv if src is rv else rv) if paired else rv
                        c2_out, kw = nxt, dict(activation=lrelu, slope=self.slope,
                                               residual=resid, sum_out=target)
                    elif j < 2:
                        c2_out, kw = None, dict(residual=resid, sum_out=xj)
                    else:
                        slope = self.final_slope if last_stage else self.slope
                        c2_out, kw = pn, dict(activation=lrelu, slope=slope, residual=resid,
                                              mix=(view(xb[0], length, cout),
                                                   view(xb[1], length, cout), 1.0 / 3.0))
                    if paired:
                        # the 32-channel pairs: h stays on chip
                        resblock_pair(src, c1, c2, c2_out, slope1=self.slope, **kw)
                    else:
                        fused_conv(src, c1, hv, activation=lrelu, slope=self.slope)
                        fused_conv(hv, c2, c2_out, **kw)
                    src = c2_out
            p = pn
        wave = torch.empty(batch, 1, length, dtype=torch.float32, device=dev)
        single_output_conv(p, self.post_weight, self.post_bias, wave, activation=N.ACT_TANH,
                           left_pad=(self.post_taps - 1) // 2)
        return wave

    __call__ = forward
