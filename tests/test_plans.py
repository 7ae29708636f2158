"""The conv launcher's plan and forced-configuration entry points without a GPU: the tile lists
have the lengths the forced-tile GPU tests sweep, the benchmarked workloads' layer shapes plan to
entries of those lists, and contract violations are refused before anything runs."""

from __future__ import annotations

import ctypes

import pytest

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import plan_shapes
from tests.test_gpu_tiles import (
    DMA_LIST,
    FUSED_LIST,
    NARROW128_DMA_LIST,
    NARROW_DMA_LIST,
    STAGED11_LIST,
    STAGED_LIST,
)


def test_list_lengths_match_the_forced_tile_sweep():
    for taps, n in DMA_LIST.items():
        c_out = 96
        n_cols = 6 * c_out if taps == 2 else c_out
        for fp8 in (False, True):  # E4M3 weights take the same tile lists
            plan = plan_shapes(batch=2, length=300, c_in=192, n_cols=n_cols, c_out=c_out,
                               taps=taps, left_pad=1 if taps == 2 else None, fp8=fp8)
            assert plan.kernel == N.CONV_KERNEL_DMA and plan.configs == n
    staged = plan_shapes(batch=2, length=300, c_in=96, n_cols=192, c_out=192, taps=7, fp8=True,
                         in_activation=N.ACT_SNAKE)
    assert staged.kernel == N.CONV_KERNEL_STAGED and staged.configs == STAGED_LIST
    s11 = plan_shapes(batch=2, length=300, c_in=64, n_cols=64, c_out=64, taps=11, dilation=5,
                      left_pad=25, in_activation=N.ACT_LEAKY_RELU)
    assert s11.kernel == N.CONV_KERNEL_STAGED11 and s11.configs == STAGED11_LIST
    for taps in NARROW_DMA_LIST:  # narrow layers with a ready bf16 operand
        for cols in (256, 128, 64, 32) if taps == 3 else (128, 64, 32):
            n = (NARROW128_DMA_LIST if cols > 64 else NARROW_DMA_LIST)[taps]
            plan = plan_shapes(batch=2, length=300, c_in=cols, n_cols=cols, c_out=cols,
                               taps=taps, dilation=5, left_pad=(taps - 1) * 5 // 2)
            assert plan.kernel == N.CONV_KERNEL_DMA and plan.configs == n
    fused = plan_shapes(batch=2, length=300, c_in=96, n_cols=96, c_out=96, taps=7, dilation=9,
                        fused_unit=True)
    assert fused.kernel == N.CONV_KERNEL_FUSED_UNIT and fused.configs == FUSED_LIST


@pytest.mark.parametrize("layer", [
    # (name, c_in, n_cols, c_out, taps, dilation, left_pad, fused) at 64 streams x 12 frames
    ("in_conv", 512, 1536, 1536, 7, 1, None, False, 12),
    ("block1.up", 768, 8 * 384, 384, 2, 1, 1, False, 96),
    ("block1.k7d9", 384, 384, 384, 7, 9, None, False, 768),
    ("block1.k1", 384, 384, 384, 1, 1, None, False, 768),
    ("block2.unit", 192, 192, 192, 7, 3, None, True, 3840),
    ("block3.up", 192, 6 * 96, 96, 2, 1, 1, False, 3840),
])
def test_streaming_step_layers_plan_to_swept_entries(layer):
    name, c_in, n_cols, c_out, taps, d, left, fused, length = layer
    plan = plan_shapes(batch=64, length=length, c_in=c_in, n_cols=n_cols, c_out=c_out, taps=taps,
                       dilation=d, left_pad=left, fused_unit=fused, history=True)
    assert 1 <= plan.config <= plan.configs
    assert plan.workgroups >= 64
    if plan.kernel == N.CONV_KERNEL_DMA:
        assert plan.configs == DMA_LIST[taps]


def test_forced_choice_contract():
    kw = dict(batch=2, length=300, c_in=192, n_cols=192, c_out=192, taps=7, dilation=3)
    # a family that cannot serve the call, and entries past the list, are "unsupported"
    with pytest.raises(N.OmniCodecError, match="status 2"):
        plan_shapes(**kw, kernel=N.CONV_KERNEL_FUSED_UNIT, config=1)
    with pytest.raises(N.OmniCodecError, match="status 2"):
        plan_shapes(**kw, kernel=N.CONV_KERNEL_DMA, config=DMA_LIST[7] + 1)
    # LDS-DMA copies the operand as it is: an operand activated on the way in never takes it
    with pytest.raises(N.OmniCodecError, match="status 2"):
        plan_shapes(**kw, in_activation=N.ACT_SNAKE, kernel=N.CONV_KERNEL_DMA, config=1)
    assert plan_shapes(**kw, fp8=True, kernel=N.CONV_KERNEL_DMA, config=1).config == 1
    # an unknown family or a configuration without a family is an invalid argument
    with pytest.raises(N.OmniCodecError, match="status 1"):
        plan_shapes(**kw, kernel=9, config=1)
    with pytest.raises(N.OmniCodecError, match="status 1"):
        plan_shapes(**kw, kernel=N.CONV_KERNEL_AUTO, config=2)
    # the forced launch refuses the automatic family, and a null argument block
    lib = N.load_library()
    assert lib.omni_conv1d_fused_with(None, N.CONV_KERNEL_DMA, 1, None) == N.INVALID_ARG
    args = N.ConvArgs()
    assert lib.omni_conv1d_fused_with(ctypes.byref(args), N.CONV_KERNEL_AUTO, 0, None) == N.INVALID_ARG


def test_an_empty_call_plans_nothing():
    plan = plan_shapes(batch=0, length=12, c_in=96, n_cols=96, c_out=96, taps=7)
    assert plan.kernel == N.CONV_KERNEL_AUTO and plan.config == 0


@pytest.mark.parametrize("channels,length", [(256, 4000), (128, 20000), (64, 60000), (32, 240000)])
@pytest.mark.parametrize("taps", [3, 7, 11])
def test_hifigan_resblock_convs_plan_to_their_tiles(channels, length, taps):
    """HiFiGAN's ResBlock convs at 16 clips x 500 mel frames ('same' padding, dilations 1 and 5)
    take the families and entries their measurements chose: LDS-DMA for all but the 256-channel
    k = 11 convs (register-staged), the one-buffer-ring entries first where c_in is one stage."""
    for d in (1, 5):
        plan = plan_shapes(batch=16, length=length, c_in=channels, n_cols=channels,
                           c_out=channels, taps=taps, dilation=d, left_pad=(taps - 1) * d // 2)
        if channels == 256 and taps == 11:
            assert plan.kernel == N.CONV_KERNEL_STAGED11
            continue
        assert plan.kernel == N.CONV_KERNEL_DMA
        if channels == 256 and taps == 7:
            assert plan.configs == DMA_LIST[7]
        elif channels >= 128:
            assert plan.configs == NARROW128_DMA_LIST[taps]
        else:
            assert plan.configs == NARROW_DMA_LIST[taps]
        # 64 channels: the two-chunk one-stage entry (k = 3) or the 64-column entry follows the
        # 32-column one-stage entry, which needs c_in = 32
        assert plan.config == (2 if channels == 64 else 1)
        assert plan.workgroups >= 256
