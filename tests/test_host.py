"""Host-side logic on the CPU: weight packing (the conv kernel's polyphase form), fp8 weight
formats, decoder geometry and algorithmic work, the slot-state layout, and that the product
path refuses to run anywhere but on the GPU kernels."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import codec_oracle as O
from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import (
    CHUNK,
    PackedConv,
    fused_conv,
    pack_conv1d,
    pack_conv_transpose1d,
    polyphase_taps,
)
from sglang_omni_amd.models.configs import (
    CODEC_24K,
    CODEC_24K_LONG,
    HIFIGAN_24K,
    DacDecoderConfig,
    dac_macs_per_frame,
    hifigan_macs_per_frame,
    make_dac_weights,
)
from sglang_omni_amd.quantization import dequantize_fp8, quantize_fp8, reference_weights


def unpack(conv: PackedConv) -> torch.Tensor:
    """The kernel's [chunks, n_cols, taps, 32] weight back to [n_cols, taps, C_in] float64, with
    the fp8 scale applied."""
    w = conv.weight.to(torch.float64) if conv.weight.dtype != torch.float8_e4m3fn \
        else conv.weight.float().double()
    chunks, n_cols, taps, _ = w.shape
    w = w.permute(1, 2, 0, 3).reshape(n_cols, taps, chunks * CHUNK)
    if conv.scale is not None:
        w = w * conv.scale.double().view(-1, 1, 1)
    return w


def emulate(x: torch.Tensor, conv: PackedConv, length: int) -> torch.Tensor:
    """The fused conv's arithmetic in float64, from the packed weights:
    out[b, i, n] = bias[n % C_out] + sum_j sum_ci W[n, j, ci] x[b, i + j*d - left_pad, ci],
    x zero outside its positions. x [B, XL, C_in] -> [B, length, n_cols]."""
    w = unpack(conv)[..., : conv.c_in]
    batch, xl, _ = x.shape
    out = torch.zeros(batch, length, conv.n_cols, dtype=torch.float64)
    xd = x.double()
    for j in range(conv.taps):
        for i in range(length):
            p = i + j * conv.dilation - conv.left_pad
            if 0 <= p < xl:
                out[:, i] += xd[:, p] @ w[:, j].t()
    if conv.bias is not None:
        out += conv.bias.double().repeat(conv.phases)
    return out


@pytest.mark.parametrize("k,d,causal", [(7, 1, True), (7, 9, True), (1, 1, True), (11, 5, False)])
def test_packed_conv1d_computes_the_conv(k, d, causal):
    gen = torch.Generator().manual_seed(k * 10 + d)
    w = torch.randn(16, 40, k, generator=gen)  # 40 channels: a partial second chunk
    b = torch.randn(16, generator=gen)
    x = torch.randn(2, 30, 40, generator=gen)
    conv = pack_conv1d(w, b, dilation=d, causal=causal)
    assert conv.weight.shape == (2, 16, k, CHUNK) and conv.weight.dtype == torch.bfloat16
    assert torch.equal(conv.weight[1, :, :, 8:], torch.zeros(16, k, 24, dtype=torch.bfloat16))
    wr = w.to(torch.bfloat16).double()
    if causal:
        expected = O.causal_conv1d(x.double().transpose(1, 2), wr, b.double(), d)
    else:
        expected = O.same_conv1d(x.double().transpose(1, 2), wr, b.double(), d)
    got = emulate(x, conv, 30)
    torch.testing.assert_close(got, expected.transpose(1, 2), rtol=1e-9, atol=1e-9)
    assert conv.macs_per_position == 16 * 40 * k


@pytest.mark.parametrize("stride", [2, 5, 6, 8])
def test_polyphase_form_of_the_causal_transposed_conv(stride):
    gen = torch.Generator().manual_seed(stride)
    w = torch.randn(32, 8, 2 * stride, generator=gen).to(torch.bfloat16).float()
    b = torch.randn(8, generator=gen)
    x = torch.randn(2, 11, 32, generator=gen)
    conv = pack_conv_transpose1d(w, b, stride=stride)
    # k = 2s: every phase has two taps, over inputs i - 1 and i
    assert (conv.taps, conv.left_pad, conv.n_cols) == (2, 1, stride * 8)
    got = emulate(x, conv, 11).view(2, 11 * stride, 8)
    expected = O.causal_conv_transpose1d(x.double().transpose(1, 2), w.double(), b.double(),
                                         stride)
    torch.testing.assert_close(got, expected.transpose(1, 2), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("rate,k", [(8, 16), (5, 11), (3, 7), (4, 8)])
def test_polyphase_form_of_the_padded_transposed_conv(rate, k):
    gen = torch.Generator().manual_seed(k)
    w = torch.randn(16, 8, k, generator=gen).to(torch.bfloat16).float()
    x = torch.randn(1, 9, 16, generator=gen)
    conv = pack_conv_transpose1d(w, None, stride=rate, padding=(k - rate) // 2)
    got = emulate(x, conv, 9).view(1, 9 * rate, 8)
    expected = O.padded_conv_transpose1d(x.double().transpose(1, 2), w.double(), None, rate)
    torch.testing.assert_close(got, expected.transpose(1, 2), rtol=1e-9, atol=1e-9)


def test_polyphase_taps_by_brute_force():
    # every (output phase r, tap delta) entry holds exactly the weight tap j with
    # s*(i + delta) + j - p = s*i + r
    w = torch.arange(3 * 2 * 7, dtype=torch.float64).view(3, 2, 7)
    s, p = 3, 2
    out, left = polyphase_taps(w, s, p)
    for r in range(s):
        for t in range(out.shape[1]):
            delta = t - left
            j = s * 0 + r + p - s * delta
            expected = w[:, :, j].t() if 0 <= j < 7 else torch.zeros(2, 3, dtype=torch.float64)
            assert torch.equal(out[r * 2:(r + 1) * 2, t], expected)


def test_fp8_packing_shares_one_scale_per_output_channel_across_phases():
    gen = torch.Generator().manual_seed(9)
    w = torch.randn(16, 8, 12, generator=gen) * torch.logspace(-2, 0, 8).view(1, 8, 1)
    conv = pack_conv_transpose1d(w, None, stride=6, fp8=True)
    assert conv.weight.dtype == torch.float8_e4m3fn
    assert torch.equal(conv.scale, conv.scale[:8].repeat(6))
    q, s = quantize_fp8(w, 1)
    torch.testing.assert_close(conv.scale[:8], s)
    deq = dequantize_fp8(q, s, 1)
    x = torch.randn(1, 7, 16, generator=gen)
    got = emulate(x, conv, 7).view(1, 42, 8)
    expected = O.causal_conv_transpose1d(x.double().transpose(1, 2), deq.double(), None, 6)
    # deq holds q * s rounded to float32; the emulation multiplies in float64
    torch.testing.assert_close(got, expected.transpose(1, 2), rtol=1e-5, atol=1e-6)
    assert torch.equal(unpack(conv)[..., :16].float().view(6, 8, 2, 16).abs().amax((0, 2, 3)),
                       s * 448)


def test_reference_weights_formats():
    cfg = DacDecoderConfig(n_codebooks=2, codebook_size=8, latent_dim=16, channels=32,
                           rates=(2, 3))
    w = make_dac_weights(cfg, seed=0)
    bf = reference_weights(w, "bf16")
    c1 = bf["blocks"][0]["units"][0]["conv1"]["weight"]
    assert torch.equal(c1, w["blocks"][0]["units"][0]["conv1"]["weight"].to(torch.bfloat16).float())
    assert torch.equal(bf["codebooks"], w["codebooks"].to(torch.bfloat16).float())
    f8 = reference_weights(w, "fp8")
    up = f8["blocks"][1]["up"]["weight"]
    q, s = O.quantize_fp8_per_channel(w["blocks"][1]["up"]["weight"].transpose(0, 1))
    torch.testing.assert_close(up, O.dequantize_fp8_per_channel(q, s).transpose(0, 1))
    with pytest.raises(ValueError):
        reference_weights(w, "int4")


def test_decoder_geometry_and_algorithmic_work():
    assert CODEC_24K.hop_length == 1920 and CODEC_24K.frame_rate == 12.5
    assert CODEC_24K.stage_channels() == [1536, 768, 384, 192, 96]
    # 1 228 910 592 multiply-adds per frame = 30.72 GFLOP per audio-second
    assert dac_macs_per_frame(CODEC_24K) == 1_228_910_592
    assert abs(2 * dac_macs_per_frame(CODEC_24K) * 12.5 / 1e9 - 30.72) < 0.01
    assert HIFIGAN_24K.hop_length == 480
    assert hifigan_macs_per_frame(HIFIGAN_24K) == 282_133_504
    assert (CODEC_24K_LONG.n_codebooks, CODEC_24K_LONG.codebook_size) == (32, 1024)


def test_macs_per_frame_by_counting_the_weights():
    cfg = DacDecoderConfig(n_codebooks=2, codebook_size=8, latent_dim=16, channels=32,
                           rates=(2, 3))
    w = make_dac_weights(cfg, seed=0)
    samples, macs = 1, w["in_conv"]["weight"].numel()
    for blk in w["blocks"]:
        macs += samples * blk["up"]["weight"].numel()
        samples *= blk["stride"]
        for u in blk["units"]:
            macs += samples * (u["conv1"]["weight"].numel() + u["conv2"]["weight"].numel())
    macs += samples * w["final"]["conv"]["weight"].numel()
    assert dac_macs_per_frame(cfg) == macs


@pytest.fixture(scope="module")
def cpu_decoder():
    from sglang_omni_amd.models.dac_codec import DacCodecDecoder

    return DacCodecDecoder(make_dac_weights(CODEC_24K, seed=0), CODEC_24K, device="cpu")


def test_slot_state_layout_of_the_24k_decoder(cpu_decoder):
    # per stream: each causal conv's (k-1)*d left context (512*6 for the input conv, 96*6 for the
    # final one, c*6*d in the residual units), one input sample per transposed conv (k = 2s), none
    # for the k = 1 convs: 118 848 elements, two copies of each in the pool. (The reference's
    # overlap form keeps (k-s)*C_out output samples per transposed conv instead: 126 720.)
    layout = cpu_decoder.state_layout()
    chans = CODEC_24K.stage_channels()
    expected = 512 * 6 + 96 * 6 + sum(chans[i] + sum(chans[i + 1] * 6 * d for d in (1, 3, 9))
                                      for i in range(4))
    assert sum(c * n for _, c, n in layout) == expected == 118_848
    overlap_form = expected - sum(chans[:4]) + sum(s * c for s, c in zip((8, 8, 5, 6), chans[1:]))
    assert overlap_form == 126_720
    pool = cpu_decoder.new_state_pool(num_slots=3, capture_slots=1)
    assert pool.bytes_per_slot == 2 * 2 * 118_848
    assert pool.available_size() == 3 and pool.scratch_slots == (3,)
    got = [pool.acquire() for _ in range(4)]
    assert got[:3] == [0, 1, 2] and got[3] is None
    pool.release(1)
    assert pool.acquire() == 1
    assert all(h.shape[:2] == (4, 2) for h in pool.histories.values())


def test_decoder_on_cpu_fails_loudly_instead_of_falling_back(cpu_decoder):
    codes = torch.zeros(1, 16, 2, dtype=torch.int64)
    with pytest.raises(N.OmniCodecError, match="GPU"):
        cpu_decoder.from_indices(codes)
    with pytest.raises(ValueError):
        cpu_decoder.from_indices(codes[0])


def test_product_path_refuses_cpu_tensors():
    from sglang_omni_amd.kernels.rvq import rvq_gather_sum

    codes = torch.zeros(1, 2, 3, dtype=torch.int64)
    tables = torch.zeros(2, 4, 8)
    with pytest.raises(N.OmniCodecError, match="GPU"):
        rvq_gather_sum(codes, tables)
    conv = pack_conv1d(torch.zeros(16, 8, 7), None)
    x = torch.zeros(1, 4, 8, dtype=torch.bfloat16)
    out = torch.zeros(1, 4, 16, dtype=torch.bfloat16)
    with pytest.raises(N.OmniCodecError, match="GPU"):
        fused_conv(x, conv, out)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(N, "_lib", None)
    with pytest.raises(N.OmniCodecError, match="missing"):
        N.load_library(tmp_path / "libomni_codec.so")


def test_rocm_platform_entry():
    from sglang_omni_amd.platforms import current_platform

    assert current_platform.device_type == "cuda"
    assert current_platform.get_device_graph_backend() == "hip_graph"
    assert current_platform.is_cuda() is False


@pytest.mark.parametrize("stride,k,padding,output_padding,dilation", [
    (4, 8, 2, 0, 2), (3, 6, 1, 2, 3), (5, 10, 0, 0, 1), (2, 7, 3, 1, 2)])
def test_polyphase_form_with_dilation_and_output_padding(stride, k, padding, output_padding,
                                                         dilation):
    """The general transposed conv (F.conv_transpose1d with padding, output padding and
    dilation) is the packed form's first L_out samples, with as many positions as cover them."""
    gen = torch.Generator().manual_seed(stride * k + dilation)
    w = torch.randn(16, 8, k, generator=gen).to(torch.bfloat16).float()
    b = torch.randn(8, generator=gen)
    x = torch.randn(2, 9, 16, generator=gen)
    conv = pack_conv_transpose1d(w, b, stride=stride, padding=padding, dilation=dilation)
    expected = F.conv_transpose1d(x.double().transpose(1, 2), w.double(), b.double(),
                                  stride=stride, padding=padding, output_padding=output_padding,
                                  dilation=dilation).transpose(1, 2)
    length_out = expected.shape[1]
    positions = -(-length_out // stride)
    got = emulate(x, conv, positions).view(2, positions * stride, 8)[:, :length_out]
    torch.testing.assert_close(got, expected, rtol=1e-9, atol=1e-9)


def test_channels_last_weight_helpers():
    """tests/unit_test/utils/test_channels_last_conv.py:103-115: the channels-last weight keeps
    the module's values and leaves the module alone; the folded weight of a stride-s conv is the
    stride-one conv over the input's phases."""
    from sglang_omni_amd.utils.channels_last_conv import (
        channels_last_folded_weight,
        channels_last_weight,
    )

    conv = torch.nn.Conv1d(4, 6, 7)
    weight = channels_last_weight(conv)
    assert torch.equal(weight, conv.weight)
    assert weight.transpose(1, 2).is_contiguous() and conv.weight.is_contiguous()
    strided = torch.nn.Conv1d(4, 6, 6, stride=3)
    x = torch.randn(2, 4, 30)
    folded = channels_last_folded_weight(strided.weight.data, 3)
    phases = x.transpose(1, 2).reshape(2, 10, 12).transpose(1, 2)
    torch.testing.assert_close(F.conv1d(phases, folded, strided.bias), strided(x))


def test_checkpoint_fp8_scales_map_onto_per_channel_scales():
    """A checkpoint's E4M3 conv weight with its weight_scale_inv (per tensor, per channel, row
    blocks, inverted) gives the per-output-channel form whose dequantized values are the
    checkpoint's; the reference's refusals (sglang_omni/quantization.py:137-166) hold."""
    from sglang_omni_amd.quantization import fp8_conv_weight

    gen = torch.Generator().manual_seed(12)
    w = torch.randn(24, 16, 7, generator=gen)
    q, s = quantize_fp8(w, 0)
    deq = dequantize_fp8(q, s, 0)
    q2, s2 = fp8_conv_weight("conv", q, s)
    assert q2 is q and torch.equal(s2, s)
    q3, s3 = fp8_conv_weight("conv", q, 1.0 / s, inverted=True)
    torch.testing.assert_close(dequantize_fp8(q3, s3, 0), deq)
    # blocks of 8 rows whose multipliers are constant along the row: exact
    blocks = s.view(3, 8).amax(1, keepdim=True).expand(3, 4).contiguous()
    qb = (w / blocks.repeat_interleave(8, 0)[:, :1].view(24, 1, 1)).to(torch.float8_e4m3fn)
    q4, s4 = fp8_conv_weight("conv", qb, blocks, block_size=(8, 28))
    torch.testing.assert_close(dequantize_fp8(q4, s4, 0),
                               qb.float() * blocks[:, :1].repeat_interleave(8, 0).view(24, 1, 1))
    # varying along the row: requantized per channel, within one E4M3 rounding
    varying = torch.rand(3, 4, generator=gen) * 0.01 + 0.001
    q5, s5 = fp8_conv_weight("conv", q, varying, block_size=(8, 28))
    dense = (q.float().view(24, -1) * varying.repeat_interleave(8, 0).repeat_interleave(28, 1)
             ).view(24, 16, 7)
    err = (dequantize_fp8(q5, s5, 0) - dense).abs() / dense.abs().amax(dim=(1, 2), keepdim=True)
    assert err.max() <= 2 ** -4
    with pytest.raises(TypeError):
        fp8_conv_weight("conv", q, torch.ones(24, dtype=torch.int32))
    with pytest.raises(ValueError):
        fp8_conv_weight("conv", q, torch.tensor([]))
    with pytest.raises(ValueError):
        fp8_conv_weight("conv", q, torch.full((24,), float("inf")))
    with pytest.raises(ValueError):
        fp8_conv_weight("conv", q, torch.zeros(24))


def test_e4m3_weights_in_a_tree_pack_as_they_are():
    gen = torch.Generator().manual_seed(13)
    w = torch.randn(16, 40, 7, generator=gen)
    q, s = quantize_fp8(w, 0)
    packed = pack_conv1d(q, None, fp8=True, scale=s)
    assert packed.weight.dtype == torch.float8_e4m3fn
    exact = q.float().double() * s.double().view(-1, 1, 1)
    torch.testing.assert_close(unpack(packed)[..., :40], exact.permute(0, 2, 1), rtol=0, atol=0)
    wt = torch.randn(32, 8, 12, generator=gen)
    qt, st = quantize_fp8(wt, 1)
    pt = pack_conv_transpose1d(qt, None, stride=6, scale=st)
    x = torch.randn(1, 5, 32, generator=gen)
    got = emulate(x, pt, 5).view(1, 30, 8)
    w_deq = qt.float().double() * st.double().view(1, -1, 1)  # the dequantized values, exactly
    expected = O.causal_conv_transpose1d(x.double().transpose(1, 2), w_deq, None, 6)
    torch.testing.assert_close(got, expected.transpose(1, 2), rtol=1e-9, atol=1e-9)
    tree = {"in_conv": {"weight": q, "weight_scale": s, "bias": None}}
    assert torch.equal(reference_weights(tree, "fp8")["in_conv"]["weight"], dequantize_fp8(q, s, 0))
