"""CPU pins of the oracle (oracle/codec_oracle.py): each oracle function is checked against
something that fixes it independently of its own formula — a brute-force loop, the C direct-sum
restatement (oracle/codec_oracle.c), an installed ``transformers`` module with the same
arithmetic, a closed form or a whole-stream invariant — chosen so that a dropped term, a wrong
sign, index or trim, or a transposed operand fails."""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import codec_oracle as O

REPO = Path(__file__).resolve().parents[1]
ORACLE_LIB = REPO / "oracle" / "_build" / "libcodec_oracle.so"


@pytest.fixture(scope="module")
def clib() -> ctypes.CDLL:
    if not ORACLE_LIB.exists():
        import subprocess

        subprocess.run(["make", "-s", "-C", str(REPO / "oracle")], check=True)
    lib = ctypes.CDLL(str(ORACLE_LIB))
    i64, p = ctypes.c_int64, ctypes.c_void_p
    lib.oracle_rvq_gather_sum.argtypes = [p, i64, i64, i64, p, i64, i64, p, ctypes.c_int]
    lib.oracle_conv1d_f64.argtypes = [p, i64, i64, i64, p, p, i64, i64, i64, i64, p]
    lib.oracle_conv_transpose1d_f64.argtypes = [p, i64, i64, i64, p, p, i64, i64, i64, i64, i64, p]
    return lib


def _np_ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def c_conv1d(lib, x, w, b, dilation, left_pad) -> torch.Tensor:
    x64 = np.ascontiguousarray(x.double().numpy())
    w64 = np.ascontiguousarray(w.double().numpy())
    b64 = None if b is None else np.ascontiguousarray(b.double().numpy())
    batch, c_in, length = x64.shape
    c_out, _, taps = w64.shape
    y = np.zeros((batch, c_out, length))
    lib.oracle_conv1d_f64(_np_ptr(x64), batch, c_in, length, _np_ptr(w64),
                          None if b64 is None else _np_ptr(b64), c_out, taps, dilation, left_pad,
                          _np_ptr(y))
    return torch.from_numpy(y)


def c_conv_transpose1d(lib, x, w, b, stride, padding, out_length) -> torch.Tensor:
    x64 = np.ascontiguousarray(x.double().numpy())
    w64 = np.ascontiguousarray(w.double().numpy())
    b64 = None if b is None else np.ascontiguousarray(b.double().numpy())
    batch, c_in, length = x64.shape
    _, c_out, taps = w64.shape
    y = np.zeros((batch, c_out, out_length))
    lib.oracle_conv_transpose1d_f64(_np_ptr(x64), batch, c_in, length, _np_ptr(w64),
                                    None if b64 is None else _np_ptr(b64), c_out, taps, stride,
                                    padding, out_length, _np_ptr(y))
    return torch.from_numpy(y)


# ------------------------------------------------------------------------------------ a1 RVQ


def test_rvq_matches_a_brute_force_loop():
    gen = torch.Generator().manual_seed(0)
    tables = torch.randn(3, 7, 5, generator=gen)
    codes = torch.randint(0, 7, (2, 3, 4), generator=gen)
    got = O.rvq_gather_sum(codes, tables)
    for b in range(2):
        for t in range(4):
            for d in range(5):
                acc = 0.0
                for k in range(3):
                    acc = float(np.float32(acc) + np.float32(tables[k, codes[b, k, t], d].item()))
                assert got[b, d, t].item() == np.float32(acc)


@pytest.mark.parametrize("clamp", [False, True])
def test_rvq_is_bit_identical_to_the_c_restatement(clib, clamp):
    gen = torch.Generator().manual_seed(1)
    k, v, d, t = 8, 1024, 256, 50
    tables = (torch.randn(k, v, d, generator=gen) * 0.02).contiguous()
    codes = torch.randint(0, v + (40 if clamp else 0), (2, k, t), generator=gen)
    out = np.zeros((2, d, t), dtype=np.float32)
    codes_np = np.ascontiguousarray(codes.numpy().astype(np.int64))
    tables_np = np.ascontiguousarray(tables.numpy())
    clib.oracle_rvq_gather_sum(_np_ptr(codes_np), 2, k, t, _np_ptr(tables_np), v, d, _np_ptr(out),
                               int(clamp))
    src = O.clamp_codes(codes, v) if clamp else codes
    assert torch.equal(O.rvq_gather_sum(src, tables), torch.from_numpy(out))


def test_rvq_with_one_codebook_is_an_embedding_lookup():
    gen = torch.Generator().manual_seed(2)
    tables = torch.randn(1, 33, 12, generator=gen)
    codes = torch.randint(0, 33, (3, 1, 9), generator=gen)
    expected = F.embedding(codes[:, 0], tables[0]).transpose(1, 2)
    assert torch.equal(O.rvq_gather_sum(codes, tables), expected)


def test_rvq_mean_is_the_sum_divided_by_k_and_permutation_changes_only_rounding():
    gen = torch.Generator().manual_seed(3)
    tables = torch.randn(6, 20, 8, generator=gen)
    codes = torch.randint(0, 20, (2, 6, 5), generator=gen)
    total = O.rvq_gather_sum(codes, tables)
    assert torch.equal(O.rvq_gather_sum(codes, tables, mean=True), total / 6)
    perm = torch.tensor([5, 3, 1, 0, 2, 4])
    permuted = O.rvq_gather_sum(codes[:, perm], tables[perm])
    torch.testing.assert_close(permuted, total, rtol=1e-6, atol=1e-6)
    # an exact float64 reference of the unordered sum
    f64 = sum(tables[k].double()[codes[:, k]] for k in range(6)).transpose(1, 2)
    torch.testing.assert_close(total.double(), f64, rtol=1e-6, atol=1e-6)


def test_rvq_code_clamp_reads_the_last_entry():
    tables = torch.arange(2 * 4 * 3, dtype=torch.float32).view(2, 4, 3)
    codes = torch.tensor([[[0, 9], [3, 4]]])
    got = O.rvq_gather_sum(O.clamp_codes(codes, 4), tables)
    assert got[0, :, 1].tolist() == (tables[0, 3] + tables[1, 3]).tolist()


# ---------------------------------------------------------------------------------- a4 Snake


def test_snake_matches_transformers_snake1d_and_the_float64_formula():
    from transformers.models.dac.modeling_dac import Snake1d

    gen = torch.Generator().manual_seed(4)
    x = torch.randn(2, 6, 40, generator=gen) * 3
    alpha = torch.rand(6, generator=gen) * 2 + 0.1
    module = Snake1d(6)
    with torch.no_grad():
        module.alpha.copy_(alpha.view(1, 6, 1))
        expected = module(x)
    got = O.snake(x, alpha)
    assert torch.equal(got, expected)
    a = alpha.double().view(1, 6, 1)
    f64 = x.double() + torch.sin(a * x.double()) ** 2 / (a + 1e-9)
    torch.testing.assert_close(got.double(), f64, rtol=1e-5, atol=1e-5)


def test_snake_limits():
    x = torch.linspace(-2, 2, 41).view(1, 1, -1)
    # x = 0 is a fixed point
    assert O.snake(torch.zeros(1, 3, 5), torch.ones(3)).abs().max().item() == 0.0
    # alpha -> 0: sin(a x)^2 / a -> a x^2 -> 0, so y -> x (and y - x ~ a x^2)
    a = torch.tensor([1e-4])
    y = O.snake(x, a)
    torch.testing.assert_close(y - x, a * x * x, rtol=1e-2, atol=1e-7)
    # the periodic term is non-negative and at most 1/alpha
    alpha = torch.tensor([0.5])
    d = O.snake(x * 10, alpha) - x * 10
    assert d.min().item() >= 0.0 and d.max().item() <= 2.0 + 1e-6


def test_snake_beta_matches_transformers():
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import Qwen3OmniMoeSnakeBeta

    gen = torch.Generator().manual_seed(5)
    x = torch.randn(2, 8, 30, generator=gen) * 2
    alpha_log = torch.randn(8, generator=gen) * 0.3
    beta_log = torch.randn(8, generator=gen) * 0.3
    module = Qwen3OmniMoeSnakeBeta(8)
    with torch.no_grad():
        module.alpha.copy_(alpha_log)
        module.beta.copy_(beta_log)
        expected = module(x)
    torch.testing.assert_close(O.snake_beta(x, alpha_log, beta_log), expected, rtol=1e-6,
                               atol=1e-6)


# ------------------------------------------------------------------------------ a2 / a3 convs


@pytest.mark.parametrize("k,d", [(7, 1), (7, 3), (7, 9), (1, 1), (3, 2)])
def test_causal_conv_matches_c_direct_summation(clib, k, d):
    gen = torch.Generator().manual_seed(10 + k * d)
    x = torch.randn(2, 5, 40, generator=gen)
    w = torch.randn(4, 5, k, generator=gen)
    b = torch.randn(4, generator=gen)
    got = O.causal_conv1d(x, w, b, d)
    expected = c_conv1d(clib, x, w, b, d, (k - 1) * d)
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("k,d", [(3, 1), (7, 3), (11, 5)])
def test_same_conv_matches_c_direct_summation(clib, k, d):
    gen = torch.Generator().manual_seed(20 + k)
    x = torch.randn(1, 4, 50, generator=gen)
    w = torch.randn(3, 4, k, generator=gen)
    got = O.same_conv1d(x, w, None, d)
    expected = c_conv1d(clib, x, w, None, d, (k * d - d) // 2)
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("stride", [2, 5, 6, 8])
def test_causal_transposed_conv_matches_c_scatter_and_keeps_t_times_s(clib, stride):
    gen = torch.Generator().manual_seed(30 + stride)
    x = torch.randn(2, 6, 9, generator=gen)
    w = torch.randn(6, 3, 2 * stride, generator=gen)
    b = torch.randn(3, generator=gen)
    got = O.causal_conv_transpose1d(x, w, b, stride)
    assert got.shape[-1] == 9 * stride
    expected = c_conv_transpose1d(clib, x, w, b, stride, 0, 9 * stride)
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rate,k", [(8, 16), (5, 11), (3, 7), (4, 8)])
def test_padded_transposed_conv_matches_c_scatter(clib, rate, k):
    gen = torch.Generator().manual_seed(40 + k)
    x = torch.randn(1, 4, 7, generator=gen)
    w = torch.randn(4, 2, k, generator=gen)
    got = O.padded_conv_transpose1d(x, w, None, rate)
    assert got.shape[-1] == 7 * rate
    expected = c_conv_transpose1d(clib, x, w, None, rate, (k - rate) // 2, 7 * rate)
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-5)


def test_causal_transposed_conv_is_the_qwen3_both_sides_trim_shifted_by_s():
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import (
        Qwen3OmniMoeCausalTransConvNet,
    )

    gen = torch.Generator().manual_seed(6)
    x = torch.randn(1, 4, 10, generator=gen)
    module = Qwen3OmniMoeCausalTransConvNet(4, 3, 10, 5)
    with torch.no_grad():
        q = module(x)
        ours = O.causal_conv_transpose1d(x, module.conv.weight, module.conv.bias, 5)
    torch.testing.assert_close(ours[..., 5:], q)


# -------------------------------------------------------------------------- a5 composition


def _unit(gen, c, dilation) -> dict:
    return {
        "dilation": dilation,
        "alpha1": torch.rand(c, generator=gen) + 0.5,
        "conv1": {"weight": torch.randn(c, c, 7, generator=gen) * 0.2,
                  "bias": torch.randn(c, generator=gen) * 0.1},
        "alpha2": torch.rand(c, generator=gen) + 0.5,
        "conv2": {"weight": torch.randn(c, c, 1, generator=gen) * 0.2,
                  "bias": torch.randn(c, generator=gen) * 0.1},
    }


def _load_qwen3_unit(module, unit):
    # SnakeBeta with alpha = beta = log(a) is Snake1d(a): exp(log a) = a up to rounding
    with torch.no_grad():
        module.act1.alpha.copy_(unit["alpha1"].log())
        module.act1.beta.copy_(unit["alpha1"].log())
        module.act2.alpha.copy_(unit["alpha2"].log())
        module.act2.beta.copy_(unit["alpha2"].log())
        module.conv1.conv.weight.copy_(unit["conv1"]["weight"])
        module.conv1.conv.bias.copy_(unit["conv1"]["bias"])
        module.conv2.conv.weight.copy_(unit["conv2"]["weight"])
        module.conv2.conv.bias.copy_(unit["conv2"]["bias"])


@pytest.mark.parametrize("dilation", [1, 3, 9])
def test_residual_unit_matches_the_causal_qwen3_residual_unit(dilation):
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import (
        Qwen3OmniMoeCode2WavDecoderResidualUnit,
    )

    gen = torch.Generator().manual_seed(50 + dilation)
    unit = _unit(gen, 6, dilation)
    module = Qwen3OmniMoeCode2WavDecoderResidualUnit(6, dilation)
    _load_qwen3_unit(module, unit)
    x = torch.randn(2, 6, 37, generator=gen)
    with torch.no_grad():
        expected = module(x)
    torch.testing.assert_close(O.residual_unit(x, unit), expected, rtol=1e-5, atol=1e-5)


def test_the_residual_unit_pin_rejects_the_conv_before_snake_order():
    # a plausible transposition (conv -> Snake instead of Snake -> conv) fails the pin above
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import (
        Qwen3OmniMoeCode2WavDecoderResidualUnit,
    )

    gen = torch.Generator().manual_seed(60)
    unit = _unit(gen, 4, 1)
    module = Qwen3OmniMoeCode2WavDecoderResidualUnit(4, 1)
    _load_qwen3_unit(module, unit)
    x = torch.randn(1, 4, 20, generator=gen)
    with torch.no_grad():
        expected = module(x)
    swapped = x + O.snake(O.causal_conv1d(O.snake(O.causal_conv1d(
        x, unit["conv1"]["weight"], unit["conv1"]["bias"]), unit["alpha1"]),
        unit["conv2"]["weight"], unit["conv2"]["bias"]), unit["alpha2"])
    assert not torch.allclose(swapped, expected, atol=1e-3)


@pytest.mark.parametrize("pad", [1, 2, 3, 4, 5])
def test_residual_trim_known_answers(pad):
    """modded_dac.py:633-640: a causal unit keeps x's first L - pad samples (``x[..., :-pad]``);
    a non-causal one centres them, floor(pad / 2) dropped on the left and ceil(pad / 2) on the
    right (``x[..., pad // 2 : -pad // 2]``)."""
    x = torch.arange(20.0).view(1, 1, 20)
    assert O.residual_trim(x, 20 - pad, "causal").flatten().tolist() == list(range(20 - pad))
    assert O.residual_trim(x, 20 - pad, "same").flatten().tolist() == \
        list(range(pad // 2, 20 - (pad + 1) // 2))
    assert O.residual_trim(x, 20, "causal") is x and O.residual_trim(x, 20, "same") is x


def test_residual_unit_cuts_x_to_a_shorter_branch():
    """A non-causal unit whose k = 6 conv returns one sample fewer than x adds the branch to
    x[..., :-1] (pad 1: x[..., 0 : -1]), the branch evaluated here with plain conv1d."""
    gen = torch.Generator().manual_seed(61)
    unit = _unit(gen, 4, 1)
    unit["conv1"]["weight"] = torch.randn(4, 4, 6, generator=gen) * 0.2
    x = torch.randn(1, 4, 21, generator=gen)
    y = O.snake(x, unit["alpha1"])
    y = F.conv1d(y, unit["conv1"]["weight"], unit["conv1"]["bias"], padding=2)
    y = O.snake(y, unit["alpha2"])
    y = F.conv1d(y, unit["conv2"]["weight"], unit["conv2"]["bias"])
    assert y.shape[-1] == 20
    torch.testing.assert_close(O.residual_unit(x, unit, "same"), x[..., :20] + y)


def test_decoder_block_matches_the_qwen3_block_up_to_the_trim():
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import (
        Qwen3OmniMoeCode2WavConfig,
        Qwen3OmniMoeCode2WavDecoderBlock,
    )

    gen = torch.Generator().manual_seed(70)
    cfg = Qwen3OmniMoeCode2WavConfig(decoder_dim=16, upsample_rates=[4], hidden_size=16,
                                     codebook_size=8, num_quantizers=2)
    module = Qwen3OmniMoeCode2WavDecoderBlock(cfg, 0).eval()
    c_in, c_out, s = 16, 8, 4
    block = {
        "stride": s,
        "alpha": torch.rand(c_in, generator=gen) + 0.5,
        "up": {"weight": torch.randn(c_in, c_out, 2 * s, generator=gen) * 0.2,
               "bias": torch.randn(c_out, generator=gen) * 0.1},
        "units": [_unit(gen, c_out, d) for d in (1, 3, 9)],
    }
    with torch.no_grad():
        module.block[0].alpha.copy_(block["alpha"].log())
        module.block[0].beta.copy_(block["alpha"].log())
        module.block[1].conv.weight.copy_(block["up"]["weight"])
        module.block[1].conv.bias.copy_(block["up"]["bias"])
        for i, unit in enumerate(block["units"]):
            _load_qwen3_unit(module.block[2 + i], unit)
    x = torch.randn(1, c_in, 12, generator=gen)
    with torch.no_grad():
        q = module(x)
    ours = O.decoder_block(x, block)
    assert ours.shape[-1] == 12 * s and q.shape[-1] == 11 * s
    # Qwen3 trims k - s samples on both sides of the transposed conv, the causal DAC block only on
    # the right, so the Qwen3 block is the same residual units run on the DAC upsampler's output
    # from sample s on.
    up = O.causal_conv_transpose1d(O.snake(x, block["alpha"]), block["up"]["weight"],
                                   block["up"]["bias"], s)

    def units(y):
        for unit in block["units"]:
            y = O.residual_unit(y, unit)
        return y

    torch.testing.assert_close(units(up[..., s:]), q, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ours, units(up))


def test_hifigan_generator_matches_transformers_speecht5_hifigan():
    from transformers import SpeechT5HifiGan, SpeechT5HifiGanConfig

    cfg = SpeechT5HifiGanConfig(model_in_dim=10, upsample_initial_channel=16,
                                upsample_rates=[2, 3], upsample_kernel_sizes=[4, 7],
                                resblock_kernel_sizes=[3, 7, 11],
                                resblock_dilation_sizes=[[1, 3, 5]] * 3, leaky_relu_slope=0.1,
                                normalize_before=False)
    torch.manual_seed(0)
    module = SpeechT5HifiGan(cfg).eval()
    with torch.no_grad():
        for p in module.parameters():
            p.normal_(0, 0.2)
    weights = {
        "slope": 0.1,
        "final_slope": 0.01,
        "conv_pre": {"weight": module.conv_pre.weight, "bias": module.conv_pre.bias},
        "stages": [],
        "conv_post": {"weight": module.conv_post.weight, "bias": module.conv_post.bias},
    }
    for i, (rate, up) in enumerate(zip(cfg.upsample_rates, module.upsampler)):
        stage = {"rate": rate, "up": {"weight": up.weight, "bias": up.bias}, "resblocks": []}
        for j in range(3):
            rb = module.resblocks[i * 3 + j]
            stage["resblocks"].append({
                "dilations": (1, 3, 5),
                "convs1": [{"weight": c.weight, "bias": c.bias} for c in rb.convs1],
                "convs2": [{"weight": c.weight, "bias": c.bias} for c in rb.convs2],
            })
        weights["stages"].append(stage)
    mel = torch.randn(2, 13, 10)
    with torch.no_grad():
        expected = module(mel)  # [B, T * 6]
        got = O.hifigan_generator(mel.transpose(1, 2), weights)
    torch.testing.assert_close(got[:, 0], expected, rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------- a6 final conv


def test_clamped_single_output_conv_is_the_float64_conv_clamped(clib):
    gen = torch.Generator().manual_seed(80)
    padded = torch.randn(2, 30 + 6, 8, generator=gen)
    w = torch.randn(1, 8, 7, generator=gen)
    b = torch.randn(1, generator=gen)
    got = O.clamped_single_output_conv(padded, w, b, 30)
    direct = c_conv1d(clib, padded.transpose(1, 2), w, b, 1, 0)[..., :30]
    assert torch.equal(got, direct.clamp(-1, 1))
    assert got.abs().max().item() <= 1.0


# ------------------------------------------------------------------------- a7 streaming


@pytest.mark.parametrize("splits", [(5, 7, 9), (1,) * 12 + (9,), (21,)])
@pytest.mark.parametrize("history", [6, 18, 54])
def test_history_exchange_reference_builds_the_whole_stream_causal_window(splits, history):
    gen = torch.Generator().manual_seed(90 + history)
    stream = torch.randn(2, sum(splits), 3, generator=gen)
    pool = torch.zeros(4, history, 3)
    slot = torch.tensor([2, 0])
    whole = F.pad(stream, (0, 0, history, 0))
    pos = 0
    for i, n in enumerate(splits):
        padded = torch.full((2, history + n + 2, 3), float("nan"))
        padded[:, history:history + n] = stream[:, pos:pos + n]
        O.history_exchange_reference(padded, pool, slot, n, i == 0)
        assert torch.equal(padded[:, :history + n], whole[:, pos:pos + history + n])
        assert torch.equal(padded[:, history + n:], torch.zeros(2, 2, 3))
        pos += n


@pytest.mark.parametrize("stride", [2, 5, 8])
def test_streamed_transposed_conv_with_overlap_reference_equals_whole(stride):
    gen = torch.Generator().manual_seed(100 + stride)
    k = 2 * stride
    x = torch.randn(1, 4, 17, generator=gen)
    w = torch.randn(4, 3, k, generator=gen)
    whole = F.conv_transpose1d(x, w, stride=stride)  # (T-1)s + k samples
    pool = torch.zeros(2, k - stride, 3)
    slot = torch.tensor([1])
    outs = []
    pos = 0
    for i, n in enumerate((4, 1, 7, 5)):
        full = F.conv_transpose1d(x[..., pos:pos + n], w, stride=stride)  # [1, 3, (n+1)s]
        chunk = full.transpose(1, 2).contiguous()
        O.overlap_exchange_reference(chunk, pool, slot, n * stride, i == 0)
        outs.append(chunk[:, :n * stride])
        pos += n
    streamed = torch.cat(outs, dim=1).transpose(1, 2)
    torch.testing.assert_close(streamed, whole[..., :17 * stride], rtol=1e-5, atol=1e-5)


def test_decoder_split_decodes_equal_the_whole_decode():
    """Causality of the oracle decoder: output sample i depends only on frames <= i / hop."""
    from sglang_omni_amd.models.configs import DacDecoderConfig, make_dac_weights

    cfg = DacDecoderConfig(n_codebooks=2, codebook_size=16, latent_dim=16, channels=32,
                           rates=(2, 3))
    weights = make_dac_weights(cfg, seed=1)
    codes = torch.randint(0, 16, (1, 2, 10), generator=torch.Generator().manual_seed(3))
    whole = O.dac_from_indices(codes, weights)
    prefix = O.dac_from_indices(codes[..., :6], weights)
    torch.testing.assert_close(whole[..., :6 * cfg.hop_length], prefix, rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------------------- a8 fp8


def test_fp8_per_channel_quantization():
    gen = torch.Generator().manual_seed(110)
    w = torch.randn(6, 5, 7, generator=gen) * torch.logspace(-3, 0, 6).view(6, 1, 1)
    q, s = O.quantize_fp8_per_channel(w)
    assert q.dtype == torch.float8_e4m3fn and s.shape == (6,)
    # each channel's largest magnitude maps to 448 exactly
    assert torch.equal(q.float().reshape(6, -1).abs().amax(1), torch.full((6,), 448.0))
    deq = O.dequantize_fp8_per_channel(q, s)
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 for normal values
    rel = ((deq - w).abs() / w.abs().clamp_min(1e-30))
    normal = w.abs() >= s.view(6, 1, 1) * 2.0 ** -6
    assert rel[normal].max().item() <= 2.0 ** -4 + 1e-7
    assert torch.equal(O.dequantize_fp8_per_channel(*O.quantize_fp8_per_channel(deq)), deq)


def test_snr_db():
    ref = torch.ones(100)
    assert O.snr_db(ref, ref) == math.inf
    # noise at 1 % of the signal amplitude is 40 dB (1.01 is inexact in float32)
    assert abs(O.snr_db(ref, ref * 1.01) - 40.0) < 1e-4
    assert abs(O.snr_db(ref, ref * 1.1) - 20.0) < 1e-4


# ------------------------------------------------------------------ HiFT iSTFT tail


def test_hann_window_is_scipys_periodic_hann():
    from scipy.signal import get_window

    for n in (8, 16, 32):
        assert torch.equal(O.hann_window(n),
                           torch.from_numpy(get_window("hann", n, fftbins=True).astype("float32")))


@pytest.mark.parametrize("n_fft,hop,length", [(16, 4, 101), (16, 4, 9), (32, 8, 257), (8, 2, 40)])
def test_stft_reference_is_torch_stft(n_fft, hop, length):
    gen = torch.Generator().manual_seed(n_fft + length)
    x = torch.randn(3, length, generator=gen, dtype=torch.float64)
    w = O.hann_window(n_fft)
    spec = O.stft_reference(x, w, n_fft, hop)
    ref = torch.stft(x, n_fft, hop, n_fft, window=w.double(), return_complex=True)
    bins = n_fft // 2 + 1
    torch.testing.assert_close(spec[:, :bins], ref.real, rtol=0, atol=1e-12)
    torch.testing.assert_close(spec[:, bins:], ref.imag, rtol=0, atol=1e-12)


@pytest.mark.parametrize("n_fft,hop,frames", [(16, 4, 26), (16, 4, 3), (32, 8, 40)])
def test_istft_reference_is_torch_istft(n_fft, hop, frames):
    gen = torch.Generator().manual_seed(frames)
    bins = n_fft // 2 + 1
    re = torch.randn(2, bins, frames, generator=gen, dtype=torch.float64)
    im = torch.randn(2, bins, frames, generator=gen, dtype=torch.float64)
    im[:, 0] = 0  # a real signal's DC and Nyquist bins are real
    im[:, -1] = 0
    w = O.hann_window(n_fft)
    y = O.istft_reference(re, im, w, n_fft, hop)
    ref = torch.istft(torch.complex(re, im), n_fft, hop, n_fft, window=w.double())
    torch.testing.assert_close(y, ref, rtol=0, atol=1e-12)


def test_istft_of_stft_reconstructs_the_signal():
    """The Hann window at hop n_fft / 4 overlap-adds to a constant: istft(stft(x)) = x."""
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(2, 400, generator=gen, dtype=torch.float64)
    w = O.hann_window(16)
    spec = O.stft_reference(x, w, 16, 4)
    y = O.istft_reference(spec[:, :9], spec[:, 9:], w, 16, 4)
    torch.testing.assert_close(y, x[:, :y.shape[1]], rtol=0, atol=1e-12)


def test_stft_reference_dc_and_nyquist_bins():
    """The periodic Hann window's DFT is N/2 at bin 0 and -N/4 at bins +-1 (w = 1/2 - cos / 2):
    a constant signal gives X[0] = N/2, X[1] = -N/4 and nothing else; an alternating one
    |X[N/2]| = N/2, |X[N/2 - 1]| = N/4 and nothing else (frames clear of the reflected edges;
    the float32 window rounds at 1e-7)."""
    n = 16
    w = O.hann_window(n)
    mid = O.stft_reference(torch.ones(1, 64, dtype=torch.float64), w, n, 4)[0, :, 4:-4]
    torch.testing.assert_close(mid[0], torch.full_like(mid[0], n / 2), rtol=0, atol=1e-6)
    torch.testing.assert_close(mid[1], torch.full_like(mid[1], -n / 4), rtol=0, atol=1e-6)
    assert mid[2:].abs().max().item() < 1e-6
    alt = (-1.0) ** torch.arange(64, dtype=torch.float64)[None]
    spec = O.stft_reference(alt, w, n, 4)[0, :, 4:-4]
    bins = n // 2 + 1
    mag = torch.sqrt(spec[:bins] ** 2 + spec[bins:] ** 2)
    torch.testing.assert_close(mag[n // 2], torch.full_like(mag[0], n / 2), rtol=0, atol=1e-6)
    torch.testing.assert_close(mag[n // 2 - 1], torch.full_like(mag[0], n / 4), rtol=0, atol=1e-6)
    assert mag[:n // 2 - 1].abs().max().item() < 1e-6


def test_hift_tail_reference_clips_and_clamps():
    """Magnitudes above the clip count as the clip; the output never leaves +-audio_limit, and
    small inputs pass through unclamped (equal to the unclamped inverse)."""
    gen = torch.Generator().manual_seed(4)
    n_fft, hop, bins = 16, 4, 9
    h = torch.randn(2, 30, 2 * bins, generator=gen, dtype=torch.float64)
    h[..., :bins] = h[..., :bins] * 0.5 - 4.0  # magnitudes around e^-4
    w = O.hann_window(n_fft)
    y = O.hift_istft_tail(h, w, n_fft, hop)
    mag = torch.exp(h[..., :bins]).transpose(1, 2)
    ph = torch.sin(h[..., bins:]).transpose(1, 2)
    free = O.istft_reference(mag * torch.cos(ph), mag * torch.sin(ph), w, n_fft, hop)
    assert free.abs().max().item() < 0.99
    torch.testing.assert_close(y, free, rtol=0, atol=0)
    h2 = h.clone()
    h2[..., :bins] = 10.0  # exp(10) > 100: clipped to 100
    y2 = O.hift_istft_tail(h2, w, n_fft, hop)
    h3 = h2.clone()
    h3[..., :bins] = math.log(100.0)
    torch.testing.assert_close(y2, O.hift_istft_tail(h3, w, n_fft, hop), rtol=0, atol=1e-12)
    assert y2.abs().max().item() <= 0.99


# ------------------------------------------------------------------------------ host egress


def test_pcm16_encode_known_answers():
    """Hand-computed codes of the clip / scale-by-32767 / truncate encoding: a rounding encoder
    (0.5 -> 16384), a 32768 scale (1.0 -> overflow), a missing clip or a floor (negative
    half-scale -> -16384) each fails one of them."""
    x = torch.tensor([0.0, 1.0, -1.0, 0.5, -0.5, 0.99999, -0.99999, 1.0 / 32767, 0.9 / 32767,
                      -0.9 / 32767, 2.0, -7.5, float("inf"), float("-inf"), float("nan"),
                      0.25, -0.000030517578125], dtype=torch.float32)
    expected = [0, 32767, -32767, 16383, -16383, 32766, -32766, 1, 0, 0, 32767, -32767, 32767,
                -32767, 0, 8191, 0]
    got = O.pcm16_encode(x)
    assert got.dtype == torch.int16
    assert got.tolist() == expected


def test_pcm16_encode_matches_numpy_cast():
    """numpy's own float32 -> int16 cast of the clipped product (the reference encoder's
    arithmetic, session_bridge.py:86-88) on finite samples, bit for bit."""
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(50_000, generator=g) * 0.7).float()
    x[::97] *= 3.0
    ref = (np.clip(x.numpy(), -1.0, 1.0) * (32768 - 1)).astype("<i2")
    assert np.array_equal(O.pcm16_encode(x).numpy(), ref)


def test_waveform_egress_reference_trims_rows():
    wave = torch.arange(24, dtype=torch.float32).view(3, 1, 8) / 32.0
    rows = O.waveform_egress_reference(wave, [8, 3, 0])
    assert [r.numel() for r in rows] == [8, 3, 0]
    assert torch.equal(rows[1], wave[1, 0, :3])
    pcm = O.waveform_egress_reference(wave, None, format="pcm16")
    assert pcm[2].tolist() == [int(v / 32.0 * 32767) for v in range(16, 24)]


# ------------------------------------------------------------------------------ MOSS channel sum


def test_channel_embedding_sum_pins():
    g = torch.Generator().manual_seed(9)
    tables = [torch.randn(v, 16, generator=g) for v in (5, 7, 3)]
    ids = torch.tensor([[0, 6, 2], [4, 0, 1], [-1, 7, 2], [2, 3, 99]])
    # one channel: the lookup itself (out-of-range rows are zero)
    one = O.channel_embedding_sum(ids[:, :1], tables[:1])
    assert torch.equal(one[:2], tables[0][ids[:2, 0]]) and torch.equal(one[2], torch.zeros(16))
    # float32 tables, ids in range: the ordered float32 sum of the RVQ gather-sum
    inr = torch.tensor([[0, 6, 2], [4, 0, 1], [1, 1, 0]])
    books = torch.stack([t[:3] for t in tables])  # equal-size tables for the RVQ form
    ids3 = inr.clamp(max=2)
    rvq = O.rvq_gather_sum(ids3.t()[None], books)[0].t()
    assert torch.equal(O.channel_embedding_sum(ids3, [t[:3] for t in tables]), rvq)
    # bf16, two channels: round(a + b) with a, b exact in bf16
    bt = [t.to(torch.bfloat16) for t in tables[:2]]
    got = O.channel_embedding_sum(inr[:, :2], bt)
    ref = (bt[0][inr[:, 0]].float() + bt[1][inr[:, 1]].float()).to(torch.bfloat16)
    assert torch.equal(got, ref)


# ------------------------------------------------------------------------------------------
# The whole DAC decoder composition against transformers' DacDecoder
# ------------------------------------------------------------------------------------------


def _tf_dac_decoder(seed: int):
    """transformers' DacDecoder (the dac library's decoder restated: conv -> blocks of Snake ->
    ConvTranspose -> residual units -> Snake -> conv -> tanh, non-causal padding) with random
    Snake alphas and conv weights scaled to keep the output inside tanh's linear range."""
    from transformers.models.dac.configuration_dac import DacConfig
    from transformers.models.dac.modeling_dac import DacDecoder

    cfg = DacConfig(hidden_size=12, decoder_hidden_size=32, upsampling_ratios=[2, 3, 4])
    torch.manual_seed(seed)
    dec = DacDecoder(cfg).eval()
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for m in dec.modules():
            if hasattr(m, "alpha"):
                m.alpha.copy_(torch.rand(m.alpha.shape, generator=gen) * 1.5 + 0.3)
            if isinstance(m, (torch.nn.Conv1d, torch.nn.ConvTranspose1d)):
                fan_in = m.weight.shape[1 if isinstance(m, torch.nn.Conv1d) else 0] * m.weight.shape[2]
                m.weight.copy_(torch.randn(m.weight.shape, generator=gen) * 0.7 / math.sqrt(fan_in))
                m.bias.copy_(torch.randn(m.bias.shape, generator=gen) * 0.05)
    return dec


def _weights_of_tf_decoder(dec) -> dict:
    """The oracle's weight tree of a transformers DacDecoder, read attribute by attribute."""

    def conv(m):
        return {"weight": m.weight.detach().clone(), "bias": m.bias.detach().clone()}

    def alpha(m):
        return m.alpha.detach().reshape(-1).clone()

    blocks = []
    for blk in dec.block:
        units = [{"alpha1": alpha(ru.snake1), "conv1": conv(ru.conv1),
                  "dilation": ru.conv1.dilation[0], "alpha2": alpha(ru.snake2),
                  "conv2": conv(ru.conv2)}
                 for ru in (blk.res_unit1, blk.res_unit2, blk.res_unit3)]
        blocks.append({"alpha": alpha(blk.snake1), "up": conv(blk.conv_t1),
                       "stride": blk.conv_t1.stride[0], "units": units})
    return {"in_conv": conv(dec.conv1), "blocks": blocks,
            "final": {"alpha": alpha(dec.snake1), "conv": conv(dec.conv2)}}


def test_dac_decoder_composition_matches_transformers_dac_decoder():
    """dac_decoder(padding="same") equals DacDecoder end to end (float64 activations on both
    sides, odd and even strides, the odd one giving T * s - 1 samples); the causal mode runs the
    same composition with the causal pad / trim rules pinned by the conv tests above. The only
    difference is the oracle's float32 Snake coefficient 1 / (alpha + 1e-9), as the reference's
    float32 Snake1d computes it: a relative 1e-7 per Snake, far below any composition mistake
    (the mutation test below)."""
    dec = _tf_dac_decoder(80).double()
    weights = _weights_of_tf_decoder(dec)
    z = torch.randn(2, 12, 9, generator=torch.Generator().manual_seed(81), dtype=torch.float64)
    with torch.no_grad():
        expected = dec(z)
    ours = O.dac_decoder(z, weights, padding="same")
    assert ours.shape == expected.shape == (2, 1, ((9 * 2) * 3 - 1) * 4)
    rms = expected.pow(2).mean().sqrt().item()
    assert 0.02 < rms < 0.5, rms  # inside tanh's linear range, far from zero
    torch.testing.assert_close(ours, expected, rtol=1e-6, atol=1e-7)
    causal = O.dac_decoder(z, weights)
    assert causal.shape == (2, 1, 9 * 2 * 3 * 4)


@pytest.mark.parametrize("mutation", ["no_final_snake", "no_tanh", "units_reordered",
                                      "no_block_snake", "blocks_share_alpha"])
def test_the_decoder_pin_fails_for_a_miscomposed_decoder(mutation):
    """Each plausible composition mistake, made on the reference side, moves the output far
    outside the pin's tolerance: the pin would catch the same mistake in the oracle."""
    dec = _tf_dac_decoder(82).double()
    weights = _weights_of_tf_decoder(dec)
    z = torch.randn(1, 12, 7, generator=torch.Generator().manual_seed(83), dtype=torch.float64)
    with torch.no_grad():
        if mutation == "no_final_snake":
            dec.snake1 = torch.nn.Identity()
        elif mutation == "no_tanh":
            dec.tanh = torch.nn.Identity()
        elif mutation == "units_reordered":
            b = dec.block[1]
            b.res_unit1, b.res_unit2 = b.res_unit2, b.res_unit1
        elif mutation == "no_block_snake":
            dec.block[2].snake1 = torch.nn.Identity()
        else:
            dec.block[0].snake1.alpha.copy_(dec.block[0].snake1.alpha.mean().expand_as(
                dec.block[0].snake1.alpha))
        mutated = dec(z)
    ours = O.dac_decoder(z, weights, padding="same")
    assert (ours - mutated).abs().max().item() > 1e-4
