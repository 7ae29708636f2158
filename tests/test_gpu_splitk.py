"""Split-K convs (``omni_conv1d_splitk``): k = 1, the GEMMs of the code2wav pre-transformer and
ConvNeXt blocks (the reference's ``F.linear`` calls, sglang_omni/models/qwen3_omni/components/
code2wav.py:266,311,318,322), and k = 7 with its slot history and output Snake, a decoder's input
conv over a streaming step (``CausalConvNet``, modded_dac.py:566-572):

* every tile of the LDS-DMA k = 1 list, forced, at 2 and 4 slices, against the float64 GEMM of
  the same bf16 operands (float32 output: float32-summation tolerance);
* a row gives the same bits whatever batch it runs in (the summation order depends on C_in and
  the slice count only): rows decoded 3, 36 and 36 at a time equal the 75-row launch;
* the split form refuses what it does not take, and a workspace that is too small;
* k = 7: every tile of its split list, forced, against the float64 causal conv + bias + Snake;
  a stream decoded in chunks through its slot history equals the whole stream bit for bit.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import (
    _conv_args,
    gemm,
    pack_conv1d,
    splitk_conv,
    splitk_workspace_elements,
)

pytestmark = pytest.mark.gpu

SPLIT_TILES = 4  # entries of the k = 1 LDS-DMA list


def operands(rows, c_in, c_out, seed, gpu):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, rows, c_in, generator=gen)).to(torch.bfloat16)
    w = (torch.randn(c_out, c_in, 1, generator=gen) / c_in ** 0.5).to(torch.bfloat16).float()
    b = (torch.randn(c_out, generator=gen) * 0.1).to(torch.bfloat16).float()
    return x.to(gpu), w, b


@pytest.mark.parametrize("splits", [2, 4])
@pytest.mark.parametrize("config", range(1, SPLIT_TILES + 1))
def test_each_split_tile_matches_the_float64_gemm(gpu, config, splits):
    rows, c_in, c_out = 300, 768, 384
    x, w, b = operands(rows, c_in, c_out, 10 * config + splits, gpu)
    packed = pack_conv1d(w, b).to(gpu)
    ws = torch.empty(splitk_workspace_elements(x, packed, splits), device=gpu)
    out = torch.empty(1, rows, c_out, device=gpu)
    gemm(x, packed, out, k_splits=splits, workspace=ws, kernel=N.CONV_KERNEL_DMA, config=config)
    ref = x.double().cpu()[0] @ w[:, :, 0].double().t() + b.double()
    scale = ref.abs().max().item()
    torch.testing.assert_close(out[0].cpu().double(), ref, rtol=1e-5, atol=1e-5 * scale)


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_a_row_gives_the_same_bits_in_any_batch(gpu, splits):
    x, w, b = operands(75, 1024, 1024, 3, gpu)
    packed = pack_conv1d(w, b).to(gpu)
    ws = torch.empty(splitk_workspace_elements(x, packed, splits), device=gpu)
    whole = torch.empty(1, 75, 1024, dtype=torch.bfloat16, device=gpu)
    gemm(x, packed, whole, k_splits=splits, workspace=ws)
    parts = []
    for a, c in ((0, 3), (3, 39), (39, 75)):
        o = torch.empty(1, c - a, 1024, dtype=torch.bfloat16, device=gpu)
        gemm(x[:, a:c].contiguous(), packed, o, k_splits=splits, workspace=ws)
        parts.append(o)
    assert torch.equal(torch.cat(parts, dim=1), whole)


def test_split_form_refusals(gpu):
    x, w, b = operands(40, 256, 128, 5, gpu)
    packed = pack_conv1d(w, b).to(gpu)
    out = torch.empty(1, 40, 128, dtype=torch.bfloat16, device=gpu)
    need = splitk_workspace_elements(x, packed, 2)
    with pytest.raises(ValueError):  # workspace too small
        gemm(x, packed, out, k_splits=2, workspace=torch.empty(need - 1, device=gpu))
    lib = N.load_library()
    ws = torch.empty(need, device=gpu)
    resid = torch.zeros(1, 40, 128, device=gpu)
    args = _conv_args(x, packed, out, residual=resid)
    status = lib.omni_conv1d_splitk(ctypes.byref(args), 2, ws.data_ptr(), ws.numel() * 4,
                                    N.CONV_KERNEL_AUTO, 0, N.stream_handle(gpu))
    assert status == N.UNSUPPORTED  # a residual is not part of the split form
    args = _conv_args(x, packed, out)
    status = lib.omni_conv1d_splitk(ctypes.byref(args), 3, ws.data_ptr(), ws.numel() * 4,
                                    N.CONV_KERNEL_AUTO, 0, N.stream_handle(gpu))
    assert status == N.UNSUPPORTED  # 256 input channels are not 3 slices of whole chunks
    status = lib.omni_conv1d_splitk(ctypes.byref(args), 2, ws.data_ptr(), 16,
                                    N.CONV_KERNEL_AUTO, 0, N.stream_handle(gpu))
    assert status == N.INVALID_ARG  # workspace_bytes below the partials' size


SPLIT7_TILES = 2  # entries of the k = 7 LDS-DMA split list


def conv7_operands(batch, length, c_in, c_out, seed):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(batch, length, c_in, generator=gen)).to(torch.bfloat16)
    w = (torch.randn(c_out, c_in, 7, generator=gen) / (7 * c_in) ** 0.5).to(torch.bfloat16).float()
    b = (torch.randn(c_out, generator=gen) * 0.1).float()
    alpha = (torch.rand(c_out, generator=gen) + 0.5).float()
    return x, w, b, alpha


def causal_conv_snake_f64(x, w, b, alpha):
    """float64 causal conv (left pad 6) + bias, then Snake(alpha): [B, L, C_out]."""
    xd = torch.nn.functional.pad(x.double().transpose(1, 2), (6, 0))
    y = torch.nn.functional.conv1d(xd, w.double(), b.double()).transpose(1, 2)
    a = alpha.double()
    return y + (a + 1e-9).reciprocal() * torch.sin(a * y) ** 2


@pytest.mark.parametrize("splits", [2, 4])
@pytest.mark.parametrize("config", range(1, SPLIT7_TILES + 1))
def test_each_k7_split_tile_matches_the_float64_conv(gpu, config, splits):
    batch, length, c_in, c_out = 6, 40, 512, 384
    x, w, b, alpha = conv7_operands(batch, length, c_in, c_out, 20 * config + splits)
    packed = pack_conv1d(w, b).to(gpu)
    xg = x.to(gpu)
    ws = torch.empty(splitk_workspace_elements(xg, packed, splits), device=gpu)
    out = torch.empty(batch, length, c_out, device=gpu)
    a = alpha.to(gpu)
    splitk_conv(xg, packed, out, k_splits=splits, workspace=ws, kernel=N.CONV_KERNEL_DMA,
                config=config, activation=N.ACT_SNAKE, act_a=a, act_b=(a + 1e-9).reciprocal())
    ref = causal_conv_snake_f64(x, w, b, alpha)
    scale = ref.abs().max().item()
    torch.testing.assert_close(out.cpu().double(), ref, rtol=1e-5, atol=1e-5 * scale)


@pytest.mark.parametrize("splits", [2, 4])
def test_k7_split_stream_in_chunks_equals_the_whole(gpu, splits):
    """Rows decoded in chunks through the slot history (chunks shorter than the six-sample context
    included) give the whole rows' bits; the rows sit in shuffled slots of a larger pool."""
    batch, c_in, c_out = 5, 512, 256
    chunks = (12, 3, 12, 25)
    length = sum(chunks)
    x, w, b, alpha = conv7_operands(batch, length, c_in, c_out, 31 + splits)
    packed = pack_conv1d(w, b).to(gpu)
    xg = x.to(gpu)
    a = alpha.to(gpu)
    act = dict(activation=N.ACT_SNAKE, act_a=a, act_b=(a + 1e-9).reciprocal())
    ws = torch.empty(splitk_workspace_elements(xg, packed, splits), device=gpu)
    whole = torch.empty(batch, length, c_out, dtype=torch.bfloat16, device=gpu)
    splitk_conv(xg, packed, whole, k_splits=splits, workspace=ws, **act)
    slots = 9
    hist = torch.randn(slots, 2, 6, c_in, device=gpu).to(torch.bfloat16)  # a cold start ignores it
    parity = torch.zeros(slots, dtype=torch.int64, device=gpu)
    slot_index = torch.tensor([7, 2, 0, 5, 3], device=gpu)
    parts, start = [], 0
    for n, size in enumerate(chunks):
        xc = xg[:, start:start + size].contiguous()
        o = torch.empty(batch, size, c_out, dtype=torch.bfloat16, device=gpu)
        splitk_conv(xc, packed, o, k_splits=splits, workspace=ws, history=hist,
                    slot_index=slot_index, slot_parity=parity, history_cold=n == 0, **act)
        parity[slot_index] += 1
        parts.append(o)
        start += size
    assert torch.equal(torch.cat(parts, dim=1), whole)
    ref = causal_conv_snake_f64(x, w, b, alpha)
    err = (whole.cpu().double() - ref).abs().max().item()
    assert err <= 2 ** -7 * ref.abs().max().item()  # the bf16 output's rounding


def test_a_split_no_tile_holds_is_refused_and_leaves_out_untouched(gpu):
    """k = 7 over 64 rows of 5 positions: a 192-position split tile would stage 192 rows plus 40
    row segments' 6-row halos (432 > 368 rows), so no split tile holds the call. It must come
    back UNSUPPORTED before any launch, out untouched, never as another family's full conv
    followed by a reduction of unwritten partials. k = 1 at 96 channels in 3 slices (one
    32-channel chunk per slice, below every split tile's two) is refused the same way."""
    batch, length, c_in, c_out = 64, 5, 512, 384
    x, w, b, alpha = conv7_operands(batch, length, c_in, c_out, 40)
    packed = pack_conv1d(w, b).to(gpu)
    xg = x.to(gpu)
    ws = torch.full((splitk_workspace_elements(xg, packed, 4),), 7.0, device=gpu)
    out = torch.full((batch, length, c_out), -3.0, device=gpu)
    a = alpha.to(gpu)
    act = dict(activation=N.ACT_SNAKE, act_a=a, act_b=(a + 1e-9).reciprocal())
    with pytest.raises(N.OmniCodecError) as err:
        splitk_conv(xg, packed, out, k_splits=4, workspace=ws, **act)
    assert err.value.status == N.UNSUPPORTED
    lib = N.load_library()
    status = lib.omni_conv1d_splitk_noalloc(ctypes.byref(_conv_args(xg, packed, out, **act)), 4,
                                            N.CONV_KERNEL_AUTO, 0, N.stream_handle(gpu))
    assert status == N.UNSUPPORTED
    torch.cuda.synchronize()
    assert bool((out == -3.0).all()) and bool((ws == 7.0).all())
    # the unsplit conv serves the same call
    from sglang_omni_amd.kernels.conv import fused_conv
    fused_conv(xg, packed, out, **act)
    ref = causal_conv_snake_f64(x, w, b, alpha)
    torch.testing.assert_close(out.cpu().double(), ref, rtol=1e-5,
                               atol=1e-5 * ref.abs().max().item())
    x1, w1, b1 = operands(40, 96, 128, 41, gpu)
    p1 = pack_conv1d(w1, b1).to(gpu)
    out1 = torch.full((1, 40, 128), -3.0, device=gpu)
    ws1 = torch.empty(splitk_workspace_elements(x1, p1, 3), device=gpu)
    with pytest.raises(N.OmniCodecError) as err:
        gemm(x1, p1, out1, k_splits=3, workspace=ws1)
    assert err.value.status == N.UNSUPPORTED
    torch.cuda.synchronize()
    assert bool((out1 == -3.0).all())


def test_the_decoder_runs_a_refused_input_conv_split_unsplit(gpu):
    """The 24 kHz decoder's input conv (512 -> 1536, k = 7, 4 slices) over 64 rows of 5 frames,
    a shape no split tile holds, through ``from_indices``: every row equals its own decode
    (1 row, which the split tiles hold) to float32 summation order, so the unsplit fallback
    ran (bf16 roundings of the two summation orders may differ, inside the decoders' 2e-3
    bound); a refused split never hands its stale partials to the reduction."""
    from sglang_omni_amd.models import DacCodecDecoder, make_dac_weights
    from sglang_omni_amd.models.configs import CODEC_24K

    decoder = DacCodecDecoder(make_dac_weights(CODEC_24K, seed=0), CODEC_24K, device=gpu)
    assert decoder.in_conv_splits == 4
    gen = torch.Generator().manual_seed(42)
    codes = torch.randint(0, CODEC_24K.codebook_size, (64, CODEC_24K.n_codebooks, 5),
                          generator=gen).to(gpu)
    batched = decoder.from_indices(codes)
    assert decoder._workspaces[(64, 5)].in_conv_split is False
    for r in (0, 17, 63):
        alone = decoder.from_indices(codes[r:r + 1])
        assert decoder._workspaces[(1, 5)].in_conv_split is True
        err = (batched[r] - alone[0]).abs().max().item()
        assert err <= 2e-3, (r, err)
