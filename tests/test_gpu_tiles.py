"""Every tile configuration of every conv kernel family, held against float64 and against each
other, through ``omni_conv1d_fused_with`` (the C ABI's forced-configuration entry point).

The decoder's convs pick their tile configuration by problem size, so the configurations the
benchmarks run (64 streams, 250- and 1500-frame utterances, 16 HiFiGAN clips) are not the ones
small shapes pick. Here each list entry is forced on a shape it fits:

* all entries of one family and input mode accumulate the same products in the same order
  (32-channel chunks ascending, taps ascending, one MFMA per step), so each must give the bits
  of the size-chosen configuration;
* a stream decoded in two chunks through the slot history equals its whole decode bit for bit,
  per entry (each entry stages history rows with its own geometry);
* each result against the float64 conv of the bf16 operands it multiplied (the restatement of
  channels_last_conv.py:45-120 in tests/unit_test/utils/test_channels_last_conv.py:18-115) at
  float32-summation tolerance (1e-5); an operand activated while staged is taken from the GPU's
  own epilogue form of the same activation (see ``staged_operands``).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import fused_conv, pack_conv1d, pack_conv_transpose1d, plan_shapes
from sglang_omni_amd.quantization import dequantize_fp8, quantize_fp8

pytestmark = pytest.mark.gpu

# entries per list (tests/test_plans.py checks these against the library's own counts)
DMA_LIST = {1: 4, 2: 4, 7: 4}
# the narrow layers' LDS-DMA lists (n_cols <= 64, bf16 weights: HiFiGAN's 64 / 32-channel stages)
NARROW_DMA_LIST = {3: 4, 7: 3, 11: 3}
# and for its 128-channel stage (n_cols == 128; k = 3 also at 256 columns)
NARROW128_DMA_LIST = {3: 2, 7: 1, 11: 2}
# k = 3 at other multiples of 96 columns (192: the three phases of HiFiGAN's 128 -> 64 up conv)
NARROW96_DMA_LIST = {3: 2}
STAGED_LIST = 10
STAGED11_LIST = 10
FUSED_LIST = 3

SHAPES = [(2, 300), (3, 100), (64, 12), (1, 700), (8, 40), (2, 20)]  # (rows, positions)


def bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


def fits(plan_kw: dict, batch: int, length: int, kernel: int, config: int) -> bool:
    try:
        plan = plan_shapes(batch=batch, length=length, kernel=kernel, config=config, **plan_kw)
    except N.OmniCodecError as err:
        if err.status != N.UNSUPPORTED:
            raise
        return False
    return plan.kernel == kernel and plan.config == config


def pick_shape(plan_kw: dict, kernel: int, config: int, *, streamed: bool):
    """The first (rows, positions) the entry serves, whole and (streamed) as two chunks with
    history; None when the entry serves none of them."""
    for batch, length in SHAPES:
        if not fits(plan_kw, batch, length, kernel, config):
            continue
        if streamed:
            a = length // 2
            hist_kw = dict(plan_kw, history=True)
            if not (fits(hist_kw, batch, a, kernel, config)
                    and fits(hist_kw, batch, length - a, kernel, config)):
                continue
        return batch, length
    return None


def advance(parity: torch.Tensor, slot_index: torch.Tensor) -> None:
    lib = N.load_library()
    N.check(lib.omni_advance_slots(parity.data_ptr(), parity.shape[0], slot_index.data_ptr(),
                                   slot_index.shape[0], N.stream_handle()), "advance")


def streamed(x: torch.Tensor, packed, length: int, n_out: int, kernel: int, config: int, *,
             collect: str = "out", out_dtype=torch.float32, residual=None, **kw) -> torch.Tensor:
    """Two chunks of x through a fresh slot history (rows on shuffled slots): the concatenated
    outputs (``collect`` "out", or the float32 "sum_out")."""
    batch, c_in = x.shape[0], x.shape[2]
    dev = x.device
    state = {}
    if packed.left_pad:  # a k = 1 conv keeps no history: its chunks are independent
        hist = torch.randn(batch + 2, 2, packed.left_pad, c_in, device=dev).to(torch.bfloat16)
        slot_index = (torch.arange(batch, device=dev).flip(0) + 1).contiguous()
        parity = torch.zeros(batch + 2, dtype=torch.int64, device=dev)
        state = dict(history=hist, slot_index=slot_index, slot_parity=parity)
    a = length // 2
    outs = []
    for i, (s, n) in enumerate(((0, a), (a, length - a))):
        out = torch.empty(batch, n, n_out, dtype=out_dtype, device=dev)
        extra = {}
        if residual is not None:
            extra["residual"] = residual[:, s:s + n].contiguous()
        if collect == "sum_out":
            extra["sum_out"] = torch.empty(batch, n, n_out, dtype=torch.float32, device=dev)
        fused_conv(x[:, s:s + n].contiguous(), packed, out, history_cold=i == 0, kernel=kernel,
                   config=config, **state, **extra, **kw)
        if state:
            advance(state["slot_parity"], state["slot_index"])
        outs.append(out if collect == "out" else extra["sum_out"])
    return torch.cat(outs, dim=1)


def conv64(u: torch.Tensor, w: torch.Tensor, b, *, dilation: int = 1, left: int | None = None,
           right: int = 0) -> torch.Tensor:
    """float64 conv of [B, L, C] -> [B, L', C_out] with `left` zeros before (causal by default)."""
    k = w.shape[-1]
    if left is None:
        left = (k - 1) * dilation
    y = F.conv1d(F.pad(u.double().transpose(1, 2), (left, right)), w.double(),
                 None if b is None else b.double(), dilation=dilation)
    return y.transpose(1, 2)


def check_float64(actual: torch.Tensor, expected: torch.Tensor) -> None:
    """float32 accumulation of exact bf16 products against float64: summation error only."""
    torch.testing.assert_close(actual.double().cpu(), expected, rtol=1e-5, atol=1e-5)


def snake64(x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    a = alpha.double().view(1, 1, -1)
    return x.double() + torch.sin(a * x.double()) ** 2 / (a + 1e-9)


# ------------------------------------------------------------------------------ LDS-DMA family

DMA_CASES = [(taps, k) for taps in (7, 1, 2) for k in range(1, DMA_LIST[taps] + 1)]


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
@pytest.mark.parametrize("taps,config", DMA_CASES, ids=lambda v: str(v))
def test_dma_tile_matches_float64_and_the_chosen_tile(gpu, taps, config, fp8):
    """bf16 weights, or E4M3 weights kept as bytes in LDS and widened on the operand read (held
    against the float64 conv with the dequantized weights)."""
    gen = torch.Generator().manual_seed(100 * taps + config + 7 * fp8)
    if taps == 2:  # the polyphase transposed conv 192 -> 96, stride 6 (k = 12)
        c_in, c_out, stride = 192, 96, 6
        w = torch.randn(c_in, c_out, 2 * stride, generator=gen) / math.sqrt(2 * c_in)
        w = dequantize_fp8(*quantize_fp8(w, 1), 1) if fp8 else bf(w)
        b = bf(torch.randn(c_out, generator=gen) * 0.1)
        packed = pack_conv_transpose1d(w, b, stride=stride, fp8=fp8).to(gpu)
        plan_kw = dict(c_in=c_in, n_cols=stride * c_out, c_out=c_out, taps=2, left_pad=1, fp8=fp8)
    else:
        c_in = c_out = 192
        d = 9 if taps == 7 else 1
        w = torch.randn(c_out, c_in, taps, generator=gen) / math.sqrt(c_in * taps)
        w = dequantize_fp8(*quantize_fp8(w, 0), 0) if fp8 else bf(w)
        b = bf(torch.randn(c_out, generator=gen) * 0.1)
        packed = pack_conv1d(w, b, dilation=d, fp8=fp8).to(gpu)
        plan_kw = dict(c_in=c_in, n_cols=c_out, c_out=c_out, taps=taps, dilation=d, fp8=fp8)
    assert (packed.weight.dtype == torch.float8_e4m3fn) == fp8
    shape = pick_shape(plan_kw, N.CONV_KERNEL_DMA, config, streamed=True)
    assert shape is not None, "every LDS-DMA entry serves one of the test shapes"
    batch, length = shape
    x = bf(torch.randn(batch, length, c_in, generator=gen)).to(gpu, torch.bfloat16)
    n = packed.n_cols
    forced = torch.empty(batch, length, n, dtype=torch.float32, device=gpu)
    fused_conv(x, packed, forced, kernel=N.CONV_KERNEL_DMA, config=config)
    chosen = torch.empty_like(forced)
    fused_conv(x, packed, chosen)
    assert torch.equal(forced, chosen)
    chunks = streamed(x, packed, length, n, N.CONV_KERNEL_DMA, config)
    assert torch.equal(chunks, forced)
    if taps == 2:
        y = F.conv_transpose1d(x.float().cpu().double().transpose(1, 2), w.double(), b.double(),
                               stride=stride)[..., : length * stride].transpose(1, 2)
        check_float64(forced.view(batch, length * stride, c_out), y)
    else:
        check_float64(forced, conv64(x.float().cpu(), w, b, dilation=packed.dilation))


def _narrow_list(cols: int) -> dict:
    if cols == 192:
        return NARROW96_DMA_LIST
    return NARROW128_DMA_LIST if cols > 64 else NARROW_DMA_LIST


NARROW_CASES = [(taps, cols, k) for taps in (3, 7, 11) for cols in (256, 192, 128, 64, 32)
                if taps == 3 or cols not in (256, 192)
                for k in range(1, _narrow_list(cols)[taps] + 1)]


@pytest.mark.parametrize("taps,cols,config", NARROW_CASES, ids=lambda v: str(v))
def test_narrow_dma_tile_matches_float64_and_the_chosen_tile(gpu, taps, cols, config):
    """HiFiGAN's convs ('same' padding, dilation 5) at 256 and 192 (k = 3), 128, 64 and 32
    channels on their LDS-DMA tiles: each entry against the float64 conv and the size-chosen
    entry's bits."""
    gen = torch.Generator().manual_seed(1000 * taps + 10 * cols + config)
    c_in = c_out = cols
    d = 5
    w = bf(torch.randn(c_out, c_in, taps, generator=gen) / math.sqrt(c_in * taps))
    b = bf(torch.randn(c_out, generator=gen) * 0.1)
    packed = pack_conv1d(w, b, dilation=d, causal=False).to(gpu)
    plan_kw = dict(c_in=c_in, n_cols=c_out, c_out=c_out, taps=taps, dilation=d,
                   left_pad=packed.left_pad)
    shape = pick_shape(plan_kw, N.CONV_KERNEL_DMA, config, streamed=False)
    if shape is None:
        pytest.skip(f"entry {config} does not take {cols} columns (column padding or a one-stage "
                    f"entry's c_in)")
    batch, length = shape
    x = bf(torch.randn(batch, length, c_in, generator=gen)).to(gpu, torch.bfloat16)
    forced = torch.empty(batch, length, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x, packed, forced, kernel=N.CONV_KERNEL_DMA, config=config)
    chosen = torch.empty_like(forced)
    fused_conv(x, packed, chosen)
    assert torch.equal(forced, chosen)
    pad = (taps - 1) * d // 2
    check_float64(forced, conv64(x.float().cpu(), w, b, dilation=d, left=pad, right=pad))


# ------------------------------------------------------------------------------ register-staged

STAGED_MODES = ["raw-bf16", "snake-bf16", "f32-snake-bf16", "raw-fp8", "f32-leaky-fp8"]


def staged_operands(mode: str, batch: int, length: int, c_in: int, gen: torch.Generator, dev):
    """(x on the device, in-activation kwargs, the bf16 operand the conv stages, as float64).

    With an input activation the operand is taken from the GPU itself: a conv with zero weights
    whose residual is x applies the same activation in its epilogue (the staging and the
    epilogues evaluate one expression, e.g. Snake through v_sin in revolutions), so its bf16
    output is the staged operand bit for bit and the conv can be held to float64 exactly."""
    if mode.startswith("f32"):
        xd = torch.randn(batch, length, c_in, generator=gen).to(dev)
    else:
        xd = bf(torch.randn(batch, length, c_in, generator=gen)).to(dev, torch.bfloat16)
    if "snake" in mode:
        a = (torch.rand(c_in, generator=gen) + 0.5).to(dev)
        kw = dict(in_activation=N.ACT_SNAKE, in_a=a, in_b=(a + 1e-9).reciprocal())
        epi = dict(activation=N.ACT_SNAKE, act_a=kw["in_a"], act_b=kw["in_b"])
    elif "leaky" in mode:
        kw = dict(in_activation=N.ACT_LEAKY_RELU, in_slope=0.1)
        epi = dict(activation=N.ACT_LEAKY_RELU, slope=0.1)
    else:
        return xd, {}, xd.float().cpu().double()
    zero = pack_conv1d(torch.zeros(c_in, c_in, 1), None).to(dev)
    u = torch.empty(batch, length, c_in, dtype=torch.bfloat16, device=dev)
    fused_conv(xd, zero, u, residual=xd.float().contiguous(), **epi)
    return xd, kw, u.float().cpu().double()


@pytest.mark.parametrize("mode", STAGED_MODES)
@pytest.mark.parametrize("config", range(1, STAGED_LIST + 1))
def test_staged_tile_matches_float64_and_the_chosen_tile(gpu, config, mode):
    gen = torch.Generator().manual_seed(config * 7 + len(mode))
    c_in, c_out, d = 96, 192, 3
    fp8 = mode.endswith("fp8")
    plan_kw = dict(c_in=c_in, n_cols=c_out, c_out=c_out, taps=7, dilation=d, fp8=fp8,
                   x_f32=mode.startswith("f32"),
                   in_activation=N.ACT_NONE if mode.startswith("raw") else N.ACT_SNAKE)
    shape = pick_shape(plan_kw, N.CONV_KERNEL_STAGED, config, streamed=True)
    assert shape is not None, "every register-staged entry serves one of the test shapes"
    batch, length = shape
    w = torch.randn(c_out, c_in, 7, generator=gen) / math.sqrt(c_in * 7)
    if fp8:
        q, s = quantize_fp8(w, 0)
        w_eff = dequantize_fp8(q, s, 0)
    else:
        w = bf(w)
        w_eff = w
    b = torch.randn(c_out, generator=gen) * 0.1
    packed = pack_conv1d(w, b, dilation=d, fp8=fp8).to(gpu)
    xd, act_kw, u64 = staged_operands(mode, batch, length, c_in, gen, gpu)
    forced = torch.empty(batch, length, c_out, dtype=torch.float32, device=gpu)
    fused_conv(xd, packed, forced, kernel=N.CONV_KERNEL_STAGED, config=config, **act_kw)
    chosen = torch.empty_like(forced)
    fused_conv(xd, packed, chosen, **act_kw)  # the size-chosen tile (LDS-DMA for raw bf16)
    assert torch.equal(forced, chosen)
    chunks = streamed(xd, packed, length, c_out, N.CONV_KERNEL_STAGED, config, **act_kw)
    assert torch.equal(chunks, forced)
    check_float64(forced, conv64(u64, w_eff, b, dilation=d))


@pytest.mark.parametrize("mode", ["raw-bf16", "snake-bf16"])
@pytest.mark.parametrize("config", range(1, STAGED11_LIST + 1))
def test_staged11_tile_matches_float64_and_the_chosen_tile(gpu, config, mode):
    """The k = 11 'same'-padded convs of the HiFiGAN resblocks (dilation 5: 25 samples of
    padding on either side)."""
    gen = torch.Generator().manual_seed(config * 11 + len(mode))
    c, k, d = 64, 11, 5
    pad = (k * d - d) // 2
    plan_kw = dict(c_in=c, n_cols=c, c_out=c, taps=k, dilation=d, left_pad=pad,
                   in_activation=N.ACT_NONE if mode.startswith("raw") else N.ACT_SNAKE)
    shape = pick_shape(plan_kw, N.CONV_KERNEL_STAGED11, config, streamed=False)
    if shape is None:
        # an entry whose weight tile does not fit the LDS at 11 taps is refused for every shape
        with pytest.raises(N.OmniCodecError, match="status 2"):
            plan_shapes(batch=1, length=16, kernel=N.CONV_KERNEL_STAGED11, config=config,
                        **plan_kw)
        pytest.skip(f"entry {config} cannot hold 11 taps (the library refuses it)")
    batch, length = shape
    w = bf(torch.randn(c, c, k, generator=gen) / math.sqrt(c * k))
    b = torch.randn(c, generator=gen) * 0.1
    packed = pack_conv1d(w, b, dilation=d, causal=False).to(gpu)
    xd, act_kw, u64 = staged_operands(mode, batch, length, c, gen, gpu)
    forced = torch.empty(batch, length, c, dtype=torch.float32, device=gpu)
    fused_conv(xd, packed, forced, kernel=N.CONV_KERNEL_STAGED11, config=config, **act_kw)
    chosen = torch.empty_like(forced)
    fused_conv(xd, packed, chosen, **act_kw)
    assert torch.equal(forced, chosen)
    check_float64(forced, conv64(u64, w, b, dilation=d, left=pad, right=pad))


# ------------------------------------------------------------------------------ fused unit


# (entry, channels, operand, fp8 weights): entry 1 is the LDS-DMA unit, which takes 192-channel
# bf16 operands as they are with bf16 weights; entries 2 and 3 (the register-staged full and
# short-row tiles) take every case
FUSED_CASES = [(config, channels, mode, fp8) for config in range(1, FUSED_LIST + 1)
               for channels in (96, 192) for mode in ("raw", "f32-snake") for fp8 in (False, True)
               if config > 1 or (channels == 192 and mode == "raw" and not fp8)]


@pytest.mark.parametrize("config,channels,mode,fp8", FUSED_CASES,
                         ids=[f"{('dma', 'full', 'short')[c - 1]}-{n}-{m}-{'fp8' if f else 'bf16'}"
                              for c, n, m, f in FUSED_CASES])
def test_fused_unit_tile_matches_its_two_launch_form(gpu, config, channels, mode, fp8):
    """conv k7 (d = 9) -> Snake -> conv k1 -> + x in one launch equals, bit for bit, the same
    unit as two launches (h through HBM as bf16); the two-launch form's convs are then held to
    float64 on the operands they read (h within one bf16 ulp of the float64 Snake)."""
    gen = torch.Generator().manual_seed(config * 1000 + channels + len(mode) + fp8)
    c, d = channels, 9
    plan_kw = dict(c_in=c, n_cols=c, c_out=c, taps=7, dilation=d, fused_unit=True, fp8=fp8,
                   x_f32=mode != "raw", in_activation=N.ACT_NONE if mode == "raw" else N.ACT_SNAKE)
    shape = pick_shape(plan_kw, N.CONV_KERNEL_FUSED_UNIT, config, streamed=True)
    assert shape is not None
    batch, length = shape
    w1 = torch.randn(c, c, 7, generator=gen) / math.sqrt(c * 7)
    w2 = torch.randn(c, c, 1, generator=gen) / math.sqrt(c)
    if fp8:
        w1_eff = dequantize_fp8(*quantize_fp8(w1, 0), 0)
        w2_eff = dequantize_fp8(*quantize_fp8(w2, 0), 0)
    else:
        w1 = w1_eff = bf(w1)
        w2 = w2_eff = bf(w2)
    b1 = torch.randn(c, generator=gen) * 0.1
    b2 = torch.randn(c, generator=gen) * 0.1
    p1 = pack_conv1d(w1, b1, dilation=d, fp8=fp8).to(gpu)
    p2 = pack_conv1d(w2, b2, fp8=fp8).to(gpu)
    xd, act_kw, u64 = staged_operands(
        "f32-snake-bf16" if mode != "raw" else "raw-bf16", batch, length, c, gen, gpu)
    resid = torch.randn(batch, length, c, generator=gen).to(gpu)
    alpha_mid = (torch.rand(c, generator=gen) + 0.5).to(gpu)
    alpha_out = (torch.rand(c, generator=gen) + 0.5).to(gpu)
    mid = dict(mid_activation=N.ACT_SNAKE, mid_a=alpha_mid, mid_b=(alpha_mid + 1e-9).reciprocal())
    outk = dict(activation=N.ACT_SNAKE, act_a=alpha_out, act_b=(alpha_out + 1e-9).reciprocal())
    out = torch.empty(batch, length, c, dtype=torch.bfloat16, device=gpu)
    x_new = torch.empty(batch, length, c, dtype=torch.float32, device=gpu)
    fused_conv(xd, p1, out, second=p2, residual=resid, sum_out=x_new,
               kernel=N.CONV_KERNEL_FUSED_UNIT, config=config, **act_kw, **mid, **outk)
    # the same unit as two launches (the register-staged family, so fp8 and float32 inputs run)
    h = torch.empty(batch, length, c, dtype=torch.bfloat16, device=gpu)
    fused_conv(xd, p1, h, activation=N.ACT_SNAKE, act_a=alpha_mid,
               act_b=(alpha_mid + 1e-9).reciprocal(), kernel=N.CONV_KERNEL_STAGED, config=1,
               **act_kw)
    out2 = torch.empty_like(out)
    x2 = torch.empty_like(x_new)
    fused_conv(h, p2, out2, residual=resid, sum_out=x2, kernel=N.CONV_KERNEL_STAGED, config=1,
               **outk)
    assert torch.equal(x_new, x2)
    assert torch.equal(out, out2)
    # streamed == whole, through the conv1 history
    chunks = streamed(xd, p1, length, c, N.CONV_KERNEL_FUSED_UNIT, config, collect="sum_out",
                      out_dtype=torch.bfloat16, second=p2, residual=resid, **act_kw, **mid,
                      **outk)
    assert torch.equal(chunks, x_new)
    # the two-launch form against float64
    h64 = snake64(conv64(u64, w1_eff, b1, dilation=d), alpha_mid.cpu())
    torch.testing.assert_close(h.float().cpu().double(), h64, rtol=2 ** -7, atol=1e-5)
    expected = conv64(h.float().cpu(), w2_eff, b2) + resid.cpu().double()
    check_float64(x_new, expected)
