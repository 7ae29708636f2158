"""GPU parity of the Qwen3-Omni code2wav path: each front kernel against the float32 oracle's
piece on the same inputs (bf16 operands, so tolerances are bf16 rounding of the outputs), the
whole decoder against the oracle (itself pinned to transformers' Qwen3OmniMoeCode2Wav) with the
weights the GPU multiplies by, the streaming invariants (a stream decoded in chunks gives the
whole decode; slot reuse after zeroing gives a fresh stream) and HIP-graph replay.

Waveform tolerances: max|err| <= 2e-3 and SNR >= 40 dB against the float32 oracle, output RMS
asserted non-trivial; a stream decoded in chunks equals its whole decode bit for bit (every
kernel's summation order, the front's GEMMs on the k = 1 conv kernel included, is independent of
the row count).
"""

from __future__ import annotations

import pytest
import torch

from oracle import codec_oracle as O
from oracle import qwen3_code2wav_oracle as Q
from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels import code2wav_front as F
from sglang_omni_amd.models import (
    CodecGraphRunner,
    GraphKey,
    Qwen3Code2WavConfig,
    Qwen3Code2WavDecoder,
    Qwen3TTSCodecConfig,
    Qwen3TTSCodecDecoder,
    make_qwen3_code2wav_weights,
)
from sglang_omni_amd.models.configs import QWEN3_CODE2WAV, QWEN3_TTS_CODEC

pytestmark = pytest.mark.gpu

# 256 hidden (4 heads of 64, 2 K/V heads), window 8; decoder 384 -> 192 -> 96 channels, x6;
# the input conv's gain puts the output RMS near the full configuration's (~0.04)
SMALL = Qwen3Code2WavConfig(hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                            num_key_value_heads=2, intermediate_size=512, sliding_window=8,
                            codebook_size=64, num_quantizers=4, decoder_dim=384,
                            upsample_rates=(2, 3), input_conv_gain=0.04)


def bf16r(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


def effective_weights(state: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """The float32 values the GPU decoder multiplies by: matrices and conv weights rounded to
    bf16 (but the depthwise conv's, which stays float32), decoder conv biases rounded to bf16."""
    out = {}
    for name, t in state.items():
        if name.startswith("quantizer."):
            out[name] = t.float()  # the split quantizer's projected tables stay float32
        elif t.dim() >= 2 and "dwconv" not in name:
            out[name] = bf16r(t)
        elif name.startswith("decoder.") and name.endswith("conv.bias"):
            out[name] = bf16r(t)
        else:
            out[name] = t.float()
    return out


def check_waveform(actual: torch.Tensor, expected: torch.Tensor, max_abs: float = 2e-3,
                   min_snr: float = 40.0) -> None:
    actual = actual.cpu()
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    err = (actual.double() - expected.double()).abs().max().item()
    snr = O.snr_db(expected, actual)
    rms = expected.double().pow(2).mean().sqrt().item()
    print(f"max|err| {err:.3e}  SNR {snr:.2f} dB  output rms {rms:.4f}")
    assert rms > 0.005, "the reference output is too quiet for the tolerance to mean anything"
    assert err <= max_abs, err
    assert snr >= min_snr, snr


# ------------------------------------------------------------------------------ kernels


def test_rms_norm_residual(gpu):
    # 1024 channels with the residual add (the unrolled kernel), 256 without (the generic one),
    # then each kernel on the other case
    g = torch.Generator().manual_seed(0)
    h = torch.randn(37, 1024, generator=g) * 3
    delta = bf16r(torch.randn(37, 1024, generator=g))
    scale = torch.rand(1024, generator=g)
    weight = 1 + 0.1 * torch.randn(1024, generator=g)
    hd = h.to(gpu)
    normed = torch.empty(37, 1024, dtype=torch.bfloat16, device=gpu)
    F.rms_norm_residual(hd, weight.to(gpu), 1e-5, normed, delta=delta.to(torch.bfloat16).to(gpu),
                        scale=scale.to(gpu))
    h_ref = h + scale * delta
    torch.testing.assert_close(hd.cpu(), h_ref, rtol=1e-6, atol=1e-5)
    ref = Q.rms_norm(h_ref, weight, 1e-5)
    torch.testing.assert_close(normed.float().cpu(), ref, rtol=2 ** -8, atol=1e-6)
    # without delta: a plain RMSNorm, h unchanged
    h2 = torch.randn(5, 256, generator=g).to(gpu)
    n2 = torch.empty(5, 256, dtype=torch.bfloat16, device=gpu)
    before = h2.clone()
    F.rms_norm_residual(h2, torch.ones(256, device=gpu), 1e-6, n2)
    assert torch.equal(h2, before)
    torch.testing.assert_close(n2.float().cpu(), Q.rms_norm(before.cpu(), torch.ones(256), 1e-6),
                               rtol=2 ** -8, atol=1e-6)
    h3 = (torch.randn(9, 1024, generator=g) * 2).to(gpu)
    n3 = torch.empty(9, 1024, dtype=torch.bfloat16, device=gpu)
    before3 = h3.clone()
    F.rms_norm_residual(h3, weight.to(gpu), 1e-5, n3)
    assert torch.equal(h3, before3)
    torch.testing.assert_close(n3.float().cpu(), Q.rms_norm(before3.cpu(), weight, 1e-5),
                               rtol=2 ** -8, atol=1e-6)
    h4 = torch.randn(6, 512, generator=g)
    d4 = bf16r(torch.randn(6, 512, generator=g))
    s4 = torch.rand(512, generator=g)
    h4d = h4.to(gpu)
    n4 = torch.empty(6, 512, dtype=torch.bfloat16, device=gpu)
    F.rms_norm_residual(h4d, torch.ones(512, device=gpu), 1e-5, n4,
                        delta=d4.to(torch.bfloat16).to(gpu), scale=s4.to(gpu))
    torch.testing.assert_close(h4d.cpu(), h4 + s4 * d4, rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(n4.float().cpu(), Q.rms_norm(h4 + s4 * d4, torch.ones(512), 1e-5),
                               rtol=2 ** -8, atol=1e-6)


def _qkv(batch: int, frames: int, heads: int, kv_heads: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch * frames, (heads + 2 * kv_heads) * 64, generator=g).to(torch.bfloat16)


def _rope_ref(qkv: torch.Tensor, batch: int, heads: int, kv_heads: int, starts: list[int],
              theta: float = 10000.0) -> torch.Tensor:
    frames = qkv.shape[0] // batch
    x = qkv.float().view(batch, frames, heads + 2 * kv_heads, 64).clone()
    for b in range(batch):
        cos, sin = Q.rope_cos_sin(torch.arange(frames) + starts[b], 64, theta)
        qk = x[b, :, : heads + kv_heads].transpose(0, 1)  # [H + Hkv, T, 64]
        x[b, :, : heads + kv_heads] = Q.apply_rope(qk, cos, sin).transpose(0, 1)
    return x.view(batch * frames, -1)


def _inv_freq(device) -> torch.Tensor:
    return (1.0 / (10000.0 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))).to(device)


def test_rope_cold_and_at_positions(gpu):
    heads, kv_heads, batch, frames = 4, 2, 3, 11
    qkv = _qkv(batch, frames, heads, kv_heads, 1)
    d = qkv.to(gpu)
    F.rope_kv_write(d, batch, heads, kv_heads, 64, _inv_freq(gpu))
    ref = _rope_ref(qkv, batch, heads, kv_heads, [0, 0, 0])
    torch.testing.assert_close(d.float().cpu(), ref, rtol=2 ** -8, atol=2e-5)
    # warm rows at their slots' positions, K / V into the rings
    ring_frames, slots = 20, 5
    positions = torch.tensor([0, 40, 7, 1000, 123457], dtype=torch.int64)
    index = torch.tensor([3, 1, 4], dtype=torch.int64)
    keys = torch.zeros(slots * ring_frames, kv_heads * 64, dtype=torch.bfloat16, device=gpu)
    values = torch.zeros_like(keys)
    d = qkv.to(gpu)
    F.rope_kv_write(d, batch, heads, kv_heads, 64, _inv_freq(gpu), slot_index=index.to(gpu),
                    positions=positions.to(gpu), cold=False, key_ring=keys, value_ring=values,
                    ring_frames=ring_frames)
    starts = [int(positions[s]) for s in index]
    ref = _rope_ref(qkv, batch, heads, kv_heads, starts)
    # float32 angles at position ~1.2e5: the rotation error grows with position * ulp
    torch.testing.assert_close(d.float().cpu(), ref, rtol=2 ** -8, atol=3e-2)
    torch.testing.assert_close(d.float().cpu()[: 2 * frames], ref[: 2 * frames], rtol=2 ** -8,
                               atol=2e-5)
    got = d.cpu()
    for b, slot in enumerate(index.tolist()):
        for t in range(frames):
            row = slot * ring_frames + (starts[b] + t) % ring_frames
            tok = got[b * frames + t]
            assert torch.equal(keys[row].cpu(), tok[heads * 64:(heads + kv_heads) * 64])
            assert torch.equal(values[row].cpu(), tok[(heads + kv_heads) * 64:])


@pytest.mark.parametrize("frames,window,heads,kv_heads", [(37, 8, 4, 2), (12, 72, 16, 16),
                                                          (300, 72, 2, 1), (5, 1, 2, 2)])
def test_window_attention_first_decode(gpu, frames, window, heads, kv_heads):
    batch = 2
    qkv = _qkv(batch, frames, heads, kv_heads, frames + window)
    x = qkv.float().view(batch, frames, heads + 2 * kv_heads, 64)
    q = x[:, :, :heads].transpose(1, 2)
    k = x[:, :, heads:heads + kv_heads].transpose(1, 2).repeat_interleave(heads // kv_heads, 1)
    v = x[:, :, heads + kv_heads:].transpose(1, 2).repeat_interleave(heads // kv_heads, 1)
    ref = Q.window_attention(q, k, v, window, 0.125).transpose(1, 2).reshape(batch * frames, -1)
    # the probabilities enter the P.V product as bf16 (relative error <= 2^-9 each) and the
    # output is rounded to bf16: |err| <= 2^-9 (sum_j p_j |v_j|) + 2 * 2^-9 |ref|, doubled
    mag = Q.window_attention(q, k, v.abs(), window, 0.125).transpose(1, 2).reshape(batch * frames, -1)
    out = torch.empty(batch * frames, heads * 64, dtype=torch.bfloat16, device=gpu)
    F.window_attention(qkv.to(gpu), batch, heads, kv_heads, 64, window, 0.125, out)
    err = (out.float().cpu() - ref).abs()
    bound = 2 ** -8 * mag + 2 ** -7 * ref.abs() + 1e-6
    assert (err <= bound).all(), (err - bound).max()


def test_window_attention_over_rings_matches_whole_sequence(gpu):
    """Chunks of a stream through rope_kv_write + ring attention give the first-decode
    attention of the whole sequence, bit for bit (same keys, same order)."""
    heads, kv_heads, window, total, ring_frames = 4, 2, 9, 29, 9 - 1 + 8
    qkv_all = _qkv(1, total, heads, kv_heads, 5)
    whole = qkv_all.to(gpu)
    F.rope_kv_write(whole, 1, heads, kv_heads, 64, _inv_freq(gpu))
    ref = torch.empty(total, heads * 64, dtype=torch.bfloat16, device=gpu)
    F.window_attention(whole, 1, heads, kv_heads, 64, window, 0.125, ref)
    slots = 3
    keys = torch.zeros(slots * ring_frames, kv_heads * 64, dtype=torch.bfloat16, device=gpu)
    values = torch.zeros_like(keys)
    positions = torch.zeros(slots, dtype=torch.int64, device=gpu)
    index = torch.tensor([2], dtype=torch.int64, device=gpu)
    outs, start = [], 0
    for n in (5, 8, 1, 7, 8):
        chunk = qkv_all[start:start + n].to(gpu)
        cold = start == 0
        ring = dict(slot_index=index, positions=positions, key_ring=keys, value_ring=values,
                    ring_frames=ring_frames)
        F.rope_kv_write(chunk, 1, heads, kv_heads, 64, _inv_freq(gpu), cold=cold, **ring)
        out = torch.empty(n, heads * 64, dtype=torch.bfloat16, device=gpu)
        F.window_attention(chunk, 1, heads, kv_heads, 64, window, 0.125, out, cold=cold, **ring)
        F.advance_positions(positions, index, n, cold)
        outs.append(out)
        start += n
    assert int(positions[2]) == total and int(positions[0]) == 0
    assert torch.equal(torch.cat(outs), ref)


def test_window_attention_rejects_a_short_ring(gpu):
    qkv = _qkv(1, 8, 2, 2, 0).to(gpu)
    out = torch.empty(8, 128, dtype=torch.bfloat16, device=gpu)
    keys = torch.zeros(10, 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(N.OmniCodecError):
        F.window_attention(qkv, 1, 2, 2, 64, 8, 0.125, out, cold=False,
                           slot_index=torch.zeros(1, dtype=torch.int64, device=gpu),
                           positions=torch.zeros(1, dtype=torch.int64, device=gpu),
                           key_ring=keys, value_ring=keys.clone(), ring_frames=10)


def test_silu_mul_bias_gelu_and_scale_residual(gpu):
    g = torch.Generator().manual_seed(3)
    gu = (torch.randn(19, 2 * 96, generator=g) * 3).to(torch.bfloat16)
    out = torch.empty(19, 96, dtype=torch.bfloat16, device=gpu)
    F.silu_mul(gu.to(gpu), out)
    ref = torch.nn.functional.silu(gu[:, :96].float()) * gu[:, 96:].float()
    torch.testing.assert_close(out.float().cpu(), ref, rtol=2 ** -8, atol=1e-5)
    y = (torch.randn(7, 64, generator=g) * 4).to(torch.bfloat16)
    b = torch.randn(64, generator=g)
    yd = y.to(gpu)
    F.bias_gelu(yd, b.to(gpu))
    torch.testing.assert_close(yd.float().cpu(), torch.nn.functional.gelu(y.float() + b),
                               rtol=2 ** -8, atol=1e-5)
    r = torch.randn(7, 64, generator=g)
    gamma = torch.rand(64, generator=g)
    rd = r.to(gpu)
    z = torch.empty(7, 64, dtype=torch.bfloat16, device=gpu)
    F.bias_scale_residual(rd, y.to(gpu), b.to(gpu), gamma.to(gpu), out=z)
    r_ref = r + gamma * (y.float() + b)
    torch.testing.assert_close(rd.cpu(), r_ref, rtol=1e-6, atol=1e-6)
    assert torch.equal(z.cpu(), rd.cpu().to(torch.bfloat16))


@pytest.mark.parametrize("c", [512, 1024])  # the generic kernel and the unrolled 1024-channel one
def test_dwconv_layernorm_whole_and_streamed(gpu, c):
    g = torch.Generator().manual_seed(4)
    batch, length = 2, 23
    x = torch.randn(batch, length, c, generator=g)
    w = torch.randn(c, 1, 7, generator=g) * 0.4
    bias = torch.randn(c, generator=g) * 0.1
    lw, lb = 1 + 0.1 * torch.randn(c, generator=g), 0.1 * torch.randn(c, generator=g)
    y = Q.causal_conv(x.transpose(1, 2), w, bias, groups=c).transpose(1, 2)
    ref = torch.nn.functional.layer_norm(y, (c,), lw, lb, eps=1e-6)
    args = (w[:, 0].t().contiguous().to(gpu), bias.to(gpu), lw.to(gpu), lb.to(gpu), 1e-6)
    out = torch.empty(batch, length, c, dtype=torch.bfloat16, device=gpu)
    F.dwconv_layernorm(x.to(gpu), *args, out)
    torch.testing.assert_close(out.float().cpu(), ref, rtol=2 ** -8, atol=2e-5)
    # streamed in chunks (2 < 6 history samples, then longer) with slot history
    hist = torch.zeros(4, 2, 6, c, device=gpu)
    parity = torch.zeros(4, dtype=torch.int64, device=gpu)
    index = torch.tensor([3, 0], dtype=torch.int64, device=gpu)
    parts, s = [], 0
    for n in (2, 9, 1, 11):
        o = torch.empty(batch, n, c, dtype=torch.bfloat16, device=gpu)
        F.dwconv_layernorm(x[:, s:s + n].contiguous().to(gpu), *args, o, history=hist,
                           slot_index=index, slot_parity=parity, history_cold=s == 0)
        parity[index] += 1
        parts.append(o.cpu())
        s += n
    torch.testing.assert_close(torch.cat(parts, 1).float(), out.float().cpu(), rtol=0, atol=0)


# ------------------------------------------------------------------------------ decoder


@pytest.fixture(scope="module")
def small(gpu):
    state = make_qwen3_code2wav_weights(SMALL, seed=0, branch_scale=0.5, activation_spread=0.1)
    return state, Qwen3Code2WavDecoder(state, SMALL, device=gpu)


def _codes(cfg, batch: int, frames: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, cfg.codebook_size, (batch, cfg.num_quantizers, frames), generator=g)


@pytest.mark.parametrize("frames", [3, 20])
def test_small_decoder_matches_oracle(small, gpu, frames):
    state, dec = small
    codes = _codes(SMALL, 2, frames, frames)
    got = dec.from_indices(codes.to(gpu))
    ref = Q.qwen3_code2wav(codes, effective_weights(state), SMALL)
    assert got.shape[-1] == Q.first_decode_samples(SMALL, frames)
    check_waveform(got, ref)


def test_small_decoder_streams_like_the_whole_decode(small, gpu):
    state, dec = small
    codes = _codes(SMALL, 3, 30, 7).to(gpu)
    whole = dec.from_indices(codes).cpu()
    pool = dec.new_state_pool(num_slots=5)
    index = torch.tensor([4, 0, 2], dtype=torch.int64, device=gpu)
    parts, s = [], 0
    for n in (4, 1, 12, 13):
        parts.append(dec.decode_slots(codes[..., s:s + n], pool, index, first_decode=s == 0).cpu())
        s += n
    streamed = torch.cat(parts, dim=-1)
    assert streamed.shape == whole.shape
    assert torch.equal(streamed, whole)
    assert pool.frame_positions[index].tolist() == [30, 30, 30]
    # a released slot, zeroed, decodes a new stream as a fresh pool does
    pool.zero_slots(index[:1])
    again = dec.decode_slots(codes[:1, :, :4], pool, index[:1], first_decode=True).cpu()
    assert torch.equal(again, parts[0][:1])


def test_small_decoder_rotary_epilogue_gives_the_two_launch_bits(small, gpu):
    """The qkv GEMM with the rotary embedding and the ring writes in its epilogue
    (omni_gemm_rope_kv) and the GEMM followed by the rotary kernel give the same waveform bits,
    whole and streamed through the K / V rings."""
    state, dec = small
    assert dec.fused_rope  # 64-wide heads, (4 + 2 * 2) * 64 qkv columns

    def run():
        codes = _codes(SMALL, 3, 26, 11).to(gpu)
        whole = dec.from_indices(codes).cpu()
        pool = dec.new_state_pool(num_slots=4)
        index = torch.tensor([3, 0, 1], dtype=torch.int64, device=gpu)
        parts, s = [], 0
        for n in (5, 9, 12):
            parts.append(dec.decode_slots(codes[..., s:s + n], pool, index,
                                          first_decode=s == 0).cpu())
            s += n
        return whole, torch.cat(parts, dim=-1)

    fused = run()
    dec.fused_rope = False
    try:
        two_launch = run()
    finally:
        dec.fused_rope = True
    assert torch.equal(fused[0], two_launch[0])
    assert torch.equal(fused[1], two_launch[1])


def test_small_decoder_rows_at_different_positions_keep_their_streams(small, gpu):
    """Two streams at different positions (12 and 20 frames in) continue in one decode: each
    row reads its own slot's ring window and histories (code2wav.py:417-460 with per-slot frame
    positions; the reference's test_code2wav.py:1262-1297)."""
    _, dec = small
    a = _codes(SMALL, 1, 18, 21).to(gpu)
    b = _codes(SMALL, 1, 26, 22).to(gpu)
    whole_a = dec.from_indices(a).cpu()
    whole_b = dec.from_indices(b).cpu()
    pool = dec.new_state_pool(num_slots=4)
    ia = torch.tensor([3], dtype=torch.int64, device=gpu)
    ib = torch.tensor([1], dtype=torch.int64, device=gpu)
    head_a = dec.decode_slots(a[..., :12], pool, ia, first_decode=True).cpu()
    head_b = dec.decode_slots(b[..., :20], pool, ib, first_decode=True).cpu()
    both = dec.decode_slots(torch.cat([a[..., 12:], b[..., 20:]]), pool,
                            torch.cat([ia, ib]), first_decode=False).cpu()
    assert pool.frame_positions[[3, 1]].tolist() == [18, 26]
    got_a = torch.cat([head_a, both[:1]], dim=-1)
    got_b = torch.cat([head_b, both[1:]], dim=-1)
    # the GEMMs run at other row counts than in the whole decodes: rounding-level differences
    # (a row reading another slot's window or the wrong positions is off by ~1e-1)
    for got, whole in ((got_a, whole_a), (got_b, whole_b)):
        assert got.shape == whole.shape
        assert (got - whole).abs().max().item() <= 2e-3
        assert O.snr_db(whole, got) >= 40.0


def test_small_decoder_reused_slot_equals_a_fresh_pool(small, gpu):
    """A slot released by one stream and zeroed gives the next stream the decode a fresh pool
    gives, bit for bit (the reference's test_code2wav.py:1242-1257)."""
    _, dec = small
    index = torch.tensor([2, 0], dtype=torch.int64, device=gpu)
    pool = dec.new_state_pool(num_slots=3)
    old = _codes(SMALL, 2, 16, 31).to(gpu)
    dec.decode_slots(old[..., :9], pool, index, first_decode=True)
    dec.decode_slots(old[..., 9:], pool, index, first_decode=False)
    pool.zero_slots(index)
    new = _codes(SMALL, 2, 10, 32).to(gpu)
    reused = [dec.decode_slots(new[..., :4], pool, index, first_decode=True),
              dec.decode_slots(new[..., 4:], pool, index, first_decode=False)]
    fresh_pool = dec.new_state_pool(num_slots=3)
    fresh = [dec.decode_slots(new[..., :4], fresh_pool, index, first_decode=True),
             dec.decode_slots(new[..., 4:], fresh_pool, index, first_decode=False)]
    for r, f in zip(reused, fresh):
        assert torch.equal(r, f)


def test_small_decoder_graph_replay(small, gpu):
    state, dec = small
    pool = dec.new_state_pool(num_slots=4, capture_slots=2)
    runner = CodecGraphRunner(dec, pool, [GraphKey(2, 6, "first"), GraphKey(2, 6, "next")])
    runner.capture_all()
    codes = _codes(SMALL, 2, 12, 9).to(gpu)
    index = torch.tensor([1, 3], dtype=torch.int64, device=gpu)
    r1 = runner.run(codes[..., :6], index, first_decode=True)
    out1, graphed1 = r1.output, r1.graph
    out1 = out1.clone()
    r2 = runner.run(codes[..., 6:], index, first_decode=False)
    out2, graphed2 = r2.output, r2.graph
    assert graphed1 and graphed2
    eager_pool = dec.new_state_pool(num_slots=4)
    e1 = dec.decode_slots(codes[..., :6], eager_pool, index, first_decode=True)
    e2 = dec.decode_slots(codes[..., 6:], eager_pool, index, first_decode=False)
    assert torch.equal(out1, e1) and torch.equal(out2, e2)


def test_full_size_decoder_matches_oracle(gpu):
    """The Qwen3-Omni configuration itself (1024 hidden, 8 layers, 1536-channel decoder, x1920)
    on 1 row x 8 frames. Layer scales and ConvNeXt gammas of 0.1 (10x and 1e5x the initial
    values): the transformer and ConvNeXt branches move the output by far more than the
    tolerance (checked on the oracle), while bf16 operands through 8 layers keep the decode
    ~42 dB from float32 (at 0.3 the margin to the 2e-3 bound closes: ~40.4 dB, 2.03e-3)."""
    cfg = QWEN3_CODE2WAV
    state = make_qwen3_code2wav_weights(cfg, seed=1, branch_scale=0.1, activation_spread=0.1)
    dec = Qwen3Code2WavDecoder(state, cfg, device=gpu)
    codes = _codes(cfg, 1, 8, 2)
    got = dec.from_indices(codes.to(gpu))
    w = effective_weights(state)
    with torch.no_grad():
        ref = Q.qwen3_code2wav(codes, w, cfg)
        plain = Q.qwen3_code2wav(codes, {k: (torch.zeros_like(v) if k.endswith(
            ("layer_scale.scale", ".gamma")) else v) for k, v in w.items()}, cfg)
    assert (ref - plain).abs().max() > 20 * 2e-3  # the branches matter
    check_waveform(got, ref)


# ------------------------------------------------------------------------------ Qwen3-TTS

# hidden 256 with 8 heads of 64 (attention twice as wide as the residual stream), latent 512
TTS_SMALL = Qwen3TTSCodecConfig(codebook_size=64, num_quantizers=4, codebook_dim=32,
                                latent_dim=512, hidden_size=256, num_hidden_layers=2,
                                num_attention_heads=8, num_key_value_heads=2, intermediate_size=512,
                                sliding_window=8, decoder_dim=384, upsample_rates=(2, 3),
                                input_conv_gain=0.04)


@pytest.fixture(scope="module")
def tts_small(gpu):
    state = make_qwen3_code2wav_weights(TTS_SMALL, seed=2, branch_scale=0.5,
                                        activation_spread=0.1)
    return state, Qwen3TTSCodecDecoder(state, TTS_SMALL, device=gpu)


def test_tts_decoder_matches_oracle(tts_small, gpu):
    state, dec = tts_small
    codes = _codes(TTS_SMALL, 2, 17, 3)
    st = dec.init_state(2)
    got = dec.decode(codes.to(gpu), st)
    assert got.shape == (2, 1, 17 * TTS_SMALL.hop_length) and st.frame_position == 17
    with torch.no_grad():
        ref = Q.qwen3_tts_decode(codes, effective_weights(state), TTS_SMALL)
    check_waveform(got, ref)


def test_tts_decoder_chunks_equal_the_whole_decode(tts_small, gpu):
    """A stream decoded in chunks of 1..12 frames gives the whole decode's samples bit for bit
    (the chunks' transformer GEMMs run at 3..36 rows, the whole decode's at 75, in one summation
    order), within the oracle bounds."""
    state, dec = tts_small
    codes_cpu = _codes(TTS_SMALL, 3, 25, 4)
    codes = codes_cpu.to(gpu)
    whole = dec.decode(codes, dec.init_state(3)).cpu()
    st = dec.init_state(3)
    parts, s = [], 0
    for n in (1, 6, 12, 6):
        parts.append(dec.decode(codes[..., s:s + n], st).cpu())
        s += n
    streamed = torch.cat(parts, dim=-1)
    assert streamed.shape == whole.shape and torch.equal(streamed, whole)
    assert st.frame_position == 25 and st.frame_positions.tolist() == [25, 25, 25]
    with torch.no_grad():
        ref = Q.qwen3_tts_decode(codes_cpu, effective_weights(state), TTS_SMALL)
    check_waveform(streamed, ref)


def test_tts_decode_contract(tts_small, gpu):
    _, dec = tts_small
    st = dec.init_state(1)
    codes = _codes(TTS_SMALL, 1, 4, 5).to(gpu)
    with pytest.raises(ValueError, match="shaped"):
        dec.decode(codes[0], st)
    with pytest.raises(ValueError, match="at least one row"):
        dec.decode(codes[:0], st)
    with pytest.raises(ValueError, match="fresh frames"):
        dec.decode(codes[..., :0], st)
    with pytest.raises(RuntimeError, match="not precompiled"):
        dec.decode(codes, st, compiled=True)
    assert st.frame_position == 0
    dec.precompile(codes, st)
    assert st.frame_position == 4
    out = dec.decode(codes, st, compiled=True)
    assert out.shape == (1, 1, 4 * TTS_SMALL.hop_length) and st.frame_position == 8


def test_tts_full_size_decoder_matches_oracle(gpu):
    """The default Qwen3-TTS decoder shape (512 hidden, 16 x 64 attention, 1024 latent,
    1536-channel decoder, x1920) on 1 row x 6 frames."""
    cfg = QWEN3_TTS_CODEC
    state = make_qwen3_code2wav_weights(cfg, seed=3, branch_scale=0.1, activation_spread=0.1)
    dec = Qwen3TTSCodecDecoder(state, cfg, device=gpu)
    codes = _codes(cfg, 1, 6, 6)
    got = dec.decode(codes.to(gpu), dec.init_state(1))
    with torch.no_grad():
        ref = Q.qwen3_tts_decode(codes, effective_weights(state), cfg)
    check_waveform(got, ref)
