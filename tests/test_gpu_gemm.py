"""``omni_gemm`` (the code2wav front's linear layers, kernels/gemm.py) against a plain PyTorch
float32 reference of the same op on the same bf16 operands: every epilogue (STORE, SILU_MUL with
the 16-row interleave of a merged gate / up weight, GELU, SCALED_RESIDUAL into float32 in place and
into bf16), every tile, ragged row counts and strided rows; then the property the streaming decode
relies on: a row's bits do not depend on the rows batched with it, nor on the tile. Last, the qkv
GEMM with the rotary embedding and the K / V ring writes in its epilogue (``linear_rope_kv``)
against ``linear`` followed by ``rope_kv_write``: the same bits in qkv and in the rings."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels import code2wav_front as F
from sglang_omni_amd.kernels.gemm import (GELU, SCALED_RESIDUAL, SILU_MUL, STORE, linear,
                                          linear_rope_kv, pack_linear)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _no_tf32():
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev


def _operands(rows, k, n, seed, gpu, bias=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, generator=g) / math.sqrt(k)
    b = torch.randn(n, generator=g) * 0.1 if bias else None
    return x.to(gpu), w, b


def _ref_acc(x, w, b):
    """float32 reference of x @ W^T (+ b) on the bf16-rounded operands."""
    acc = x.float() @ w.to(torch.bfloat16).float().to(x.device).t()
    return acc if b is None else acc + b.to(x.device)


def _close(got, want, what):
    err = (got.float() - want).abs().max().item()
    # bf16 output: half an ulp of the value; float32 accumulation over k: far below
    bound = (want.abs() * 2.0 ** -8 + 1e-4).max().item() if got.dtype == torch.bfloat16 else 1e-4
    assert err <= bound, f"{what}: max|err| {err:.3g} > {bound:.3g}"
    if got.dtype == torch.bfloat16:
        assert torch.all((got.float() - want).abs() <= want.abs() * 2.0 ** -8 + 1e-4), what


@pytest.mark.parametrize("rows,k,n,config", [(768, 1024, 3072, 0), (768, 1024, 3072, 2),
                                             (100, 512, 192, 4), (1, 1024, 1024, 0),
                                             (3072, 4096, 1024, 1), (200, 1024, 256, 6)])
def test_store(gpu, rows, k, n, config):
    x, w, b = _operands(rows, k, n, rows + k + n, gpu, bias=n == 192)
    lw = pack_linear(w, b).to(gpu)
    out = torch.full((rows, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    if config in (1, 3, 6) and n % 128:
        pytest.skip("64 x 128 tiles need n % 128 == 0")
    linear(x, lw, out, config=config)
    _close(out, _ref_acc(x, w, b), f"store {rows}x{k}x{n}")


@pytest.mark.parametrize("rows,k,inter", [(768, 1024, 3072), (37, 512, 1024)])
def test_silu_mul(gpu, rows, k, inter):
    x, w, _ = _operands(rows, k, 2 * inter, 5 + rows, gpu)
    lw = pack_linear(w, gated=True).to(gpu)
    out = torch.empty(rows, inter, dtype=torch.bfloat16, device=gpu)
    linear(x, lw, out)
    acc = _ref_acc(x, w, None)
    gate, up = acc[:, :inter], acc[:, inter:]
    _close(out, torch.nn.functional.silu(gate) * up, "silu_mul")


def test_gelu(gpu):
    x, w, b = _operands(1536, 1024, 4096, 7, gpu, bias=True)
    lw = pack_linear(w, b).to(gpu)
    out = torch.empty(1536, 4096, dtype=torch.bfloat16, device=gpu)
    linear(x, lw, out, epilogue=GELU)
    _close(out, torch.nn.functional.gelu(_ref_acc(x, w, b)), "gelu")


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_scaled_residual(gpu, out_dtype):
    rows, k, n = 700, 3072, 1024
    x, w, b = _operands(rows, k, n, 9, gpu, bias=out_dtype == torch.bfloat16)
    lw = pack_linear(w, b).to(gpu)
    g = torch.Generator().manual_seed(10)
    r = torch.randn(rows, n, generator=g).to(gpu)
    scale = (torch.rand(n, generator=g) * 0.02).to(gpu)
    want = r + scale * _ref_acc(x, w, b)
    if out_dtype == torch.float32:
        h = r.clone()
        linear(x, lw, h, epilogue=SCALED_RESIDUAL, scale=scale, residual=h)  # in place
        _close(h, want, "scaled residual in place")
    else:
        z = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
        linear(x, lw, z, epilogue=SCALED_RESIDUAL, scale=scale, residual=r)
        _close(z, want, "scaled residual to bf16")


def test_strided_rows(gpu):
    """x rows inside a wider buffer, out rows inside a wider buffer."""
    rows, k, n = 130, 1024, 512
    x, w, _ = _operands(rows, k, n, 11, gpu)
    wide = torch.zeros(rows, k + 64, dtype=torch.bfloat16, device=gpu)
    wide[:, 32:32 + k] = x
    out_wide = torch.zeros(rows, n + 128, dtype=torch.bfloat16, device=gpu)
    lw = pack_linear(w).to(gpu)
    linear(wide[:, 32:32 + k], lw, out_wide[:, 64:64 + n])
    _close(out_wide[:, 64:64 + n], _ref_acc(x, w, None), "strided")
    assert torch.all(out_wide[:, :64] == 0) and torch.all(out_wide[:, 64 + n:] == 0)


@pytest.mark.parametrize("epilogue", [STORE, SILU_MUL, GELU, SCALED_RESIDUAL])
def test_rows_are_batch_invariant(gpu, epilogue):
    """Each row's bits are the same whatever rows it is batched with and whichever tile runs it:
    the streaming decode's chunked == whole property."""
    k, n = 1024, 2048
    x, w, b = _operands(768, k, n, 13, gpu, bias=True)
    lw = pack_linear(w, b, gated=epilogue == SILU_MUL).to(gpu)
    cols = lw.out_features
    g = torch.Generator().manual_seed(14)
    r = torch.randn(768, cols, generator=g).to(gpu)
    scale = torch.rand(cols, generator=g).to(gpu)

    def run(xs, config):
        out = torch.empty(xs.shape[0], cols, dtype=torch.bfloat16, device=gpu)
        kw = {}
        if epilogue == SCALED_RESIDUAL:
            kw = {"scale": scale, "residual": r[:xs.shape[0]]}
        return linear(xs, lw, out, epilogue=epilogue, config=config, **kw)

    whole = run(x, 1)
    for config in (2, 3, 4, 5, 6):
        if config == 4 and epilogue == SILU_MUL:
            continue
        assert torch.equal(run(x, config), whole), config
    for rows in (1, 63, 65, 200):
        assert torch.equal(run(x[:rows], 0), whole[:rows]), rows
        assert torch.equal(run(x[:rows].contiguous(), 5), whole[:rows]), rows


def test_contract(gpu):
    x, w, _ = _operands(64, 1024, 256, 15, gpu)
    lw = pack_linear(w).to(gpu)
    with pytest.raises(ValueError, match="multiples of 64"):
        pack_linear(torch.randn(100, 1024))
    with pytest.raises(ValueError, match="silu_mul"):
        linear(x, lw, torch.empty(64, 256, dtype=torch.bfloat16, device=gpu), epilogue=SILU_MUL)
    with pytest.raises(ValueError, match="out must be"):
        linear(x, lw, torch.empty(64, 256, device=gpu))
    # rows = 0 does nothing; a k that is not a multiple of 64 is refused by the library
    lib = N.load_library()
    args = N.GemmArgs()
    out = torch.empty(64, 256, dtype=torch.bfloat16, device=gpu)
    args.a, args.a_stride, args.w = x.data_ptr(), 1024, lw.weight.data_ptr()
    args.rows, args.k, args.n = 0, 1024, 256
    args.out, args.out_stride, args.out_dtype = out.data_ptr(), 256, N.DTYPE_BF16
    assert lib.omni_gemm(ctypes.byref(args), N.stream_handle(gpu)) == N.OK
    args.rows, args.k = 64, 1000
    assert lib.omni_gemm(ctypes.byref(args), N.stream_handle(gpu)) == N.INVALID_ARG
    args.k, args.out_dtype = 1024, N.DTYPE_F32  # float32 out only for the scaled residual
    assert lib.omni_gemm(ctypes.byref(args), N.stream_handle(gpu)) == N.INVALID_ARG


def _inv_freq(gpu, theta=10000.0):
    return (1.0 / (theta ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))).to(gpu)


@pytest.mark.parametrize("batch,frames,heads,kv_heads,bias,config",
                         [(3, 11, 4, 2, False, 0), (64, 12, 16, 16, False, 0),
                          (2, 37, 2, 1, True, 1), (1, 1, 4, 4, True, 6), (5, 40, 8, 4, False, 1)])
def test_rope_kv_epilogue_first_decode(gpu, batch, frames, heads, kv_heads, bias, config):
    """A first decode (cold, no rings): the rotated q and k at positions 0 .. frames - 1."""
    rows, k, n = batch * frames, 1024, (heads + 2 * kv_heads) * 64
    x, w, b = _operands(rows, k, n, rows + n, gpu, bias=bias)
    lw = pack_linear(w, b).to(gpu)
    ref = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
    linear(x, lw, ref)
    F.rope_kv_write(ref, batch, heads, kv_heads, 64, _inv_freq(gpu))
    got = torch.full((rows, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    linear_rope_kv(x, lw, got, batch, heads, kv_heads, 64, _inv_freq(gpu), config=config)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("cold", [False, True])
def test_rope_kv_epilogue_rings(gpu, cold):
    """Rows at their slots' positions (one far along, one slot out of range, one slot -1): qkv
    and both rings hold the bits of the two-launch form, other ring rows untouched."""
    batch, frames, heads, kv_heads, ring_frames, slots = 4, 7, 4, 2, 10, 6
    rows, k, n = batch * frames, 512, (heads + 2 * kv_heads) * 64
    x, w, b = _operands(rows, k, n, 21, gpu, bias=True)
    lw = pack_linear(w, b).to(gpu)
    positions = torch.tensor([0, 40, 7, 1000, 123457, 3], dtype=torch.int64, device=gpu)
    index = torch.tensor([3, 1, -1, 9], dtype=torch.int64, device=gpu)
    g = torch.Generator().manual_seed(22)
    keys = torch.randn(slots * ring_frames, kv_heads * 64, generator=g).to(torch.bfloat16).to(gpu)
    values = torch.randn(slots * ring_frames, kv_heads * 64, generator=g).to(torch.bfloat16).to(gpu)
    ring = dict(slot_index=index, positions=positions, cold=cold, ring_frames=ring_frames)
    ref = torch.empty(rows, n, dtype=torch.bfloat16, device=gpu)
    k_ref, v_ref = keys.clone(), values.clone()
    linear(x, lw, ref)
    F.rope_kv_write(ref, batch, heads, kv_heads, 64, _inv_freq(gpu), key_ring=k_ref,
                    value_ring=v_ref, **ring)
    got = torch.full((rows, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    k_got, v_got = keys.clone(), values.clone()
    linear_rope_kv(x, lw, got, batch, heads, kv_heads, 64, _inv_freq(gpu), key_ring=k_got,
                   value_ring=v_got, **ring)
    assert torch.equal(got, ref)
    assert torch.equal(k_got, k_ref) and torch.equal(v_got, v_ref)
    assert not torch.equal(k_got, keys)  # the in-range rows were written


def test_rope_kv_epilogue_contract(gpu):
    x, w, _ = _operands(24, 512, 512, 23, gpu)
    lw = pack_linear(w).to(gpu)
    qkv = torch.empty(24, 512, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="rings"):
        linear_rope_kv(x, lw, qkv, 2, 4, 2, 64, _inv_freq(gpu), slot_index=torch.zeros(
            2, dtype=torch.int64, device=gpu), key_ring=torch.empty(
            40, 64, dtype=torch.bfloat16, device=gpu), value_ring=torch.empty(
            40, 64, dtype=torch.bfloat16, device=gpu), ring_frames=10)
    with pytest.raises(ValueError, match="batch"):
        linear_rope_kv(x, lw, qkv, 5, 4, 2, 64, _inv_freq(gpu))
    # n must be (heads + 2 kv_heads) * 64; head_dim 64 only
    lib = N.load_library()
    args = N.GemmArgs()
    args.a, args.a_stride, args.w = x.data_ptr(), 512, lw.weight.data_ptr()
    args.rows, args.k, args.n = 24, 512, 512
    args.out, args.out_stride, args.out_dtype = qkv.data_ptr(), 512, N.DTYPE_BF16
    inv = _inv_freq(gpu)
    call = lambda heads, kv, hd: lib.omni_gemm_rope_kv(
        ctypes.byref(args), 12, heads, kv, hd, inv.data_ptr(), None, None, 1, 0, None, None, 0,
        N.stream_handle(gpu))
    assert call(2, 2, 64) == N.INVALID_ARG
    assert call(4, 2, 32) == N.UNSUPPORTED
    assert call(4, 2, 64) == N.OK
