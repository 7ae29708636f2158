"""The allocation-free split-K entry point (``omni_conv1d_splitk_noalloc``): its partials in the
library's static per-GPU array instead of a workspace argument. Through the C ABI, on two calls in
a row (the second smaller, so it runs over what the first left in the array), it gives the bits
of ``omni_conv1d_splitk`` with a workspace; partials beyond the array are refused before any
launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import _conv_args, pack_conv1d, splitk_workspace_elements

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def operands(rows, c_in, c_out, seed, gpu):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(1, rows, c_in, generator=gen).to(torch.bfloat16).to(gpu)
    w = (torch.randn(c_out, c_in, 1, generator=gen) / c_in ** 0.5).to(torch.bfloat16).float()
    b = (torch.randn(c_out, generator=gen) * 0.1).to(torch.bfloat16).float()
    return x, pack_conv1d(w, b).to(gpu)


def test_noalloc_split_gemm_equals_the_workspace_entry_on_two_calls(gpu):
    lib = N.load_library()
    stream = N.stream_handle(gpu)
    for rows, c_in, c_out, splits, seed in ((700, 1024, 1024, 4, 1), (45, 768, 384, 2, 2)):
        x, packed = operands(rows, c_in, c_out, seed, gpu)
        ws = torch.empty(splitk_workspace_elements(x, packed, splits), device=gpu)
        expected = torch.empty(1, rows, c_out, dtype=torch.bfloat16, device=gpu)
        args = _conv_args(x, packed, expected)
        assert lib.omni_conv1d_splitk(ctypes.byref(args), splits, ws.data_ptr(), ws.numel() * 4,
                                      N.CONV_KERNEL_AUTO, 0, stream) == 0
        got = torch.full((1, rows, c_out), float("nan"), dtype=torch.bfloat16, device=gpu)
        args = _conv_args(x, packed, got)
        assert lib.omni_conv1d_splitk_noalloc(ctypes.byref(args), splits, N.CONV_KERNEL_AUTO, 0,
                                              stream) == 0
        torch.cuda.synchronize(gpu)
        assert torch.equal(got, expected)
        ref = x.double().cpu()[0] @ packed_weight_t(packed).double() + packed.bias.double().cpu()
        assert (got[0].double().cpu() - ref).abs().max().item() < 2e-2 * ref.abs().max().item()


def packed_weight_t(packed):
    """The packed k = 1 weight [chunks, n_cols, 1, 32] back as [c_in, n_cols] (CPU)."""
    w = packed.weight.float().cpu()[:, :, 0, :]  # [chunks, n, 32]
    return w.permute(0, 2, 1).reshape(-1, w.shape[1])[: packed.c_in]


def test_noalloc_refuses_partials_beyond_its_array(gpu):
    lib = N.load_library()
    rows, c_in, c_out, splits = 8192, 256, 1024, 4  # 4 * 8192 * 1024 * 4 bytes = 128 MiB
    assert splits * rows * c_out * 4 > SCRATCH_BYTES
    x, packed = operands(rows, c_in, c_out, 3, gpu)
    out = torch.zeros(1, rows, c_out, dtype=torch.bfloat16, device=gpu)
    args = _conv_args(x, packed, out)
    status = lib.omni_conv1d_splitk_noalloc(ctypes.byref(args), splits, N.CONV_KERNEL_AUTO, 0,
                                            N.stream_handle(gpu))
    assert status == N.UNSUPPORTED
    torch.cuda.synchronize(gpu)
    assert not out.any()  # nothing ran
