"""``pack_linear`` (kernels/gemm.py) on the CPU: a merged gate / up weight [2 I, in] is stored in
blocks of 16 rows, gate block q then up block q, which is the layout ``omni_gemm``'s SiLU-mul
epilogue reads (output column 16 q + r from rows 32 q + r and 32 q + 16 + r)."""

import pytest
import torch

from sglang_omni_amd.kernels.gemm import pack_linear


def test_gated_rows_interleave_by_sixteen():
    inter, k = 64, 64
    w = torch.arange(2 * inter, dtype=torch.float32)[:, None].expand(2 * inter, k).contiguous()
    b = torch.arange(2 * inter, dtype=torch.float32) + 1000
    lw = pack_linear(w, b, gated=True)
    assert lw.out_features == inter and lw.in_features == k and lw.gated
    for col in range(inter):
        q, r = divmod(col, 16)
        assert lw.weight[32 * q + r, 0].item() == col  # gate row of output column col
        assert lw.weight[32 * q + 16 + r, 0].item() == inter + col  # its up row
        assert lw.bias[32 * q + r].item() == 1000 + col
        assert lw.bias[32 * q + 16 + r].item() == 1000 + inter + col


def test_plain_weight_is_bf16_as_stored():
    w = torch.randn(128, 192)
    lw = pack_linear(w)
    assert lw.weight.dtype == torch.bfloat16 and torch.equal(lw.weight, w.to(torch.bfloat16))
    assert lw.bias is None and lw.out_features == 128
    with pytest.raises(ValueError, match="multiples of 64"):
        pack_linear(torch.randn(96, 100))
