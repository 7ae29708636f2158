"""GPU parity of MOSS-TTS's fused multi-channel embedding sum: ChannelEmbeddingTables.embed
against the eager ordered sum of the channels' lookups (the reference's own contract,
tests/unit_test/moss_tts/test_input_embeddings.py:82-109: 33 channels of width 257, strided
int32 / int64 ids, moved storage, independent outputs) and against the oracle, bit for bit."""

from __future__ import annotations

import pytest
import torch

from oracle import codec_oracle as O
from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.channel_embedding import ChannelEmbeddingTables

pytestmark = pytest.mark.gpu


def _eager(token_ids: torch.Tensor, weights: list[torch.Tensor]) -> torch.Tensor:
    out = torch.zeros(token_ids.shape[0], weights[0].shape[1], device=weights[0].device,
                      dtype=weights[0].dtype)
    for c, w in enumerate(weights):
        out = out + w[token_ids[:, c].long()]
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("token_dtype", [torch.int32, torch.int64])
def test_matches_the_eager_ordered_sum_through_storage_changes(gpu, dtype, token_dtype):
    g = torch.Generator(device=gpu).manual_seed(42)
    weights = [torch.randn(128, 257, device=gpu, dtype=dtype, generator=g) for _ in range(33)]
    tables = ChannelEmbeddingTables()
    assert tables.refresh(weights)
    token_ids = torch.randint(0, 128, (17, 66), device=gpu, dtype=token_dtype, generator=g)[:, ::2]
    for moved in (weights, [w.clone() * 2 for w in weights]):
        assert tables.refresh(moved)
        actual = tables.embed(token_ids, moved)
        assert actual.dtype == dtype and actual.shape == (17, 257)
        assert torch.equal(actual, _eager(token_ids, moved))
        assert torch.equal(actual.cpu(), O.channel_embedding_sum(token_ids.cpu(), [w.cpu() for w in moved]))
        saved = actual.clone()
        tables.embed(token_ids, moved).zero_()
        assert torch.equal(actual, saved)
    assert not tables.refresh([weights[0].t()])
    assert tables.embed(token_ids[:0], moved).shape == (0, 257)


@pytest.mark.parametrize("hidden", [8, 1024, 2048, 2056, 4096, 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_widths_vocabularies_and_out_of_range_ids(gpu, hidden, dtype):
    """The 16-byte path (hidden % 8 == 0), the element path, several column blocks per row,
    tables of different vocabulary sizes, and ids outside a table adding nothing."""
    g = torch.Generator().manual_seed(hidden)
    vocab = [1025, 7, 300, 1, 64]
    weights_cpu = [torch.randn(v, hidden, generator=g).to(dtype) for v in vocab]
    ids = torch.stack([torch.randint(-3, v + 3, (45,), generator=g) for v in vocab], dim=1)
    ids[0] = torch.tensor([1024, 6, 299, 0, 63])  # each table's last row
    ids[1] = torch.tensor([-1, 7, 300, 1, 64])  # every id just out of range
    weights = [w.to(gpu) for w in weights_cpu]
    tables = ChannelEmbeddingTables()
    assert tables.refresh(weights)
    actual = tables.embed(ids.to(gpu), weights).cpu()
    expected = O.channel_embedding_sum(ids, weights_cpu)
    assert torch.equal(actual.view(torch.int32 if dtype == torch.float32 else torch.int16),
                       expected.view(torch.int32 if dtype == torch.float32 else torch.int16))
    assert torch.equal(actual[1], torch.zeros(hidden, dtype=dtype))


def test_unaligned_tables_take_the_element_path(gpu):
    """Contiguous tables whose storage starts 2 bytes past a 16-byte boundary."""
    g = torch.Generator().manual_seed(5)
    hidden = 64
    flat = [torch.randn(50 * hidden + 1, generator=g).to(torch.bfloat16) for _ in range(4)]
    weights_cpu = [f[1:].view(50, hidden) for f in flat]
    weights = [f.to(gpu)[1:].view(50, hidden) for f in flat]
    assert all(w.data_ptr() % 16 == 2 and w.is_contiguous() for w in weights)
    ids = torch.randint(0, 50, (9, 4), generator=g)
    tables = ChannelEmbeddingTables()
    assert tables.refresh(weights)
    got = tables.embed(ids.to(gpu), weights).cpu()
    assert torch.equal(got.view(torch.int16), O.channel_embedding_sum(ids, weights_cpu).view(torch.int16))


def test_refuses_what_cannot_be_fused(gpu):
    w = [torch.randn(4, 8, device=gpu, dtype=torch.bfloat16) for _ in range(2)]
    tables = ChannelEmbeddingTables()
    assert not tables.refresh([w[0], w[1].float()])  # mixed dtypes
    assert not tables.refresh([w[0], torch.randn(4, 16, device=gpu, dtype=torch.bfloat16)])
    assert not tables.refresh([w[0].cpu(), w[1].cpu()])
    assert not tables.refresh([w[0].to(torch.float64), w[1].to(torch.float64)])
    with pytest.raises(N.OmniCodecError):
        tables.embed(torch.zeros(3, 2, dtype=torch.int64, device=gpu), w)  # never refreshed
    assert tables.refresh(w)
    with pytest.raises(N.OmniCodecError):
        tables.embed(torch.zeros(3, 2, dtype=torch.int64), w)  # ids on the host
    with pytest.raises(ValueError):
        tables.embed(torch.zeros(3, 3, dtype=torch.int64, device=gpu), w)


@pytest.mark.parametrize("rows,hidden,channels,dtype", [
    (600, 2056, 70, torch.bfloat16),   # 256-thread workgroups, two channel chunks
    (5, 24, 65, torch.float32),        # 64-thread workgroups, a one-channel second chunk
    (700, 2048, 33, torch.float16),    # the MOSS-TTS channel count at prefill size
])
def test_many_channels_and_both_workgroup_sizes(gpu, rows, hidden, channels, dtype):
    g = torch.Generator().manual_seed(rows + channels)
    vocab = [int(v) for v in torch.randint(1, 40, (channels,), generator=g)]
    weights_cpu = [torch.randn(v, hidden, generator=g).to(dtype) for v in vocab]
    ids = torch.stack([torch.randint(-1, v + 1, (rows,), generator=g) for v in vocab], dim=1)
    ids32 = ids.to(torch.int32)
    weights = [w.to(gpu) for w in weights_cpu]
    tables = ChannelEmbeddingTables()
    assert tables.refresh(weights)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    expected = O.channel_embedding_sum(ids, weights_cpu).view(bits)
    assert torch.equal(tables.embed(ids.to(gpu), weights).cpu().view(bits), expected)
    assert torch.equal(tables.embed(ids32.to(gpu), weights).cpu().view(bits), expected)
