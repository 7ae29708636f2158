"""GPU parity of HiFT's transforms (the iSTFT tail after the config-4 body) against the float64
oracle, itself pinned to torch.stft / torch.istft: the forward spectrum (centred, reflect padding
in the kernel, and the reference kernel's pre-padded form), the overlap-add inverse, and the fused
exp / sin / inverse / clamp tail from the last conv's channels-last output. Float32 kernels with
one fixed summation order per output: bounds are float32 rounding of 16-32 term sums."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import codec_oracle as O
from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.hift import HiftStft, overlap_add_inverse, short_time_spectrum

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_fft,hop,rows,length", [(16, 4, 3, 1001), (16, 4, 1, 9), (32, 8, 2, 4099),
                                                     (8, 2, 5, 300), (16, 4, 2, 96000)])
def test_short_time_spectrum_matches_the_oracle(gpu, n_fft, hop, rows, length):
    gen = torch.Generator().manual_seed(n_fft * 7 + length)
    x = torch.randn(rows, length, generator=gen)
    st = HiftStft(O.hann_window(n_fft), hop, device=gpu)
    got = st.spectrum(x.to(gpu)).cpu()
    ref = O.stft_reference(x, O.hann_window(n_fft), n_fft, hop)
    assert got.shape == ref.shape
    torch.testing.assert_close(got.double(), ref, rtol=1e-5, atol=2e-5)
    # the reference kernel's form: the caller pads
    padded = F.pad(x[:, None], (n_fft // 2, n_fft // 2), mode="reflect")[:, 0].contiguous()
    got2 = short_time_spectrum(padded.to(gpu), st.forward_basis, hop).cpu()
    assert torch.equal(got2, got)


@pytest.mark.parametrize("n_fft,hop,rows,frames", [(16, 4, 3, 251), (16, 4, 1, 2), (32, 8, 2, 700),
                                                     (16, 4, 4, 24001)])
def test_overlap_add_inverse_matches_the_oracle(gpu, n_fft, hop, rows, frames):
    gen = torch.Generator().manual_seed(frames + n_fft)
    bins = n_fft // 2 + 1
    re = torch.randn(rows, bins, frames, generator=gen)
    im = torch.randn(rows, bins, frames, generator=gen)
    st = HiftStft(O.hann_window(n_fft), hop, device=gpu)
    got = overlap_add_inverse(re.to(gpu), im.to(gpu), st.inverse_basis, st.squared_window, hop).cpu()
    ref = O.istft_reference(re, im, O.hann_window(n_fft), n_fft, hop)
    assert got.shape == ref.shape
    torch.testing.assert_close(got.double(), ref, rtol=1e-5, atol=1e-5)


def test_spectrum_then_inverse_reconstructs_the_signal(gpu):
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(4, 24000, generator=gen)
    st = HiftStft(O.hann_window(16), 4, device=gpu)
    spec = st.spectrum(x.to(gpu))
    y = overlap_add_inverse(spec[:, :9].contiguous(), spec[:, 9:].contiguous(), st.inverse_basis,
                            st.squared_window, 4).cpu()
    torch.testing.assert_close(y, x[:, :y.shape[1]], rtol=0, atol=1e-5)


@pytest.mark.parametrize("rows,frames,channels", [(16, 4001, 18), (1, 3, 18), (3, 500, 24)])
def test_istft_tail_matches_the_oracle(gpu, rows, frames, channels):
    """The fused tail from a channels-last conv output (extra channels past 2 * bins ignored),
    with magnitudes around e^-3 (unclamped) and a band of rows driven past the clip and the clamp."""
    gen = torch.Generator().manual_seed(rows + frames)
    h = torch.randn(rows, frames, channels, generator=gen)
    h[..., :9] = h[..., :9] * 0.5 - 3.0
    if frames > 10:
        h[:, 5:9, :9] = 6.0  # exp(6) = 403 > 100: clipped, and loud enough to clamp
    st = HiftStft(O.hann_window(16), 4, device=gpu)
    got = st.tail(h.to(gpu)).cpu()
    ref = O.hift_istft_tail(h, O.hann_window(16), 16, 4)
    assert got.shape == ref.shape == (rows, 4 * (frames - 1))
    torch.testing.assert_close(got.double(), ref, rtol=1e-5, atol=2e-6)
    limit = torch.tensor(0.99, dtype=torch.float32)  # torch.clamp of a float32 tensor at 0.99
    assert (got.abs() <= limit).all()
    if frames > 10:
        assert (got.abs() == limit).any()  # the clamp engaged


def test_transforms_reject_bad_geometry(gpu):
    st = HiftStft(O.hann_window(16), 4, device=gpu)
    with pytest.raises(ValueError):
        short_time_spectrum(torch.zeros(2, 100, device=gpu), st.forward_basis, 3)  # hop !| n_fft
    with pytest.raises(ValueError):
        st.tail(torch.zeros(2, 10, 12, device=gpu))  # fewer than 2 * bins channels
    lib = N.load_library()
    out = torch.empty(1, 100, device=gpu)
    # too short to reflect-pad
    status = lib.omni_short_time_spectrum(out.data_ptr(), 1, 8, 100, 1, st.forward_basis.data_ptr(),
                                          9, 16, 4, out.data_ptr(), 3, N.stream_handle(gpu))
    assert status == N.INVALID_ARG
