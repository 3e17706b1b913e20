"""The mel front end's oracle (oracle_mel_spectrogram, a restatement of
Tests/Mel/ScalarMel.h), checked on the CPU against an independent numpy
spectrogram (np.fft.rfft over np.pad(mode="reflect") frames), against closed
forms (digital silence is the floor everywhere; a tone centred on a bin lands
in the band over that bin), and with planted mistakes (a symmetric window, edge
padding instead of reflect) that the numpy comparison must reject."""

import numpy as np
import pytest

from whispereacp_amd import synthetic as S


def numpy_mel(samples, filters, fft, hop, frames, window=None, pad_mode="reflect"):
    n = np.arange(fft)
    w = 0.5 * (1.0 - np.cos(2.0 * np.pi * n / fft)) if window is None else window
    padded = np.pad(samples.astype(np.float64), fft // 2, mode=pad_mode)
    index = np.arange(frames)[:, None] * hop + n[None, :]
    spectrum = np.fft.rfft(padded[index] * w[None, :], axis=1)
    power = spectrum.real ** 2 + spectrum.imag ** 2
    mel = np.log10(np.maximum(filters.astype(np.float64) @ power.T, 1e-10))
    return (np.maximum(mel, mel.max() - 8.0) + 4.0) / 4.0


def test_oracle_matches_numpy_fft(oracle):
    s = S.reduced_mel_shape()
    x = S.tone_and_noise(s.sample_count)
    f = S.triangular_filters(s.mel_count, s.bin_count)
    got = oracle.mel_spectrogram(x, f, s.fft_length, s.hop_length, s.frame_count)
    assert got.shape == (s.mel_count, s.frame_count)
    assert np.max(np.abs(got - numpy_mel(x, f, s.fft_length, s.hop_length, s.frame_count))) < 1e-9


def test_silence_is_the_floor_everywhere(oracle):
    s = S.reduced_mel_shape()
    got = oracle.mel_spectrogram(np.zeros(s.sample_count, np.float32), S.triangular_filters(s.mel_count, s.bin_count),
                                 s.fft_length, s.hop_length, s.frame_count)
    assert np.all(got == (-10.0 + 4.0) / 4.0)


def test_a_centred_tone_lands_in_its_band(oracle):
    s = S.reduced_mel_shape()
    bin_ = 11   # a tone exactly on bin 11 of the 64-point transform
    x = np.sin(2 * np.pi * bin_ * np.arange(s.sample_count) / s.fft_length).astype(np.float32)
    f = S.triangular_filters(s.mel_count, s.bin_count)
    got = oracle.mel_spectrogram(x, f, s.fft_length, s.hop_length, s.frame_count)
    frame = s.frame_count // 2
    assert int(np.argmax(got[:, frame])) == int(np.argmax(f[:, bin_]))
    # the clamp keeps everything within eight decades (two after the scale) of the peak
    assert got.max() - got.min() <= 2.0 + 1e-12


@pytest.mark.parametrize("mistake", ["symmetric_window", "edge_padding"])
def test_planted_mistakes_are_rejected(oracle, mistake):
    s = S.reduced_mel_shape()
    x = S.tone_and_noise(s.sample_count)
    f = S.triangular_filters(s.mel_count, s.bin_count)
    got = oracle.mel_spectrogram(x, f, s.fft_length, s.hop_length, s.frame_count)
    if mistake == "symmetric_window":
        wrong = numpy_mel(x, f, s.fft_length, s.hop_length, s.frame_count, window=np.hanning(s.fft_length))
    else:
        wrong = numpy_mel(x, f, s.fft_length, s.hop_length, s.frame_count, pad_mode="edge")
    assert np.max(np.abs(got - wrong)) > 1e-4
