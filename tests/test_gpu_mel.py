"""The mel front end on the MI355X against the oracle
(oracle_mel_spectrogram, pinned in tests/test_mel_oracle.py), as
Tests/Mel/MelSpectrogramTests.cpp checks it: the reduced shape cell by cell
within 1e-4, and Whisper's own shape (30 s, 80 bands, 3000 frames) with a
silent first second, whose output spans exactly two, plus the oracle's cells.
Then the chain into the encoder: the GPU mel fed to the GPU encoder against
the oracle's mel fed to the oracle's encoder."""

import numpy as np
import pytest
import torch

from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu


def gpu_mel(shape, samples, filters):
    from whispereacp_amd.mel import MelSpectrogram
    front = MelSpectrogram(shape)
    out = torch.empty((shape.mel_count, shape.frame_count), dtype=torch.float32, device="cuda")
    front.encode(torch.from_numpy(samples).cuda(), torch.from_numpy(filters).cuda(), out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_reduced_shape_matches_oracle(oracle):
    s = S.reduced_mel_shape()
    x = S.tone_and_noise(s.sample_count)
    f = S.triangular_filters(s.mel_count, s.bin_count)
    got = gpu_mel(s, x, f)
    expected = oracle.mel_spectrogram(x, f, s.fft_length, s.hop_length, s.frame_count)
    err = float(np.max(np.abs(got - expected)))
    print(f"reduced mel: worst absolute error {err:.2e}")
    assert err <= 1e-4


def test_whisper_shape_spans_two_and_matches_oracle(oracle):
    s = S.MelShape()
    x = S.tone_and_noise(s.sample_count)
    x[:16000] = 0.0   # a silent first second reaches the floor
    f = S.triangular_filters(s.mel_count, s.bin_count)
    got = gpu_mel(s, x, f)
    assert got.shape == (80, 3000)
    assert abs((got.max() - got.min()) - 2.0) <= 1e-5
    expected = oracle.mel_spectrogram(x, f, s.fft_length, s.hop_length, s.frame_count)
    err = float(np.max(np.abs(got - expected)))
    print(f"whisper-shape mel: worst absolute error {err:.2e}")
    assert err <= 1e-4


def test_mel_into_encoder_matches_the_oracle_chain(oracle):
    from whispereacp_amd.encoder import Encoder, EncoderWeights
    from whispereacp_amd.mel import MelSpectrogram
    s = S.MelShape()
    x = S.tone_and_noise(s.sample_count)
    f = S.triangular_filters(s.mel_count, s.bin_count)
    shape = S.encoder_workload_shape("tiny.en")
    encoder_file = S.workload_encoder_file(shape, "F16", 3000)
    front = MelSpectrogram(s)
    mel = torch.empty((80, 3000), dtype=torch.float32, device="cuda")
    front.encode(torch.from_numpy(x).cuda(), torch.from_numpy(f).cuda(), mel)
    rows = torch.empty((shape.positions(), shape.width), dtype=torch.float32, device="cuda")
    Encoder(shape).encode(mel, EncoderWeights(shape, encoder_file), rows)
    torch.cuda.synchronize()
    mel_expected = oracle.mel_spectrogram(x, f, s.fft_length, s.hop_length, s.frame_count)
    tensors = [encoder_file[n].floats() for n in S.encoder_canonical_names(shape.layers)]
    expected = oracle.encode(shape, tensors, mel_expected.astype(np.float32))
    got = rows.cpu().numpy()
    err = float(np.max(np.abs(got - expected) / (1 + np.abs(expected))))
    print(f"mel -> tiny.en encoder: worst error {err:.2e}")
    assert err <= 1e-4
