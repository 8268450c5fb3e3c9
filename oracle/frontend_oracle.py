"""CPU oracle of the bucket-masked fbank front end -- TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module.  Only ``tests/`` use it, as
the checker.

The encoder's input features: w2v-BERT 2.0's SeamlessM4T fbank of one 16 kHz
chunk padded with 160 zeros on each side (src/sidon_triton/frontend.py:1-15,
:175-216, :249-260):

  per 400-sample frame (hop 160), scaled by 2^15:
    remove the frame's mean; pre-emphasis y[0] = 0.03 x[0],
    y[n] = x[n] - 0.97 x[n-1]; Povey window (0.5 - 0.5 cos(2 pi n / 399))^0.85;
    512-point power spectrum (257 bins); 80 Kaldi mel bins (20 Hz - 8 kHz,
    triangles in mel space, mel(f) = 1127 ln(1 + f / 700));
    log(max(mel, 1.192092955078125e-07))
  per mel bin over the chunk's frames: (x - mean) / sqrt(var_ddof1 + 1e-7)
  an odd frame count gets one more frame of 1.0; frames are stacked in pairs
  -> [frames / 2, 160].

``fbank_bucketed`` is the masked form of frontend.py:218-240: a chunk
zero-padded to a bucket of S samples (a multiple of 320) with ``valid`` true
samples gives S / 320 rows whose valid part equals the exact-length features;
the statistics use the true frames only, the pad frame of 1.0 sits at its
exact position, and everything after it is 0.

Sources restated here (read, not run): src/sidon_triton/frontend.py:122-246
and transformers' ``SeamlessM4TFeatureExtractor`` / ``audio_utils.spectrogram``
/ ``audio_utils.mel_filter_bank`` (installed 5.15.0), the extractor the
reference reproduces.  Pinning: tests/test_frontend_oracle.py compares it with
golden vectors written by the installed extractor and mel_filter_bank
(tests/golden/make_fbank_golden.py), with planted mistakes, and with closed
forms (a DC-only frame has zero spectrum, the per-bin statistics of the
output are 0 and 1).
"""

from __future__ import annotations

import math

import numpy as np

SAMPLE_RATE = 16_000
FRAME_SIZE = 400
FRAME_SHIFT = 160
N_FFT = 512
N_BINS = N_FFT // 2 + 1
NUM_MEL = 80
PREEMPH = 0.97
MEL_FLOOR = 1.192092955078125e-07
VAR_EPS = 1e-7
PAD_VALUE = 1.0
KALDI_SCALE = 2.0 ** 15
EDGE_PAD = 160


def povey_window(n: int = FRAME_SIZE) -> np.ndarray:
    i = np.arange(n, dtype=np.float64)
    return (0.5 - 0.5 * np.cos(2 * math.pi * i / (n - 1))) ** 0.85


def kaldi_mel_banks(num_mel: int = NUM_MEL, low: float = 20.0, high: float = SAMPLE_RATE / 2) -> np.ndarray:
    """[257, num_mel] float64: triangles in Kaldi mel space over the rFFT bins."""

    def mel(f):
        return 1127.0 * np.log(1.0 + np.asarray(f, dtype=np.float64) / 700.0)

    lo, hi = mel(low), mel(high)
    delta = (hi - lo) / (num_mel + 1)
    left = lo + delta * np.arange(num_mel)
    center, right = left + delta, left + 2 * delta
    bins = mel(np.linspace(0.0, SAMPLE_RATE / 2, N_BINS))[:, None]
    up = (bins - left) / (center - left)
    down = (right - bins) / (right - center)
    return np.maximum(0.0, np.minimum(up, down))


def frame_features(padded: np.ndarray, frames: int, window=None, preemph: float = PREEMPH,
                   remove_dc: bool = True) -> np.ndarray:
    """log-mel [frames, 80] of an edge-padded signal (float64)."""
    window = povey_window() if window is None else window
    mel = kaldi_mel_banks()
    x = padded.astype(np.float64) * KALDI_SCALE
    idx = np.arange(frames)[:, None] * FRAME_SHIFT + np.arange(FRAME_SIZE)[None, :]
    fr = x[idx]
    if remove_dc:
        fr = fr - fr.mean(axis=1, keepdims=True)
    pre = fr.copy()
    pre[:, 1:] = fr[:, 1:] - preemph * fr[:, :-1]
    pre[:, 0] = fr[:, 0] * (1.0 - preemph)
    spec = np.fft.rfft(pre * window, n=N_FFT, axis=1)
    power = spec.real ** 2 + spec.imag ** 2
    return np.log(np.maximum(power @ mel, MEL_FLOOR))


def num_frames(samples: int) -> int:
    return 1 + (samples + 2 * EDGE_PAD - FRAME_SIZE) // FRAME_SHIFT


def normalize_stack(logmel: np.ndarray, ddof: int = 1) -> np.ndarray:
    """Per-bin normalization, odd-count pad frame, stride-2 stacking."""
    x = (logmel - logmel.mean(axis=0, keepdims=True)) / np.sqrt(logmel.var(axis=0, ddof=ddof, keepdims=True)
                                                                 + VAR_EPS)
    if x.shape[0] % 2:
        x = np.concatenate([x, np.full((1, NUM_MEL), PAD_VALUE)], axis=0)
    return x.reshape(x.shape[0] // 2, 2 * NUM_MEL)


def fbank_exact(chunk: np.ndarray, **kw) -> np.ndarray:
    """Features [ceil(frames / 2), 160] of one chunk of n samples (float64)."""
    chunk = np.asarray(chunk, dtype=np.float64)
    padded = np.pad(chunk, (EDGE_PAD, EDGE_PAD))
    ddof = kw.pop("ddof", 1)
    return normalize_stack(frame_features(padded, num_frames(chunk.shape[0]), **kw), ddof=ddof)


def fbank_bucketed(chunks: np.ndarray, valid) -> np.ndarray:
    """chunks [B, S] (S % 320 == 0, zero past each valid length), valid [B]
    -> [B, S / 320, 160]: the exact-length features of each item's valid
    samples, zeros after them."""
    chunks = np.asarray(chunks, dtype=np.float64)
    batch, samples = chunks.shape
    assert samples % (2 * FRAME_SHIFT) == 0
    out = np.zeros((batch, samples // (2 * FRAME_SHIFT), 2 * NUM_MEL))
    for b, n in enumerate(valid):
        feats = fbank_exact(chunks[b, :int(n)])
        out[b, :feats.shape[0]] = feats
    return out
