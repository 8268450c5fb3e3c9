"""Write golden vectors for the fbank front end with the installed transformers
``SeamlessM4TFeatureExtractor`` (padding_value 1.0, the w2v-bert-2.0
preprocessor setting the reference uses, src/sidon_triton/frontend.py:249-260)
and ``audio_utils.mel_filter_bank`` (the Kaldi mel bank of frontend.py:159-172).

transformers is a third-party library, not the reference; it runs here and only
its outputs are committed (.npz).  The chunks are regenerated from a seed by
``fbank_chunk`` (speech-like: a few decaying tones plus noise, |x| < 1), each
padded (160, 160) before the extractor as the demo does.  Run:
python tests/golden/make_fbank_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# name: (samples, seed); frame counts 1 + (n - 80) // 160 of both parities
CASES = {
    "fbank_n16123": (16123, 41),
    "fbank_n8000": (8000, 42),
    "fbank_n24007": (24007, 43),
    "fbank_n3280": (3280, 44),
}


def fbank_chunk(samples: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    t = np.arange(samples) / 16000.0
    x = 0.02 * rng.standard_normal(samples)
    for _ in range(4):
        f = rng.uniform(80.0, 4000.0)
        x += rng.uniform(0.05, 0.2) * np.sin(2 * np.pi * f * t + rng.uniform(0, 6.3)) * np.exp(-t * rng.uniform(0.1, 2))
    return (x / max(1.0, np.abs(x).max() / 0.9)).astype(np.float32)


def main() -> None:
    from transformers import SeamlessM4TFeatureExtractor
    from transformers.audio_utils import mel_filter_bank

    mel = mel_filter_bank(num_frequency_bins=257, num_mel_filters=80, min_frequency=20, max_frequency=8000,
                          sampling_rate=16000, norm=None, mel_scale="kaldi", triangularize_in_mel_space=True)
    np.savez_compressed(HERE / "fbank_mel_bank.npz", mel=np.asarray(mel, dtype=np.float64))
    fe = SeamlessM4TFeatureExtractor(padding_value=1.0)
    for name, (samples, seed) in CASES.items():
        x = fbank_chunk(samples, seed)
        feats = fe(np.pad(x, (160, 160)), sampling_rate=16000, return_tensors="np")["input_features"][0]
        np.savez_compressed(HERE / f"{name}.npz", expected=feats.astype(np.float32))
        print(name, feats.shape)


if __name__ == "__main__":
    main()
