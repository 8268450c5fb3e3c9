"""The encoder's bucket-masked fbank front end on the MI355X library.

Mirrors ``SeamlessFbank`` of src/sidon_triton/frontend.py:175-246 (the GPU
twin of w2v-BERT 2.0's SeamlessM4T feature extractor) for chunks zero-padded
to a bucket of S samples (S a multiple of 320) with their true lengths:

  1. ``sidon_fbank_frames`` (HIP): pad (160, 160) and cut 400-sample frames
     with hop 160 -> [B, S / 160, 400];
  2. framing GEMM with the constant [400, 514] matrix of ``frame_transform``
     (DC removal, pre-emphasis 0.97, Povey window, 512-point rDFT, x 2^15),
     fp32 on rocBLAS with the kernel chosen by timing (``blas.gemm_nt``;
     gfx950 has no reduced-precision fp32 GEMM path, so
     the quiet bins keep full fp32, as frontend.py:178-180 requires);
  3. ``sidon_fbank_logmel`` (HIP): power, 80 Kaldi mel bins (sparse
     triangles), log(max(., 1.19e-7));
  4. ``sidon_fbank_normalize`` (HIP): per-bin mean / variance (ddof 1) over
     each item's true frames, the odd-count pad frame of 1.0, zeros after,
     written in the stride-2 stacked layout [B, S / 320, 160].

The valid rows equal the exact-length extractor's; ``valid_features`` gives
their count (frontend.py:243-246), the encoder's ``frames``.  Given a
workspace the call allocates nothing and can be captured into a HIP graph.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib
from .blas import gemm_nt
from .flexrel import _check_device_tensor, _stream_handle

SAMPLE_RATE = 16_000
FRAME_SIZE = 400
FRAME_SHIFT = 160
N_FFT = 512
N_BINS = N_FFT // 2 + 1
NUM_MEL = 80
PREEMPH = 0.97
KALDI_SCALE = 2.0 ** 15
EDGE_PAD = 160
BUCKET_QUANTUM = 2 * FRAME_SHIFT  # samples per encoder frame


def num_frames(samples: int) -> int:
    """fbank frames of a chunk of ``samples`` samples (before stacking)."""
    return 1 + (samples + 2 * EDGE_PAD - FRAME_SIZE) // FRAME_SHIFT


def num_features(samples: int) -> int:
    """Encoder frames (50 Hz) of a chunk of ``samples`` samples."""
    return (num_frames(samples) + 1) // 2


def valid_features(samples: torch.Tensor) -> torch.Tensor:
    """Encoder frames of chunks with ``samples`` true samples (elementwise)."""
    true_frames = (samples.to(torch.long) + 2 * EDGE_PAD - FRAME_SIZE) // FRAME_SHIFT + 1
    return (true_frames + 1) // 2


def _povey_window() -> np.ndarray:
    i = np.arange(FRAME_SIZE, dtype=np.float64)
    return (0.5 - 0.5 * np.cos(2.0 * math.pi * i / (FRAME_SIZE - 1))) ** 0.85


def frame_transform() -> torch.Tensor:
    """[400, 514] float64: a frame (in [-1, 1] units) -> (real 257 | imag 257)
    of its Kaldi-processed 512-point rDFT, x 2^15.  Every step is linear in the
    frame: y = W_dft . diag(window) . P . D . x with D the mean removal and P
    the pre-emphasis (y[0] = 0.03 x[0], y[n] = x[n] - 0.97 x[n-1])."""
    n = FRAME_SIZE
    dc = np.eye(n) - np.full((n, n), 1.0 / n)
    pre = np.eye(n)
    pre[0, 0] = 1.0 - PREEMPH
    pre[np.arange(1, n), np.arange(n - 1)] = -PREEMPH
    chain = _povey_window()[:, None] * (pre @ dc)
    k = np.arange(N_BINS, dtype=np.float64)[:, None]
    t = np.arange(n, dtype=np.float64)[None, :]
    angle = 2.0 * math.pi * k * t / N_FFT
    w = np.concatenate([np.cos(angle) @ chain, -np.sin(angle) @ chain], axis=0) * KALDI_SCALE
    return torch.from_numpy(np.ascontiguousarray(w.T))


def mel_banks(num_mel: int = NUM_MEL, low: float = 20.0, high: float = SAMPLE_RATE / 2) -> np.ndarray:
    """[257, num_mel] float64 Kaldi mel filters: triangles in mel space,
    mel(f) = 1127 ln(1 + f / 700), over the rFFT bin frequencies."""

    def mel(f):
        return 1127.0 * np.log1p(np.asarray(f, dtype=np.float64) / 700.0)

    edges = mel(low) + (mel(high) - mel(low)) / (num_mel + 1) * np.arange(num_mel + 2)
    bins = mel(np.linspace(0.0, SAMPLE_RATE / 2, N_BINS))[:, None]
    left, center, right = edges[None, :-2], edges[None, 1:-1], edges[None, 2:]
    return np.clip(np.minimum((bins - left) / (center - left), (right - bins) / (right - center)), 0.0, None)


def sparse_mel(dense: np.ndarray):
    """Sparse form of a [257, M] mel bank: (start bin [M] int32, length [M]
    int32, weights [M, max length] float32, zero-padded)."""
    mels = dense.shape[1]
    lo = np.zeros(mels, np.int32)
    length = np.zeros(mels, np.int32)
    spans = []
    for m in range(mels):
        nz = np.nonzero(dense[:, m])[0]
        if nz.size:
            lo[m], length[m] = nz[0], nz[-1] - nz[0] + 1
        spans.append(dense[lo[m]:lo[m] + length[m], m])
    weights = np.zeros((mels, max(1, int(length.max()))), np.float32)
    for m, span in enumerate(spans):
        weights[m, :span.size] = span
    return lo, length, weights


class Fbank:
    """Bucketed chunks [B, S] fp32 (+ true samples [B]) -> features
    [B, S / 320, 160] fp32 on the device."""

    def __init__(self, device="cuda") -> None:
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        # Kept as [514, 400] (rows K-contiguous), the w operand of
        # blas.gemm_nt (y = x . w^T); this order was also the faster one when
        # the GEMM ran on hipBLASLt (57.5 against 59.6 us at a 96 s chunk).
        self.weight_t = frame_transform().float().t().contiguous().to(device)
        lo, length, weights = sparse_mel(mel_banks())
        self.mel_lo = torch.from_numpy(lo).to(device)
        self.mel_len = torch.from_numpy(length).to(device)
        self.mel_w = torch.from_numpy(weights).to(device)

    def workspace(self, batch: int, samples: int) -> dict:
        """Buffers for calls of up to ``batch`` chunks of ``samples`` samples."""
        frames = samples // FRAME_SHIFT
        f32 = dict(device=self.device, dtype=torch.float32)
        nbytes = int(_lib.load().sidon_fbank_workspace_bytes(batch, frames))
        return {"batch": batch, "samples": samples, "frames": torch.empty(batch * frames * FRAME_SIZE, **f32),
                "spec": torch.empty(batch * frames * 2 * N_BINS, **f32),
                "logmel": torch.empty(batch * frames * NUM_MEL, **f32),
                "stats": torch.empty(max(4, nbytes // 4), **f32)}

    @torch.no_grad()
    def __call__(self, chunk: torch.Tensor, valid: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 workspace: dict | None = None) -> torch.Tensor:
        """chunk [B, S] fp32 on the device, zero past each item's true length
        (S % 320 == 0); valid int32 [B] true samples on the device (None: S).
        out: optional fp32 [B, S / 320, 160]."""
        if chunk.dim() != 2 or chunk.dtype != torch.float32:
            raise ValueError("chunk must be a float32 [B, S] tensor")
        batch, samples = chunk.shape
        if samples % BUCKET_QUANTUM or samples < BUCKET_QUANTUM:
            raise ValueError(f"S={samples} must be a positive multiple of {BUCKET_QUANTUM} (pad to the bucket)")
        device = self.device
        _check_device_tensor("chunk", chunk, device)
        if valid is None:
            valid = torch.full((batch,), samples, dtype=torch.int32, device=device)
        else:
            _check_device_tensor("valid", valid, device)
            if valid.dtype != torch.int32 or tuple(valid.shape) != (batch,) or not valid.is_contiguous():
                raise ValueError("valid must be a contiguous int32 [B] tensor")
        frames = samples // FRAME_SHIFT
        ws = workspace if workspace is not None else self.workspace(batch, samples)
        if ws["batch"] < batch or ws["samples"] < samples:
            raise ValueError("the workspace is smaller than the call")
        if not chunk.is_contiguous():
            chunk = chunk.contiguous()
        fr = ws["frames"][:batch * frames * FRAME_SIZE].view(batch * frames, FRAME_SIZE)
        lib = _lib.load()
        stream = _stream_handle(device)
        with torch.cuda.device(device):
            rc = lib.sidon_fbank_frames(chunk.data_ptr(), fr.data_ptr(), batch, samples, stream)
        _lib.check("sidon_fbank_frames", rc)
        spec = ws["spec"][:batch * frames * 2 * N_BINS].view(batch * frames, 2 * N_BINS)
        gemm_nt(fr, self.weight_t, spec)
        logmel = ws["logmel"][:batch * frames * NUM_MEL]
        if out is None:
            out = torch.empty(batch, frames // 2, 2 * NUM_MEL, device=device)
        elif (out.dtype != torch.float32 or tuple(out.shape) != (batch, frames // 2, 2 * NUM_MEL)
              or not out.is_contiguous()):
            raise ValueError("out must be a contiguous float32 [B, S / 320, 160] tensor")
        stats = ws["stats"]
        with torch.cuda.device(device):
            rc = lib.sidon_fbank_logmel(spec.data_ptr(), self.mel_w.data_ptr(), self.mel_lo.data_ptr(),
                                        self.mel_len.data_ptr(), self.mel_w.shape[1], logmel.data_ptr(),
                                        batch * frames, stream)
            _lib.check("sidon_fbank_logmel", rc)
            rc = lib.sidon_fbank_normalize(logmel.data_ptr(), valid.data_ptr(), stats.data_ptr(),
                                           stats.numel() * 4, out.data_ptr(), batch, frames, stream)
        _lib.check("sidon_fbank_normalize", rc)
        return out
