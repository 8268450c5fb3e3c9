"""Bucketed HIP-graph runtime for the encoder.

Mirrors the encoder side of src/sidon_triton/runtime.py:

  * flat max-size device buffers (features, valid frames, hidden) re-viewed
    per (batch, bucket), allocated once (:140-156 of ``EngineSet``);
  * a chunk runs zero-padded to its bucket with its true length passed
    alongside, so every chunk of a bucket shares one captured graph: 1 s
    buckets up to 32 s, 4 s buckets above, capped at the maximum (:366-372;
    here in 50 Hz frames: 50-frame steps up to 1600 frames, 200-frame steps
    above);
  * graphs keyed by (batch, bucket), captured after a warm-up on a side
    stream, drawing from one shared memory pool, least recently used evicted
    past ``max_graphs`` (:374-401, via ``graphs.BucketGraphs``);
  * all work enqueued on a non-default compute stream (:27, :360).

The valid rows of a bucketed run equal an exact-length run: the front end
takes its statistics over the true frames only, the attention masks the
padded keys, the depthwise conv is causal and every other op is row-wise.

Two entries: ``run`` takes 160-channel features (bucketed in frames);
``run_wave`` takes 16 kHz waveforms and runs the fbank front end and the
encoder in one graph per (batch, bucket), bucketed in samples exactly as
runtime.py:366-372 does.  The decoder is not part of this runtime.
"""

from __future__ import annotations

import torch

from .encoder import HipEncoder
from .frontend import BUCKET_QUANTUM, Fbank, num_features
from .graphs import BucketGraphs

FRAME_RATE = 50                 # encoder frames per second
FINE_BUCKET_FRAMES = 50         # 1 s
FINE_LIMIT_FRAMES = 32 * 50     # 32 s
COARSE_BUCKET_FRAMES = 4 * 50   # 4 s
IN_RATE = 16_000
FINE_BUCKET_SAMPLES = IN_RATE           # 1 s
FINE_LIMIT_SAMPLES = 32 * IN_RATE       # 32 s
COARSE_BUCKET_SAMPLES = 4 * IN_RATE     # 4 s
MIN_SEQ = 2


def bucket_frames(frames: int, max_frames: int) -> int:
    """Bucket length (frames) of a chunk with ``frames`` valid frames."""
    if frames < 1:
        raise ValueError("a chunk needs at least one frame")
    step = FINE_BUCKET_FRAMES if frames <= FINE_LIMIT_FRAMES else COARSE_BUCKET_FRAMES
    return min(max_frames, -(-frames // step) * step)


def bucket_samples(samples: int, max_samples: int) -> int:
    """Bucket length (samples, a multiple of 320) of a chunk of ``samples``
    samples (runtime.py:366-372)."""
    if samples < 1:
        raise ValueError("a chunk needs at least one sample")
    step = FINE_BUCKET_SAMPLES if samples <= FINE_LIMIT_SAMPLES else COARSE_BUCKET_SAMPLES
    return min(max_samples, -(-samples // step) * step)


class EncoderRuntime:
    """Encoder calls on bucketed, graph-captured, fixed-address buffers."""

    def __init__(self, encoder: HipEncoder, max_batch: int = 1, max_seconds: float = 96.0,
                 use_graph: bool = True, max_graphs: int = 48, frontend: Fbank | None = None) -> None:
        self.encoder = encoder
        self.max_batch = int(max_batch)
        self.max_seq = int(max_seconds * FRAME_RATE)
        if self.max_seq < MIN_SEQ:
            raise ValueError("max_seconds is too short")
        device = encoder.device
        b, s = self.max_batch, self.max_seq
        self.features = torch.zeros(b * s * encoder.features, device=device)
        self.lens = torch.zeros(b, dtype=torch.int32, device=device)
        self.hidden = torch.zeros(b * s * encoder.hidden, device=device)
        self.workspace = encoder.workspace(b * s)
        self.use_graph = use_graph
        self.graphs = BucketGraphs(max_graphs)
        self.compute = torch.cuda.Stream(device=device)
        self.frontend = frontend
        self.max_samples = self.max_seq * BUCKET_QUANTUM
        if frontend is not None:
            self.wave = torch.zeros(b * self.max_samples, device=device)
            self.wave_valid = torch.zeros(b, dtype=torch.int32, device=device)
            self.fbank_workspace = frontend.workspace(b, self.max_samples)

    def bucket(self, frames: int) -> int:
        return bucket_frames(frames, self.max_seq)

    def _views(self, batch: int, length: int):
        enc = self.encoder
        feats = self.features[:batch * length * enc.features].view(batch, length, enc.features)
        hidden = self.hidden[:batch * length * enc.hidden].view(batch, length, enc.hidden)
        return feats, hidden

    def _enqueue(self, batch: int, length: int) -> None:
        feats, hidden = self._views(batch, length)
        self.encoder(feats, self.lens[:batch], out=hidden, workspace=self.workspace)

    def run(self, features: torch.Tensor, frames=None) -> torch.Tensor:
        """features [B, n, F] (any device; fp32) with ``frames`` valid frames
        per item (a sequence of ints, None: all n) -> hidden [B, n, C], a view
        of the runtime's buffer valid until the next call.  Enqueued on the
        compute stream; the current stream waits for it."""
        batch, n, nfeat = features.shape
        if not 1 <= batch <= self.max_batch:
            raise ValueError(f"batch {batch} outside [1, {self.max_batch}]")
        if nfeat != self.encoder.features:
            raise ValueError(f"features must have {self.encoder.features} channels")
        frames = [n] * batch if frames is None else [int(f) for f in frames]
        if len(frames) != batch or min(frames) < MIN_SEQ or max(frames) > n:
            raise ValueError(f"frames {frames} must lie in [{MIN_SEQ}, {n}]")
        if n > self.max_seq:
            raise ValueError(f"{n} frames exceed the runtime's maximum of {self.max_seq}")
        length = self.bucket(n)
        caller = torch.cuda.current_stream(self.encoder.device)
        self.compute.wait_stream(caller)
        with torch.cuda.stream(self.compute):
            feats, hidden = self._views(batch, length)
            feats[:, :n].copy_(features, non_blocking=True)
            if n < length:
                feats[:, n:].zero_()
            self.lens[:batch].copy_(torch.tensor(frames, dtype=torch.int32), non_blocking=False)
            if self.use_graph:
                self.graphs.run((batch, length), lambda: self._enqueue(batch, length))
            else:
                self._enqueue(batch, length)
        caller.wait_stream(self.compute)
        return hidden[:, :n]

    def _enqueue_wave(self, batch: int, samples: int) -> None:
        length = samples // BUCKET_QUANTUM
        feats, hidden = self._views(batch, length)
        wave = self.wave[:batch * samples].view(batch, samples)
        self.frontend(wave, self.wave_valid[:batch], out=feats, workspace=self.fbank_workspace)
        self.encoder(feats, self.lens[:batch], out=hidden, workspace=self.workspace)

    def run_wave(self, wave: torch.Tensor, samples=None) -> torch.Tensor:
        """wave [B, n] 16 kHz fp32 (any device) with ``samples`` true samples
        per item (None: all n) -> hidden [B, num_features(n), C], a view of the
        runtime's buffer valid until the next call; item b's first
        num_features(samples[b]) rows are its valid frames.  Front end and
        encoder run as one graph per (batch, bucket)."""
        if self.frontend is None:
            raise RuntimeError("this runtime was built without a front end")
        batch, n = wave.shape
        if not 1 <= batch <= self.max_batch:
            raise ValueError(f"batch {batch} outside [1, {self.max_batch}]")
        samples = [n] * batch if samples is None else [int(x) for x in samples]
        if len(samples) != batch or max(samples) > n or min(num_features(x) for x in samples) < MIN_SEQ:
            raise ValueError(f"samples {samples} must lie in [1, {n}] and give >= {MIN_SEQ} frames")
        if n > self.max_samples:
            raise ValueError(f"{n} samples exceed the runtime's maximum of {self.max_samples}")
        bucket = bucket_samples(n, self.max_samples)
        caller = torch.cuda.current_stream(self.encoder.device)
        self.compute.wait_stream(caller)
        with torch.cuda.stream(self.compute):
            view = self.wave[:batch * bucket].view(batch, bucket)
            view[:, :n].copy_(wave, non_blocking=True)
            for b, x in enumerate(samples):
                view[b, x:].zero_()
            self.wave_valid[:batch].copy_(torch.tensor(samples, dtype=torch.int32))
            self.lens[:batch].copy_(torch.tensor([num_features(x) for x in samples], dtype=torch.int32))
            if self.use_graph:
                self.graphs.run(("wave", batch, bucket), lambda: self._enqueue_wave(batch, bucket))
            else:
                self._enqueue_wave(batch, bucket)
        caller.wait_stream(self.compute)
        _, hidden = self._views(batch, bucket // BUCKET_QUANTUM)
        return hidden[:, :num_features(n)]
