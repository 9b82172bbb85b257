"""Seeded synthetic batches shaped like the benchmark configurations.

All arrays are produced on the CPU in fp32 with numpy (the first config also
uses torch's CPU generator), so they are bit-identical on every machine.

  C1 plumbing: B=2, T=500/320, V=32, targets [3,7,7,12] and [4,9,2], blank 0.
  C2 wav2vec2-char: B=64, T~U{250..1750}, V=32, L=round(T/3.3), peaky emissions.
  C3 long-form: B=4, T=30000, L=9000, V=32, peaky with 15% of frames flattened.
  C4 subword: B=128, T~U{125..500}, V=1024, L=round(T/6), Zipf(1.1) tokens.
  C5 short/edge: B=1024, T~U{50..400}, V=32, L=round(T/3); 10% tight rows,
     2% infeasible rows, 5% flat near-tie rows.

Peaky emissions: sample a random monotone CTC alignment of the target (blanks
mandatory between repeats, optional elsewhere with probability 1/2), split the
T frames over its states by a random composition with every part >= 1, draw
N(0,1) logits, add +8 on each frame's aligned label, and apply log_softmax.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEEDS = {"c1": 1, "c2": 2, "c3": 3, "c4": 4, "c5": 5}


@dataclass
class Batch:
    name: str
    emissions: list[np.ndarray]
    targets: list[np.ndarray]
    blank: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def frames(self) -> int:
        return int(sum(e.shape[0] for e in self.emissions))

    @property
    def cells(self) -> int:
        return int(sum(e.shape[0] * (2 * t.size + 1) for e, t in zip(self.emissions, self.targets)))

    def min_bytes(self) -> int:
        """Algorithmic HBM bytes: each needed emission value read once, int64
        label + fp32 score written per frame, targets read once:
        sum_r 4*T_r*D_r + 12*T_r + 8*L_r, D_r = distinct labels incl. blank."""
        total = 0
        for e, t in zip(self.emissions, self.targets):
            d = len(set(t.tolist()) | {self.blank})
            total += 4 * e.shape[0] * d + 12 * e.shape[0] + 8 * t.size
        return total


def _log_softmax(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32, copy=False)
    m = x.max(axis=1, keepdims=True)
    z = x - m
    return (z - np.log(np.exp(z).sum(axis=1, keepdims=True, dtype=np.float32))).astype(np.float32)


def ctc_frame_labels(rng: np.random.Generator, targets: np.ndarray, frames: int, blank: int) -> np.ndarray:
    """A random monotone CTC alignment of `targets` over `frames` frames."""
    states: list[int] = []
    previous = None
    for token in targets.tolist():
        if token == previous or rng.random() < 0.5:
            states.append(blank)
        states.append(token)
        previous = token
    if rng.random() < 0.5:
        states.append(blank)
    # drop optional blanks while the alignment does not fit
    while len(states) > frames:
        for i in range(len(states)):
            if states[i] == blank and not (0 < i < len(states) - 1 and states[i - 1] == states[i + 1]):
                del states[i]
                break
        else:
            raise ValueError("targets need more frames than available")
    m = len(states)
    cuts = np.sort(rng.choice(np.arange(1, frames), size=m - 1, replace=False)) if m > 1 else np.array([], int)
    lengths = np.diff(np.concatenate([[0], cuts, [frames]]))
    return np.repeat(np.asarray(states, dtype=np.int64), lengths)


def peaky(rng: np.random.Generator, targets: np.ndarray, frames: int, vocab: int, blank: int = 0,
          boost: float = 8.0, raw: bool = False) -> np.ndarray:
    labels = ctc_frame_labels(rng, targets, frames, blank)
    logits = rng.standard_normal((frames, vocab), dtype=np.float32)
    logits[np.arange(frames), labels] += np.float32(boost)
    return logits if raw else _log_softmax(logits)


# Every generator takes raw=True to return the logits before the log-softmax
# (the input of the fused logits path); the random draws are the same.
def _finish(x: np.ndarray, raw: bool) -> np.ndarray:
    return x.astype(np.float32, copy=False) if raw else _log_softmax(x)


def c1(raw: bool = False) -> Batch:
    import torch

    generator = torch.Generator().manual_seed(SEEDS["c1"])
    logits = [torch.randn(t, 32, generator=generator) for t in (500, 320)]
    emissions = [x.numpy() if raw else x.log_softmax(-1).numpy() for x in logits]
    targets = [np.array([3, 7, 7, 12], dtype=np.int64), np.array([4, 9, 2], dtype=np.int64)]
    return Batch("c1", emissions, targets)


def c2(batch: int = 64, raw: bool = False) -> Batch:
    rng = np.random.default_rng(SEEDS["c2"])
    emissions, targets = [], []
    for _ in range(batch):
        T = int(rng.integers(250, 1751))
        L = int(round(T / 3.3))
        y = rng.integers(1, 32, size=L).astype(np.int64)
        emissions.append(peaky(rng, y, T, 32, raw=raw))
        targets.append(y)
    return Batch("c2", emissions, targets)


def c3(batch: int = 4, frames: int = 30000, tokens: int = 9000, raw: bool = False) -> Batch:
    rng = np.random.default_rng(SEEDS["c3"])
    emissions, targets = [], []
    for _ in range(batch):
        y = rng.integers(1, 32, size=tokens).astype(np.int64)
        labels = ctc_frame_labels(rng, y, frames, 0)
        logits = rng.standard_normal((frames, 32), dtype=np.float32)
        boost = np.full(frames, 8.0, dtype=np.float32)
        flat = int(0.15 * frames)
        spans = 0
        while spans < flat:  # contiguous noisy spans of 50..400 frames
            width = int(min(rng.integers(50, 401), flat - spans))
            start = int(rng.integers(0, frames - width))
            boost[start:start + width] = 0.0
            spans += width
        logits[np.arange(frames), labels] += boost
        emissions.append(_finish(logits, raw))
        targets.append(y)
    return Batch("c3", emissions, targets)


def c4(batch: int = 128, raw: bool = False) -> Batch:
    rng = np.random.default_rng(SEEDS["c4"])
    ids = np.arange(1, 1024)
    p = ids.astype(np.float64) ** -1.1
    p /= p.sum()
    emissions, targets = [], []
    for _ in range(batch):
        T = int(rng.integers(125, 501))
        L = int(round(T / 6))
        y = rng.choice(ids, size=L, p=p).astype(np.int64)
        emissions.append(peaky(rng, y, T, 1024, raw=raw))
        targets.append(y)
    return Batch("c4", emissions, targets)


def c5(batch: int = 1024, raw: bool = False) -> Batch:
    rng = np.random.default_rng(SEEDS["c5"])
    emissions, targets = [], []
    kinds = []
    for i in range(batch):
        T = int(rng.integers(50, 401))
        L = int(round(T / 3))
        y = rng.integers(1, 32, size=L).astype(np.int64)
        R = int((y[1:] == y[:-1]).sum())
        u = rng.random()
        if u < 0.10:
            kind, T = "tight", L + R
        elif u < 0.12:
            kind, T = "infeasible", L + R - 1
        elif u < 0.17:
            kind = "flat"
        else:
            kind = "peaky"
        if kind == "flat":
            e = _finish(rng.normal(0.0, 0.01, size=(T, 32)).astype(np.float32), raw)
        elif kind == "infeasible":
            e = _finish(rng.standard_normal((T, 32), dtype=np.float32), raw)
        else:
            e = peaky(rng, y, T, 32, raw=raw)
        emissions.append(e)
        targets.append(y)
        kinds.append(kind)
    return Batch("c5", emissions, targets, notes={"kinds": kinds})


CONFIGS = {"c1": c1, "c2": c2, "c3": c3, "c4": c4, "c5": c5}


def make(name: str, **kwargs) -> Batch:
    return CONFIGS[name](**kwargs)
