"""Non-greedy picks: the reference's sampler (src/sampler.ts) and penalty
window (src/penalty-window.ts) on the host, over the candidates the GPU
picks (wg_pick_candidates: the best 256-token chunks by penalized logit).

The distribution and the draws run in the library's host code
(wg_sample_distribution, wg_sample_draw, wg_sample_draw_at), which keeps
the reference's float32 stores and its heap order, so a given uniform
draw picks the reference's token; the penalty window's bookkeeping and
the speculative verify are here.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import lib as L

DEFAULT_REPEAT_LAST_N = 64  # src/penalty-window.ts:13
MAX_SEEN_ROWS = 16          # src/penalty-window.ts:24


class _Sampling(C.Structure):
    _fields_ = [("temperature", C.c_double), ("top_p", C.c_double), ("min_p", C.c_double),
                ("top_k", C.c_int32)]


def _bind():
    lib = L.load()
    if not getattr(lib, "_sampler_bound", False):
        P, I32 = C.c_void_p, C.c_int32
        lib.wg_sample_distribution.restype = C.c_int
        lib.wg_sample_distribution.argtypes = [C.POINTER(_Sampling), P, P, I32, P, P,
                                               C.POINTER(I32)]
        for name in ("wg_sample_draw", "wg_sample_draw_at"):
            getattr(lib, name).restype = I32
            getattr(lib, name).argtypes = [P, P, I32, C.c_double]
        lib._sampler_bound = True
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


@dataclass
class Distribution:
    ids: np.ndarray  # int32
    p: np.ndarray    # float32


class PenaltyWindow:
    """The last `size` tokens read or written (llama.cpp's repeat_last_n),
    each penalized once (src/penalty-window.ts:26-141): 0 penalizes none, a
    negative size every token. States: 1 in the window from the prompt only,
    3 written in this reply, 0 out of it."""

    def __init__(self, size: int = DEFAULT_REPEAT_LAST_N):
        self.size = size
        self.ring: list[tuple[int, bool]] = []
        self.start = 0
        self.counts: dict[int, list[int]] = {}  # token -> [all, generated]

    def _state(self, token: int) -> int:
        c = self.counts.get(token)
        return 0 if not c else (3 if c[1] > 0 else 1)

    def push(self, tokens, generated: bool = False) -> list:
        """Takes tokens in order; returns [(token, state)] of those whose state changed."""
        if self.size == 0:
            return []
        before: dict[int, int] = {}

        def note(t):
            if t not in before:
                before[t] = self._state(t)
        for t in tokens:
            t = int(t)
            note(t)
            self.ring.append((t, generated))
            c = self.counts.setdefault(t, [0, 0])
            c[0] += 1
            if generated:
                c[1] += 1
            if self.size > 0 and len(self.ring) - self.start > self.size:
                old, gen = self.ring[self.start]
                self.start += 1
                note(old)
                c = self.counts[old]
                c[0] -= 1
                if gen:
                    c[1] -= 1
                if c[0] == 0:
                    del self.counts[old]
        if self.start > 4096:
            del self.ring[:self.start]
            self.start = 0
        return [(t, self._state(t)) for t, was in before.items() if self._state(t) != was]

    def ahead(self, drafts) -> list:
        """The SeenRows [token, state, first row, end row] of a batch whose
        inputs after the first are `drafts` (src/penalty-window.ts:81-130)."""
        if self.size == 0 or len(drafts) == 0:
            return []
        rows = len(drafts) + 1
        changed: dict[int, list[int]] = {}

        def count(t):
            c = changed.get(t)
            if c is None:
                now = self.counts.get(t)
                c = [now[0], now[1]] if now else [0, 0]
                changed[t] = c
            return c
        live = len(self.ring) - self.start
        out = 0
        open_: dict[int, list] = {}
        segments: list = []
        for i, d in enumerate(drafts):
            d = int(d)
            row = i + 1
            touched = [d]
            c = count(d)
            c[0] += 1
            c[1] += 1
            if self.size > 0 and live + i + 1 - out > self.size:
                if out < live:
                    old, gen = self.ring[self.start + out]
                else:
                    old, gen = int(drafts[out - live]), True
                out += 1
                o = count(old)
                o[0] -= 1
                if gen:
                    o[1] -= 1
                touched.append(old)
            for t in touched:
                c = count(t)
                state = 0 if c[0] == 0 else (3 if c[1] > 0 else 1)
                seg = open_.get(t)
                if state == (seg[1] if seg else self._state(t)):
                    continue
                if seg:
                    seg[3] = row
                    del open_[t]
                if state != self._state(t):
                    nxt = [t, state, row, rows]
                    segments.append(nxt)
                    open_[t] = nxt
        return segments

    def entries(self) -> list:
        return [(t, self._state(t)) for t in self.counts]

    def counted(self) -> list:
        return [(t, c[0]) for t, c in self.counts.items()]


class Sampler:
    """createSampler (src/sampler.ts:27-143) for one reply."""

    def __init__(self, temperature: float, top_k: int, repetition_penalty: float = 1.0,
                 top_p: float = 1.0, min_p: float = 0.0, presence_penalty: float = 0.0,
                 frequency_penalty: float = 0.0, repeat_last_n: int = DEFAULT_REPEAT_LAST_N):
        self.settings = _Sampling(float(temperature), float(top_p), float(min_p), int(top_k))
        self.repetition_penalty = repetition_penalty
        self.presence_penalty = presence_penalty
        self.frequency_penalty = frequency_penalty
        self.window = PenaltyWindow(repeat_last_n)

    def see(self, tokens, output: bool = False):
        return self.window.push(tokens, output)

    def distribution(self, logits: np.ndarray, penalize: bool = True,
                     ids: np.ndarray | None = None) -> Distribution:
        """The kept tokens and their probabilities; changes `logits` (float32)
        by the penalties unless penalize is False (for logits the GPU
        penalized). `ids` names each logit's token (the candidates'), else
        its index."""
        if logits.dtype != np.float32 or not logits.flags.c_contiguous:
            raise ValueError("logits must be a contiguous float32 array")
        rp, pp, fp = self.repetition_penalty, self.presence_penalty, self.frequency_penalty
        if penalize and (rp != 1 or pp != 0 or fp != 0):
            for token, count in self.window.counted():
                if token < 0 or token >= logits.size:
                    continue
                x = float(logits[token])
                if rp != 1:
                    logits[token] = x * rp if x < 0 else x / rp
                logits[token] = float(logits[token]) - (count * fp + pp)
        n = logits.size
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int32)
        out_ids = np.empty(n, np.int32)
        out_p = np.empty(n, np.float32)
        got = C.c_int32()
        L.check(_bind().wg_sample_distribution(C.byref(self.settings), _ptr(logits), _ptr(ids),
                                               n, _ptr(out_ids), _ptr(out_p), C.byref(got)))
        return Distribution(out_ids[:got.value].copy(), out_p[:got.value].copy())

    def sample(self, logits: np.ndarray, random=None) -> int:
        return draw(self.distribution(logits), random)

    def candidates(self, chunks: np.ndarray, cand: np.ndarray) -> Distribution:
        """The distribution over one row's pick (wg_pick_candidates): token
        chunk * 256 + t for candidate t of chunk k, already penalized."""
        chunks = np.asarray(chunks, np.int64)
        ids = (chunks[:, None] * 256 + np.arange(256)[None, :]).astype(np.int32).reshape(-1)
        return self.distribution(np.ascontiguousarray(cand, np.float32).reshape(-1).copy(),
                                 penalize=False, ids=ids)


class GpuPick:
    """Engine.pick's device half for one vocabulary (src/engine.ts:8352-8473)
    with its buffers kept: the penalty mask on the device (updated from the
    window's changes in one write), wg_pick_candidates into preallocated
    outputs, and one read-back into pinned host memory."""

    def __init__(self, vocab: int, count: int = 64, device="cuda"):
        import torch
        from . import ops
        self.V = vocab
        self.count = min(count, (vocab + 255) // 256)
        self.mask = torch.zeros(vocab, dtype=torch.uint8, device=device)
        self.scratch = torch.empty(int(_bind().wg_pick_scratch_bytes(1, vocab)),
                                   dtype=torch.uint8, device=device)
        n = self.count * 256
        # chunk ids then candidates, one buffer so that one copy reads both back
        self.dev = torch.empty(self.count + n, dtype=torch.float32, device=device)
        self.host = torch.empty(self.count + n, dtype=torch.float32, pin_memory=True)
        self.offsets = np.arange(256, dtype=np.int64)
        self._ops = ops

    def see(self, changes) -> None:
        """The window's state changes [(token, state)] into the device mask."""
        import torch
        if changes:
            t = torch.tensor([c[0] for c in changes], dtype=torch.int64)
            v = torch.tensor([c[1] for c in changes], dtype=torch.uint8)
            self.mask[t.to(self.mask.device)] = v.to(self.mask.device)

    def __call__(self, logits_row, sampler: "Sampler") -> Distribution:
        import torch
        lib = L.load()
        chunks = self.dev[:self.count].view(torch.int32)
        L.check(lib.wg_pick_candidates(
            logits_row.data_ptr(), 1, self.V, self.V, self.mask.data_ptr(), None, 0, 0,
            float(sampler.repetition_penalty), float(sampler.presence_penalty), None, 0, 0,
            self.count, chunks.data_ptr(), self.dev[self.count:].data_ptr(),
            self.scratch.data_ptr(), self.scratch.numel(), self._ops._stream()))
        self.host.copy_(self.dev, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        h = self.host.numpy()
        ch = h[:self.count].view(np.int32).astype(np.int64)
        ids = (ch[:, None] * 256 + self.offsets[None, :]).astype(np.int32).reshape(-1)
        return sampler.distribution(h[self.count:].copy(), penalize=False, ids=ids)


def _random(random):
    import random as _r
    return random if random is not None else _r.random


def draw(d: Distribution, random=None) -> int:
    """draw (src/sampler.ts:188-200)."""
    return int(_bind().wg_sample_draw(_ptr(d.ids), _ptr(d.p), d.ids.size, _random(random)()))


def draw_at(d: Distribution, u: float) -> int:
    """drawAt (src/sampler.ts:227-242)."""
    return int(_bind().wg_sample_draw_at(_ptr(d.ids), _ptr(d.p), d.ids.size, float(u)))


def verify(d: Distribution, drafted: int, random=None):
    """Speculative sampling's step for a drafted token (src/sampler.ts:
    209-223): (True, drafted) when kept, else (False, a token drawn from d
    without it). The uniform draws are taken in the reference's order."""
    rnd = _random(random)
    hit = np.nonzero(d.ids == drafted)[0]
    j = int(hit[-1]) if hit.size else -1
    pd = 0.0 if j < 0 else float(d.p[j])
    if pd >= 1 or (pd > 0 and rnd() < pd):
        return True, drafted
    if j < 0:
        return False, draw(d, rnd)
    rest = d.p.copy()
    rest[j] = 0
    total = 1 - pd
    rest = (rest.astype(np.float64) / total).astype(np.float32)
    return False, draw(Distribution(d.ids, rest), rnd)


def verify_at(d: Distribution, drafted: int, u: float):
    """verifyAt (src/sampler.ts:250-257)."""
    token = draw_at(d, u)
    return (True, drafted) if token == drafted else (False, token)

