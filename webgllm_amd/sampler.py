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
from collections import Counter, deque
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
    """The tokens the repetition and presence penalties apply to: the last
    `size` tokens read or written (llama.cpp's repeat_last_n), each counted
    however often it appears (src/penalty-window.ts:26-141 states the
    contract). 0 penalizes none, a negative size every token seen. A token's
    state is 1 while it is in the window from the prompt only, 3 once a
    written copy is in it, 0 out of it.

    The window is a bounded deque of (token, written) entries with two
    counters: copies in the window and written copies in it."""

    def __init__(self, size: int = DEFAULT_REPEAT_LAST_N):
        self.size = size
        self._entries: deque = deque(maxlen=size if size > 0 else None)
        self._seen: Counter = Counter()
        self._written: Counter = Counter()

    @staticmethod
    def _state_of(seen: int, written: int) -> int:
        return 0 if seen <= 0 else (3 if written > 0 else 1)

    def state(self, token: int) -> int:
        return self._state_of(self._seen[token], self._written[token])

    def _leaving(self, incoming: list) -> list:
        """The entries that leave when `incoming` entries join, oldest first
        (some of `incoming` itself when it is longer than the window)."""
        if self.size < 0:
            return []
        over = len(self._entries) + len(incoming) - self.size
        if over <= 0:
            return []
        old = len(self._entries)
        return [self._entries[k] if k < old else incoming[k - old] for k in range(over)]

    def push(self, tokens, generated: bool = False) -> list:
        """Takes tokens in order (the prompt's, then each one written);
        returns [(token, state)] of the tokens whose state changed: the
        tokens taken first, then those that left, each once."""
        if self.size == 0:
            return []
        incoming = [(int(t), bool(generated)) for t in tokens]
        leaving = self._leaving(incoming)
        touched = list(dict.fromkeys([t for t, _ in incoming] + [t for t, _ in leaving]))
        before = [self.state(t) for t in touched]
        for t, g in incoming:
            self._seen[t] += 1
            self._written[t] += g
        for t, g in leaving:
            self._seen[t] -= 1
            self._written[t] -= g
            if self._seen[t] == 0:
                del self._seen[t]
                self._written.pop(t, None)
        self._entries.extend(incoming)
        return [(t, self.state(t)) for t, b in zip(touched, before) if self.state(t) != b]

    def ahead(self, drafts) -> list:
        """The window's states at each row of a batch whose inputs after the
        first are `drafts` (row r has read drafts 0..r-1 as written), as
        SeenRows [token, state, first row, end row): the runs of rows where
        a token's state differs from its state now, ordered by first row,
        a row's draft before the token it pushed out. Nothing changes.

        The drafts are replayed on copies of the touched tokens' counts
        (the drafts and the entries they push out, known up front), giving
        a token x row table of states; each token's row is then cut into
        runs."""
        drafts = [int(d) for d in drafts]
        if self.size == 0 or not drafts:
            return []
        rows = len(drafts) + 1
        incoming = [(d, True) for d in drafts]
        leaving = self._leaving(incoming)
        # the entry that leaves at row r (1-based), if any
        first_out = len(drafts) - len(leaving) + 1
        out_at = {first_out + k: e for k, e in enumerate(leaving)}
        touched = list(dict.fromkeys(drafts + [t for t, _ in leaving]))
        seen = {t: self._seen[t] for t in touched}
        written = {t: self._written[t] for t in touched}
        base = {t: self._state_of(seen[t], written[t]) for t in touched}
        table = {t: [base[t]] for t in touched}  # state at rows 0 .. rows - 1
        rank = {}  # (token, row) -> 0 for the row's draft, 1 for what it pushed out
        for r in range(1, rows):
            d = drafts[r - 1]
            seen[d] += 1
            written[d] += 1
            rank.setdefault((d, r), 0)
            if r in out_at:
                t, g = out_at[r]
                seen[t] -= 1
                written[t] -= g
                rank.setdefault((t, r), 1)
            for t in touched:
                table[t].append(self._state_of(seen[t], written[t]))
        segments = []
        for t in touched:
            states = table[t]
            r = 1
            while r < rows:
                if states[r] == base[t]:
                    r += 1
                    continue
                end = r + 1
                while end < rows and states[end] == states[r]:
                    end += 1
                segments.append((r, rank.get((t, r), 0), [t, states[r], r, end]))
                r = end
        segments.sort(key=lambda s: (s[0], s[1]))
        return [seg for _, _, seg in segments]

    def entries(self) -> list:
        """The tokens in the window, each once, with its state."""
        return [(t, self.state(t)) for t in self._seen]

    def counted(self) -> list:
        """Each token in the window and its copies there (the frequency
        penalty's count)."""
        return list(self._seen.items())


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

    STAGE = 64  # mask changes a see() stages without blocking

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
        self.tok_host = torch.empty(self.STAGE, dtype=torch.int64, pin_memory=True)
        self.val_host = torch.empty(self.STAGE, dtype=torch.uint8, pin_memory=True)
        self.tok_dev = torch.empty(self.STAGE, dtype=torch.int64, device=device)
        self.val_dev = torch.empty(self.STAGE, dtype=torch.uint8, device=device)

    def see(self, changes) -> None:
        """The window's state changes [(token, state)] into the device mask.
        Up to STAGE changes (a decode step's) go through pinned buffers kept
        for it and copies that do not wait for the device, so a step's
        update does not stall the host behind work already queued; the
        buffers are written again only after finish() has waited for an
        event recorded behind the last copies. More (a prompt's) are
        written with blocking copies."""
        import torch
        if not changes:
            return
        n = len(changes)
        if n > self.STAGE:
            t = torch.tensor([c[0] for c in changes], dtype=torch.int64)
            v = torch.tensor([c[1] for c in changes], dtype=torch.uint8)
            self.mask[t.to(self.mask.device)] = v.to(self.mask.device)
            return
        th, vh = self.tok_host.numpy(), self.val_host.numpy()
        for j, (tok, state) in enumerate(changes):
            th[j], vh[j] = tok, state
        self.tok_dev[:n].copy_(self.tok_host[:n], non_blocking=True)
        self.val_dev[:n].copy_(self.val_host[:n], non_blocking=True)
        self.mask.index_put_((self.tok_dev[:n],), self.val_dev[:n])

    def __call__(self, logits_row, sampler: "Sampler") -> Distribution:
        self.start(logits_row, sampler)
        return self.finish(sampler)

    def start(self, logits_row, sampler: "Sampler", also=()) -> None:
        """Enqueues the pick and its read-back (and the copies in `also`,
        (pinned host, device) pairs) and records an event after them: work
        enqueued later runs on while finish() waits for this alone."""
        import torch
        lib = L.load()
        chunks = self.dev[:self.count].view(torch.int32)
        L.check(lib.wg_pick_candidates(
            logits_row.data_ptr(), 1, self.V, self.V, self.mask.data_ptr(), None, 0, 0,
            float(sampler.repetition_penalty), float(sampler.presence_penalty), None, 0, 0,
            self.count, chunks.data_ptr(), self.dev[self.count:].data_ptr(),
            self.scratch.data_ptr(), self.scratch.numel(), self._ops._stream()))
        self.host.copy_(self.dev, non_blocking=True)
        for host, dev in also:
            host.copy_(dev, non_blocking=True)
        self.done = torch.cuda.Event()
        self.done.record()

    def finish(self, sampler: "Sampler") -> Distribution:
        """The distribution over the candidates start() read back."""
        self.done.synchronize()
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
    """Speculative sampling's accept-or-resample step for a drafted token
    (src/sampler.ts:209-223 states it): the draft survives with the
    probability d gives it, else the token comes from the residual, d with
    the draft's mass taken out and the rest renormalized (float32 stores of
    p / (1 - p_draft)). Returns (kept, token). One uniform decides the keep
    (only when 0 < p_draft < 1) and the draw takes the next, the order that
    makes a seeded reply reproduce the reference's tokens."""
    rnd = _random(random)
    where = np.flatnonzero(d.ids == drafted)
    j = int(where[-1]) if where.size else None
    p_draft = 0.0 if j is None else float(d.p[j])
    keep = p_draft >= 1.0 or (p_draft > 0.0 and rnd() < p_draft)
    if keep:
        return True, drafted
    if j is None:
        return False, draw(d, rnd)
    residual = (d.p.astype(np.float64) / (1.0 - p_draft)).astype(np.float32)
    residual[j] = 0.0
    return False, draw(Distribution(d.ids, residual), rnd)


def verify_at(d: Distribution, drafted: int, u: float):
    """verifyAt (src/sampler.ts:250-257)."""
    token = draw_at(d, u)
    return (True, drafted) if token == drafted else (False, token)

