"""The load-time numeric self-check: this device's kernels against the CPU.

The reference runs a short prompt through the engine when it loads a model,
recomputes every attention layer's output in float64 from the GPU's own
queries and cache, and the head's logits from the last layer's output, and
reloads with its simplest passes when the largest relative error passes
SELF_CHECK_MAX (src/engine.ts:4493-4580 selfCheck, :4582-4627 headError,
src/attention-check.ts:17-100 attentionError, src/handler.ts:455 and
:696-731). This module does the same for the HIP kernels: the prompt goes
through both attention kernels (the prompt form, then the decode form at
one and at several rows), each layer's output is compared with a float64
recomputation from the queries and cache rows the device wrote, and the
head's logits with a float64 product of the final-normed last row and the
embedding rows the device's dequantizer returns. checked_engine() builds an
Engine, runs the check, and on failure runs it again with the library's
simplest kernel forms before it gives up with an error.

The recomputation here is this module's own numpy code: nothing in the
product imports the test oracle."""
from __future__ import annotations

import math

import numpy as np
import torch

from . import engine as E, lib as L

# the largest relative error a loaded model may show (src/handler.ts:455)
SELF_CHECK_MAX = 1e-2
# tokens the check's prompt takes, and how many of its first the head check
# reads (src/engine.ts:866-869)
CHECK_TOKENS = 40
HEAD_CHECK_TOKENS = 8
# the library's simplest kernel forms (the reference's "plain" passes):
# attention without MFMA, XCD grouping or the one-launch split, GEMVs and
# prompt attention on the vector units, GEMMs unsplit
PLAIN_TUNING = {"attn_mfma": 0, "attn_xcd": 0, "attn_fused": 0, "gemv_mfma": 0,
                "attn_prefill_mfma": 0, "gemm_splits": 1}


class SelfCheckError(RuntimeError):
    """The device computes the model wrong even with the simplest kernels."""


def check_token(i: int, vocab: int) -> int:
    """The check's i-th token, spread over the vocabulary (checkToken,
    src/engine.ts:866)."""
    return (i * 7919 + 13) % vocab


def attention_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray, pos0: int, heads: int,
                   kv_heads: int, head_dim: int) -> np.ndarray:
    """Causal attention of query rows q [M, heads * head_dim] (scaled by
    1/sqrt(head_dim) already, as the kernels store them) at positions
    pos0 .. pos0 + M - 1 over cache rows k, v [>= pos0 + M, kv_heads *
    head_dim], in float64: row m sees keys 0 .. pos0 + m."""
    M = q.shape[0]
    G = heads // kv_heads
    q = q.astype(np.float64).reshape(M, heads, head_dim)
    k = k.astype(np.float64).reshape(k.shape[0], kv_heads, head_dim)
    v = v.astype(np.float64).reshape(v.shape[0], kv_heads, head_dim)
    kv_of = np.arange(heads) // G
    out = np.empty((M, heads, head_dim))
    for m in range(M):
        n = pos0 + m + 1
        kh, vh = k[:n][:, kv_of], v[:n][:, kv_of]          # [n, heads, hd]
        s = np.einsum("hd,nhd->hn", q[m], kh)
        s -= s.max(axis=1, keepdims=True)
        e = np.exp(s)
        out[m] = np.einsum("hn,nhd->hd", e, vh) / e.sum(axis=1, keepdims=True)
    return out.reshape(M, heads * head_dim)


def relative_error(got: np.ndarray, want: np.ndarray) -> float:
    """sqrt(sum (got - want)^2 / sum want^2) of one row (infinite when got
    has a value that is not finite)."""
    got = got.astype(np.float64)
    if not np.isfinite(got).all():
        return math.inf
    return math.sqrt(float(((got - want) ** 2).sum()) / max(float((want ** 2).sum()), 1e-30))


def _read(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def attention_error(engine: "E.Engine", tokens) -> float:
    """The largest relative error of any attention row over `tokens` from
    an empty cache: all but the last three as a prompt, then one token,
    then two (the decode kernel at one and at several rows). Leaves the
    engine reset."""
    s = engine.shape
    worst = 0.0

    def probe(layer, name, rows):
        nonlocal worst
        if name != "attention":
            return
        q, out = rows
        M = q.shape[0]
        pos0 = engine.position
        n = pos0 + M
        want = attention_rows(_read(q), _read(engine.k_cache[layer][:n]),
                              _read(engine.v_cache[layer][:n]), pos0, s.heads, s.kv_heads,
                              s.head_dim)
        got = _read(out)
        for m in range(M):
            worst = max(worst, relative_error(got[m], want[m]))

    tokens = list(tokens)
    engine.reset()
    engine.probe = probe
    try:
        engine.forward(tokens[:-3])
        engine.forward(tokens[-3:-2])
        engine.forward(tokens[-2:])
    finally:
        engine.probe = None
        engine.reset()
    return worst


def head_error(engine: "E.Engine", ids) -> float:
    """The embedding rows the device looked up for `ids` against the rows
    its dequantizer returns, and the head's logits of the last row against
    a float64 product of that row's final-normed output with those rows
    (headError, src/engine.ts:4582-4627). The largest relative error.
    Leaves the engine reset."""
    s, w = engine.shape, engine.w
    seen = {}

    def probe(layer, name, rows):
        if name in ("embedding", "output"):
            seen[name] = _read(rows)

    ids = list(ids)
    engine.reset()
    engine.probe = probe
    try:
        engine.forward(ids)
        logits = _read(engine.logits[len(ids) - 1])
    finally:
        engine.probe = None
        engine.reset()
    table = np.stack([_read(w.embedding.dequant(i, 1))[0] for i in ids]).astype(np.float64)
    worst = 0.0
    for r in range(len(ids)):
        diff = float(np.abs(seen["embedding"][r] - table[r]).max())
        scale = float(np.abs(table[r]).max())
        worst = max(worst, diff / scale if scale > 0 else diff)
    x = seen["output"][-1].astype(np.float64)
    r = 1.0 / math.sqrt(float((x * x).mean()) + s.eps)
    want = table @ (x * r * _read(w.final_norm).astype(np.float64))
    got = logits[ids].astype(np.float64)
    if not np.isfinite(got).all():
        return math.inf
    scale = float(np.abs(want).max())
    diff = float(np.abs(got - want).max())
    return max(worst, diff / scale if scale > 0 else diff)


def self_check(engine: "E.Engine") -> float:
    """The largest relative error of the attention and head checks (about
    1e-4 where the kernels compute right)."""
    n = min(CHECK_TOKENS, engine.ctx - 1)
    tokens = [check_token(i, engine.shape.vocab) for i in range(n)]
    worst = 0.0
    if any(engine.shape.layer_type(i) == "attn" for i in range(engine.shape.layers)):
        worst = attention_error(engine, tokens)
    return max(worst, head_error(engine, tokens[:min(HEAD_CHECK_TOKENS, n)]))


def checked_engine(weights: "E.Weights", ctx: int) -> tuple["E.Engine", float]:
    """An Engine over `weights` whose self-check passed, and its error. A
    failed check retries with the simplest kernel forms, which then stay set
    for the process (the engine's kernels read the knobs at every launch);
    a second failure raises SelfCheckError."""
    engine = E.Engine(weights, ctx)
    error = self_check(engine)
    if error <= SELF_CHECK_MAX:
        return engine, error
    for k, v in PLAIN_TUNING.items():
        L.tuning_set(k, v)
    error = self_check(engine)
    if error <= SELF_CHECK_MAX:
        return engine, error
    raise SelfCheckError(
        f"this device computes the model wrong: at load its kernels differ from the CPU's "
        f"float64 results by a relative {error:.1e} (the limit is {SELF_CHECK_MAX:g}), "
        f"also with the simplest kernel forms")
