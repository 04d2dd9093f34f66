"""The sampled decode's pick after the LM head, on the GPU (otpu_sample): the reference's device
sampler bit for bit (`opentpu/llm/generate.py:217-247` Sampling, `:323-337` Sampler, `:492-557`
reference_pick at one slice): the repetition penalty, an optional soft cap, the k blocks of 64
logits with the largest maxima, the k largest logits among them, the exp2 softmax at the
temperature, top-p, and the inverse-CDF pick for a uniform u."""
from __future__ import annotations

import math

import numpy as np

from . import _lib as X

K_MAX = 64
TOPP_MIN = 2.0 ** -126


class Sampling:
    """The sampled loop's parameters, as the reference's `generate.Sampling` takes them:
    temperature (<= 0: greedy), top_k (1 .. 64), top_p, repetition_penalty (>= 1)."""

    def __init__(self, temperature: float, top_k: int, top_p: float = 1.0,
                 repetition_penalty: float = 1.0):
        # a non-positive temperature, or a top_p that flushes to zero, picks the largest logit:
        # one candidate, unit scale, no top-p cut
        self.greedy = temperature <= 0 or top_p < TOPP_MIN
        if repetition_penalty < 1.0:
            raise ValueError(f"Sampling: repetition_penalty {repetition_penalty} is below 1")
        if self.greedy:
            self.k, self.itemp, self.top_p = 1, 1.0, 1.0
        else:
            if not 1 <= top_k <= K_MAX:
                raise ValueError(f"Sampling: top_k {top_k} outside 1 .. {K_MAX}")
            self.k = int(top_k)
            self.itemp = math.log2(math.e) / temperature       # exp2 of logit * itemp = exp(logit / T)
            self.top_p = float(top_p)
        self.penalty = float(repetition_penalty)
        self.pen = self.penalty != 1.0
        self.kmax = 8 * -(-self.k // 8)                        # candidate buffers in whole 8s


def penalty_factors(V: int, context, R: float):
    """The penalty's factor rows pa, pb [V] (device fp32): 1 / R and R at the context's ids, 1
    elsewhere (the reference keeps them in DRAM and updates them per token)."""
    a, b = np.ones(V, np.float32), np.ones(V, np.float32)
    ix = np.unique(np.asarray(list(context), np.int64))
    if ix.size:
        a[ix], b[ix] = np.float32(1.0) / np.float32(R), np.float32(R)
    return X.dev(a, np.float32), X.dev(b, np.float32)


class Sampler:
    """A reusable sampler for vocabulary V: its work area, the penalty's factor rows and the
    output ids stay on the device; `pick` launches the two kernels on the current stream."""

    def __init__(self, V: int, samp: Sampling, context=(), softcap: float | None = None):
        self.V, self.samp, self.softcap = V, samp, float(softcap or 0.0)
        self.work = X.empty((int(X.load().otpu_sample_work_bytes(V)),), np.uint8)
        self.status = X.zeros((1,), np.int32)
        self.pa = self.pb = None
        if samp.pen:
            self.pa, self.pb = penalty_factors(V, context, samp.penalty)

    def after(self, tok: int) -> None:
        """tok joins the penalty's context: pa[tok] = 1 / R, pb[tok] = R."""
        if self.pa is not None:
            self.pa[tok] = float(np.float32(1.0) / np.float32(self.samp.penalty))
            self.pb[tok] = float(np.float32(self.samp.penalty))

    def pick_device(self, logits, u):
        """ids [len(u)] (int32, device) for the device logits [V] and uniforms u (device fp32)."""
        ids = X.empty((u.numel(),), np.int32)
        s = self.samp
        X.call("otpu_sample", X.ptr(logits), self.V, X.ptr(self.pa), X.ptr(self.pb), self.softcap, s.k,
               float(np.float32(s.itemp)), float(np.float32(s.top_p)), X.ptr(u), u.numel(), X.ptr(self.work),
               X.ptr(ids), X.ptr(self.status), X.stream())
        return ids

    def check(self) -> None:
        if int(X.host(self.status)[0]):
            raise ValueError(f"top_p {self.samp.top_p} keeps no token (Sampling: P >= TOPP_MIN)")

    def candidates(self):
        """(values [kmax] fp32, ids [kmax] int32) of the last pick: the k largest logits."""
        km = self.samp.kmax
        w = X.host(self.work[:512]).view(np.float32)             # vs [64], then si [64]
        return w[:km].copy(), w[64:64 + km].view(np.int32).copy()


def pick(logits, samp: Sampling, context=(), u=0.5, softcap: float | None = None):
    """`generate.reference_pick(logits, samp, context, u, 1, softcap)` on the GPU: the id (an
    array of uniforms: an array of ids)."""
    lg = X.dev(logits, np.float32).reshape(-1)
    sm = Sampler(lg.numel(), samp, context, softcap)
    uu = X.dev(np.atleast_1d(np.asarray(u, np.float32)), np.float32)
    ids = sm.pick_device(lg, uu)
    sm.check()
    out = X.host(ids).astype(np.int64)
    return out if np.ndim(u) else int(out[0])


def lm_head_sample(x, w, sampler: Sampler, u):
    """The sampled token(s) of x [1, K] @ w^T (w: the LM head, an `mxu.QWeight`): the LM head's
    GEMV writes the logits, the sampler picks from them, with no host round trip between (one
    stream). u: device uniforms. Returns the ids (int32, device)."""
    from . import fp32 as F32M
    from . import mxu
    q, Sa, da = F32M.quantize_mx(X.dev(x, np.float32).reshape(1, -1), 32)
    _, lg, _ = mxu.lm_head_argmax(q, Sa, da, w.rows, w.srows, w.fmt, w.K, rsc=w.rsc)
    return sampler.pick_device(lg, u)
