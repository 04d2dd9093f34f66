"""Oracle: the sampled decode's pick after the LM head (numpy, the machine's fp32 arithmetic).
TEST INFRASTRUCTURE ONLY.

Restated from `opentpu/llm/generate.py:217-247` (Sampling), `:323-337` (the device sampler's
steps) and `:492-557` (reference_pick, one slice), with the ISA's exp2 and sums
(`opentpu/fp32.py:110-160`, `:187-202`, `:227-229`; `docs/isa.md`):
  1. l = ftz(logits); with a soft cap c: l = 2c recip(1 + exp2(l (-2 log2(e) / c))) - c;
     with a repetition penalty R: l = fmin(l pa, l pb), pa = 1/R and pb = R at the context's
     ids (1 elsewhere);
  2. the k blocks of 64 logits with the largest maxima (total order; ties: the lower block),
     their logits in that order, then the k largest of those (ties: the earlier position):
     values vs (descending, -inf past k up to kmax = k rounded up to 8) and ids;
  3. p = exp2((vs - vs[0]) itemp); cum[i] = RDOT of the triangular row with p (64 interleaved
     partials, then a folding tree); kept = step(cum[last] P - cum[i - 1]); zk = the largest
     kept cum; t = min(u, 1 - 2^-24) zk; pick = min(kmax - #{cum > t}, #kept - 1); its id.
  step(x) = fmin(fmax(x 2^126, 0), 1); every op rounds (RNE), flushes denormals and makes NaN
  the canonical one.

Pinning (tests/test_oracle_sampler.py): golden vectors written from the reference
(tests/golden/make_golden.py: exp2's bits on a grid, and reference_pick's ids for several
Samplings, contexts and soft caps over thousands of uniforms), since the machine's exp2
polynomial and its sums' order are fixed by no closed form; and by what the mathematics fixes:
exp2 exact at the integers and within its fit's error elsewhere, the picks' shares of u in
[0, 1) equal to a float64 sampler's probabilities (penalty, top-k, softmax, top-p), greedy at
temperature 0 and top-1 the argmax with the lowest id on ties.
"""
from __future__ import annotations

import math

import numpy as np

from . import fp32 as F

F32 = np.float32
BLK = 64                         # the sampler's block of logits
K_MAX = 64                       # the largest top-k
TOPP_MIN = 2.0 ** -126           # below: the first token only
BIG = F32(2.0 ** 126)            # step(): x BIG >= 1 for every normal x > 0
RED_PARTIALS = 64                # RDOT / RSUM: interleaved partial sums, then a folding tree
LOG2E = 1.0 / math.log(2.0)
# 2^f on [0, 1): the machine's degree-7 polynomial (fp32 coefficients, Horner from C7 down)
EXP2_C = [np.uint32(b).view(F32) for b in (0x3F800000, 0x3F317218, 0x3E75FDE9, 0x3D63593E,
                                            0x3C1D8534, 0x3AAFE2F6, 0x3916C07C, 0x37B3C7D6)]


class Sampling:
    """temperature (<= 0: greedy), top_k (1 .. 64), top_p, repetition_penalty (>= 1)."""

    def __init__(self, temperature: float, top_k: int, top_p: float = 1.0,
                 repetition_penalty: float = 1.0):
        greedy = temperature <= 0 or top_p < TOPP_MIN
        if not greedy and not 0 < top_k <= K_MAX:
            raise ValueError(f"top_k 1 .. {K_MAX}")
        if repetition_penalty < 1.0:
            raise ValueError("repetition_penalty >= 1")
        self.k = 1 if greedy else int(top_k)
        self.itemp = 1.0 if greedy else LOG2E / temperature
        self.top_p = 1.0 if greedy else float(top_p)
        self.penalty = float(repetition_penalty)
        self.kmax = -(-self.k // 8) * 8
        self.pen = self.penalty != 1.0


def gt(a, b):
    return F.key(a) > F.key(b)


def fmax(a, b):
    a, b = F.ftz(a), F.ftz(b)
    return np.where(gt(a, b), a, b).astype(F32)


def fmin(a, b):
    a, b = F.ftz(a), F.ftz(b)
    return np.where(gt(b, a), a, b).astype(F32)


def step(x):
    return fmin(fmax(F.mul(x, BIG), F32(0)), F32(1))


def exp2(x):
    """The machine's exp2: x < -126 -> 0, x >= 128 or NaN -> inf; else i = floor(x),
    f = x - i, the polynomial in f by Horner (a rounded mul, then a rounded add, per step),
    and i added to its exponent field."""
    x = F._finish(F.ftz(x))
    lo = gt(F32(-126), x)
    hi = ~gt(F32(128), x)
    xf = np.where(~lo & ~hi, x, F32(0)).astype(F32)
    i = np.floor(xf.astype(np.float64)).astype(np.int64)
    f = F.sub(xf, F.i2f(i))
    p = np.full(f.shape, EXP2_C[7], F32)
    for c in EXP2_C[6::-1]:
        p = F.add(F.mul(p, f), c)
    r = F.from_bits((F.bits(p).astype(np.int64) + (i << 23)).astype(np.uint32))
    r = np.where(lo, F32(0), r)
    return np.where(hi, F32(np.inf), r).astype(F32)


def tree_sum(a):
    """Row sums of a [rows, n], n <= 64: partial c = +0 + a[:, c] (+0 for c >= n), then while
    the partials are more than one, the first half plus the second (a rounded add each)."""
    a = F.ftz(np.atleast_2d(np.asarray(a, F32)))
    R, n = a.shape
    if n > RED_PARTIALS:
        raise ValueError("tree_sum: at most 64 columns")
    x = np.zeros((R, RED_PARTIALS), F32)
    x[:, :n] = F.add(F32(0), a)
    while x.shape[1] > 1:
        h = x.shape[1] // 2
        x = F.add(x[:, :h], x[:, h:])
    return x[:, 0]


def softcap(x, c: float):
    k1, k2, k3 = F32(-2.0 * LOG2E / c), F32(2.0 * c), F32(c)
    t = F.recip(F.add(exp2(F.mul(x, k1)), F32(1.0)))
    return F.sub(F.mul(t, k2), k3)


def penalty_factors(V: int, context, R: float):
    """pa, pb [V]: 1 / R and R at the context's ids, 1 elsewhere."""
    a, b = np.ones(V, F32), np.ones(V, F32)
    ix = np.unique(np.asarray(list(context), np.int64))
    a[ix], b[ix] = F32(1.0) / F32(R), F32(R)
    return a, b


def knock_out(vals, n):
    """n rounds of: the position of the largest (total order; ties: the first), then that
    entry set to -inf. Returns (positions, the values taken, ftz'd). A position can come back
    once every entry left is -inf or below (the knocked-out ones are -inf too)."""
    v = F.ftz(np.asarray(vals, F32)).copy()
    pos, val = np.zeros(n, np.int64), np.zeros(n, F32)
    for i in range(n):
        q = int(np.argmax(F.key(v)))
        pos[i], val[i] = q, v[q]
        v[q] = -np.inf
    return pos, val


def candidates(logits, samp: Sampling, context=(), softcap_c: float | None = None):
    """Steps 1-2: (vs [kmax], ids [kmax] int64)."""
    lg = F.ftz(np.asarray(logits, F32)).copy()
    if softcap_c:
        lg = softcap(lg, softcap_c)
    V = len(lg)
    if samp.pen:
        a, b = penalty_factors(V, context, samp.penalty)
        lg = fmin(F.mul(lg, a), F.mul(lg, b))
    km, k = samp.kmax, samp.k
    nb = -(-V // BLK)
    x = np.full(nb * BLK, -np.inf, F32)
    x[:V] = lg
    xb = x.reshape(nb, BLK)
    bm = xb[np.arange(nb), np.argmax(F.key(xb), axis=1)]
    blocks, _ = knock_out(bm, min(k, nb))
    cand = np.full(km * BLK, -np.inf, F32)
    ids = np.zeros(km * BLK, np.int64)
    for j, q in enumerate(blocks):
        cand[j * BLK:(j + 1) * BLK] = xb[q]
        ids[j * BLK:(j + 1) * BLK] = q * BLK + np.arange(BLK)
    pos, val = knock_out(cand, k)
    vs = np.full(km, -np.inf, F32)
    si = np.zeros(km, np.int64)
    vs[:k] = val
    si[:k] = ids[pos]
    return vs, si


def pick(logits, samp: Sampling, context=(), u=0.5, softcap_c: float | None = None):
    """The id (an array of uniforms: an array of ids) the device's sampler picks."""
    vs, si = candidates(logits, samp, context, softcap_c)
    km = samp.kmax
    p = exp2(F.mul(F.sub(vs, vs[0]), F32(samp.itemp)))
    c = np.arange(km)
    U = (c[None, :] <= c[:, None]).astype(F32)                 # step(i + 1 - j)
    cum = tree_sum(F.mul(U, p[None, :]))
    prev = np.concatenate([[F32(0)], cum[:-1]]).astype(F32)
    kept = step(F.sub(F.mul(cum[-1], F32(samp.top_p)), prev))
    if not kept[0]:
        raise ValueError(f"top_p {samp.top_p} keeps no token")
    zk = F.mul(cum, kept)[np.argmax(F.key(F.mul(cum, kept)))]
    uu = np.minimum(np.atleast_1d(np.asarray(u, F32)), F32(1 - 2.0 ** -24))
    t = F.mul(uu, zk)[:, None]
    le = F.add(F.mul(tree_sum(step(F.sub(cum[None, :], t))), F32(-1)), F32(km))
    nk = F.sub(tree_sum(kept[None, :]), F32(1))
    pk = fmin(le, nk).astype(np.int64)
    ids = si[pk]
    return ids if np.ndim(u) else int(ids[0])
