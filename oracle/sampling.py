"""CPU restatement of Kandle's token sampling — TEST INFRASTRUCTURE ONLY.

Only tests/ (as the checker) may import this module; the product (kandle_amd) never does.

sample_reference() follows packages/model-utils/src/sampling/index.ts line by line, in the
arithmetic the JavaScript performs: Float32Array stores round to float32, everything else is an f64
JavaScript number, sums run sequentially in index (or sorted) order.  The random number r is an
argument (the reference calls Math.random(); the device path draws philox4x32-10(seed, counter)).

philox4x32_10() restates the counter-based generator of Salmon, Moraes, Dror and Shaw (SC'11,
"Parallel random numbers: as easy as 1, 2, 3"), pinned in tests/test_oracle.py by the published
Random123 known-answer vectors.

Pinning of sample_reference (tests/test_oracle.py): hand-worked draws that distinguish id order from
sorted order, top-k = 1 and a vanishing top-p giving the argmax, the unfiltered probabilities equal
to a closed-form softmax, a grid of r reproducing the exact inverse-CDF counts, and stable tie order.
"""
from __future__ import annotations

import numpy as np

_M0, _M1, _W0, _W1 = 0xD2511F53, 0xCD9E8D57, 0x9E3779B9, 0xBB67AE85
_MASK = 0xFFFFFFFF


def philox4x32_10(counter, key):
    """Four 32-bit outputs of Philox4x32 with 10 rounds for a 4-word counter and a 2-word key."""
    c0, c1, c2, c3 = (int(x) & _MASK for x in counter)
    k0, k1 = (int(x) & _MASK for x in key)
    for r in range(10):
        if r:
            k0, k1 = (k0 + _W0) & _MASK, (k1 + _W1) & _MASK
        p0, p1 = _M0 * c0, _M1 * c2
        c0, c1, c2, c3 = ((p1 >> 32) ^ c1 ^ k0) & _MASK, p1 & _MASK, ((p0 >> 32) ^ c3 ^ k1) & _MASK, p0 & _MASK
    return c0, c1, c2, c3


def uniform24(seed: int, counter: int) -> float:
    """r in [0, 1): word 0 of philox4x32-10(counter = (counter, 0, 0, 0), key = seed's 32-bit halves),
    top 24 bits, times 2^-24."""
    w = philox4x32_10((counter & _MASK, 0, 0, 0), (seed & _MASK, (seed >> 32) & _MASK))[0]
    return (w >> 8) * (1.0 / 16777216.0)


def _seq_sum(a64: np.ndarray) -> float:
    """Left-to-right f64 sum (a JavaScript loop or reduce)."""
    return float(np.cumsum(a64)[-1]) if a64.size else 0.0


def _sorted_order(data: np.ndarray) -> np.ndarray:
    """Ids by logit, descending, stable: Array.sort with the comparator b - a (:132).  -0.0 and
    +0.0 compare equal there, and do here, because the key is the f64 negation."""
    return np.argsort(-data.astype(np.float64), kind="stable")


def _softmax_cpu(x: np.ndarray, temperature: float) -> np.ndarray:
    """softmaxCPU (:268-291): f32 max, f32(exp((f64 x - f64 max) * (1 / T))), f64 running sum of
    the stored f32 values, f32 quotient."""
    mx = np.float64(x.max())
    e = np.exp((x.astype(np.float64) - mx) * (1.0 / temperature)).astype(np.float32)
    z = _seq_sum(e.astype(np.float64))
    return (e.astype(np.float64) / z).astype(np.float32)


def filtered_probs(logits, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0):
    """(order, q): the sorted order and the renormalised probabilities in id order that the draw
    walks (sampling/index.ts:166-223)."""
    data = np.asarray(logits, dtype=np.float32).reshape(-1)
    V = data.size
    order = _sorted_order(data)
    if temperature != 1.0:                                                # :169-176
        scaled = (data.astype(np.float64) * (1.0 / temperature)).astype(np.float32)
    else:
        scaled = data
    probs = _softmax_cpu(scaled, 1.0)                                     # :179
    k_eff = V
    if 0 < top_k < V:                                                     # :183-194
        k_eff = top_k
        mask = np.zeros(V, np.float32)
        mask[order[:top_k]] = 1.0
        probs = (probs * mask).astype(np.float32)
    if top_p < 1.0:                                                       # :197-215
        cum = np.cumsum(probs[order[:k_eff]].astype(np.float64))          # the loop's running sum
        hit = np.nonzero(cum >= top_p)[0]
        cutoff = int(hit[0]) + 1 if hit.size else k_eff
        probs[order[cutoff:]] = 0.0
    psum = _seq_sum(probs.astype(np.float64))                             # :218-223
    if psum > 0:
        probs = (probs.astype(np.float64) / psum).astype(np.float32)
    return order, probs


def draw_from_probs(q: np.ndarray, r: float) -> int:
    """sampleFromProbs (:294-311): the first id whose f64 running sum of q exceeds r, else the last
    id with q > 0, else 0."""
    cum = np.cumsum(q.astype(np.float64))
    hit = np.nonzero(r < cum)[0]
    if hit.size:
        return int(hit[0])
    nz = np.nonzero(q > 0)[0]
    return int(nz[-1]) if nz.size else 0


def sample_reference(logits, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0, r: float = 0.5,
                     display_k: int = 10, do_sample: bool = True):
    """(token, log_prob, display_ids, display_probs) of sample() (sampling/index.ts:103-243)."""
    data = np.asarray(logits, dtype=np.float32).reshape(-1)
    if not do_sample:                                                     # :138-160
        order = _sorted_order(data)
        q = _softmax_cpu(data, temperature)
        token = int(order[0])
    else:
        order, q = filtered_probs(data, temperature, top_k, top_p)
        token = draw_from_probs(q, r)
    k = min(display_k, data.size)
    return token, float(np.log(np.float64(q[token]) + 1e-10)), order[:k].astype(np.int64), q[order[:k]]


def draw_margin(logits, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0, r: float = 0.5) -> float:
    """Distance from r to the nearest running sum of the draw.  Summation orders that differ by
    float rounding (about 1e-16 per step) may pick different ids only when this is that small."""
    _, q = filtered_probs(logits, temperature, top_k, top_p)
    return float(np.min(np.abs(np.cumsum(q.astype(np.float64)) - r)))


def topp_margin(logits, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0) -> float:
    """Distance from top_p to the nearest sorted running sum inside the top-k prefix (inf when
    top-p is off): the cutoff is summation-order independent when this exceeds rounding."""
    if top_p >= 1.0:
        return float("inf")
    data = np.asarray(logits, dtype=np.float32).reshape(-1)
    order = _sorted_order(data)
    scaled = (data.astype(np.float64) * (1.0 / temperature)).astype(np.float32) if temperature != 1.0 else data
    p = _softmax_cpu(scaled, 1.0)
    k_eff = top_k if 0 < top_k < data.size else data.size
    return float(np.min(np.abs(np.cumsum(p[order[:k_eff]].astype(np.float64)) - top_p)))
