"""Token sampling on the device (reference: packages/model-utils/src/sampling/index.ts).

`sample(logits, config, display_top_k)` mirrors the reference's sample(): greedy (do_sample=False)
takes the lowest-index maximum; otherwise temperature, top-k, top-p and a draw.  Both run on the
device (kh_sample) -- the reference reads the 151,936 logits back and sorts them in JavaScript.  The random
number is philox4x32-10(seed, counter) instead of Math.random(), so a draw is reproducible; `counter`
may be a device int32 tensor that a generation loop advances.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Union

import numpy as np

from .. import env
from ..tensor import HipTensorHandle, Tensor


@dataclass
class SamplerConfig:
    """sampling/index.ts SamplerConfig and DEFAULT_SAMPLER_CONFIG."""

    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    do_sample: bool = True


@dataclass
class SampleResult:
    token_id: int
    log_prob: float
    top_k_token_ids: List[int] = field(default_factory=list)
    top_k_probs: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))


def _row(logits: Tensor):
    """(row, views): the first row of [vocab] or [..., vocab] logits as a contiguous [vocab]-element
    tensor (the reference samples batch 0), and the temporaries to dispose afterwards."""
    from .. import functional as F

    if len(logits.shape) == 1:
        return logits, []
    views = []
    x = logits
    if len(x.shape) > 2:
        x = F.reshape(x, [-1, x.shape[-1]])
        views.append(x)
    row = F.narrow(x, 0, 0, 1)
    views.append(row)
    if not row.handle.is_contiguous():
        row = F.contiguous(row)
        views.append(row)
    return row, views


def sample_device(logits: Tensor, config: SamplerConfig, seed: int, counter: Optional[Tensor], token: Tensor,
                  display_top_k: int = 0, logprob: Optional[Tensor] = None, display_ids: Optional[Tensor] = None,
                  display_probs: Optional[Tensor] = None) -> None:
    """Enqueue one choice into device tensors (no host synchronisation): token (int32 [1]) and the
    optional outputs.  `counter` is an int32 [1] device tensor (unused, and may be None, when
    config.do_sample is False)."""
    ops = env.get_backend("hip").operators
    row, views = _row(logits)
    h = lambda t: t.handle if t is not None else None  # noqa: E731
    try:
        ops.find("sample")(row.handle, {
            "do_sample": config.do_sample, "temperature": config.temperature, "top_k": config.top_k,
            "top_p": config.top_p, "seed": seed, "counter": h(counter), "token": token.handle, "logprob": h(logprob),
            "display_k": display_top_k, "display_ids": h(display_ids), "display_probs": h(display_probs)})
    finally:
        for v in views:
            v.dispose()


class SampleOutputs:
    """Device outputs of one draw in a single int32-sized storage, read back with one copy:
    token (int32), log-probability (float32), k display ids (int32), k display probabilities
    (float32)."""

    def __init__(self, k: int):
        self.k = k
        kk = max(k, 1)
        self._buf = Tensor(np.zeros(2 + 2 * kk, np.int32), dtype="int32")
        st = self._buf.handle.storage
        view = lambda off, n, dt: Tensor(handle=HipTensorHandle.create_view(st, (n,), dt, (1,), off))  # noqa: E731
        self.token, self.logprob = view(0, 1, "int32"), view(1, 1, "float32")
        self.ids, self.probs = view(2, kk, "int32"), view(2 + kk, kk, "float32")

    def read(self) -> SampleResult:
        kk = max(self.k, 1)
        raw = self._buf.handle.storage.download(4 * (2 + 2 * kk))
        w = raw.view(np.int32)
        f = raw.view(np.float32)
        return SampleResult(int(w[0]), float(f[1]), [int(i) for i in w[2:2 + self.k]],
                            f[2 + kk:2 + kk + self.k].copy())

    def dispose(self) -> None:
        for t in (self.token, self.logprob, self.ids, self.probs, self._buf):
            t.dispose()


def sample(logits: Tensor, config: Optional[SamplerConfig] = None, display_top_k: int = 10, seed: int = 0,
           counter: Union[int, Tensor] = 0) -> SampleResult:
    """sample() (sampling/index.ts:103-243): the token, its log-probability and the display_top_k
    most likely ids with their probabilities.  Greedy (do_sample=False) takes the lowest id of the
    largest logit and reports the unfiltered softmax of logits / temperature, as the reference does."""
    config = config or SamplerConfig()
    k = min(display_top_k, logits.shape[-1])
    own_ctr = config.do_sample and not isinstance(counter, Tensor)
    ctr = Tensor(np.array([counter], np.int32), dtype="int32") if own_ctr else (
        counter if isinstance(counter, Tensor) else None)
    out = SampleOutputs(k)
    try:
        sample_device(logits, config, seed, ctr, out.token, k, out.logprob, out.ids, out.probs)
        return out.read()
    finally:
        out.dispose()
        if own_ctr:
            ctr.dispose()


def sample_greedy(logits: Tensor, display_top_k: int = 10) -> SampleResult:
    """sampleGreedy (sampling/index.ts:248-253)."""
    return sample(logits, SamplerConfig(do_sample=False), display_top_k)
