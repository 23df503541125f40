"""GPU parity of on-device sampling (kh_sample, kh_philox4x32_10) with the CPU restatement of
sample() (packages/model-utils/src/sampling/index.ts:103-311) in oracle/sampling.py.

Bar: display ids and greedy tokens bit-exact; the drawn token exact unless r lies within 1e-12 of a
running sum (the device sums in another order than the reference's loop, so ties at that distance
are rounding, not semantics; no case here comes that close, and the test says so if one does);
probabilities within 2e-6 relative (f64 sums in another order may move an f32 quotient by one ulp);
log-probabilities within 2e-6 absolute."""
import numpy as np
import pytest

from kandle_amd import Tensor
from kandle_amd import kernels
from kandle_amd.model_utils.sampling import SamplerConfig, sample, sample_device, sample_greedy
from oracle.sampling import draw_margin, philox4x32_10, sample_reference, topp_margin, uniform24

pytestmark = pytest.mark.gpu

VOCAB = 151936


def _logits(seed, n=VOCAB, scale=3.0):
    return (np.random.default_rng(seed).normal(size=n) * scale).astype(np.float32)


def _check(x, cfg, seed, counter, display_k=10):
    lg = Tensor(x, dtype="float32")
    res = sample(lg, cfg, display_k, seed=seed, counter=counter)
    lg.dispose()
    r = uniform24(seed, counter)
    tok, lp, ids, probs = sample_reference(x, cfg.temperature, cfg.top_k, cfg.top_p, r, display_k, cfg.do_sample)
    assert res.top_k_token_ids == [int(i) for i in ids]
    np.testing.assert_allclose(res.top_k_probs, probs, rtol=2e-6, atol=1e-30)
    near = cfg.do_sample and (topp_margin(x, cfg.temperature, cfg.top_k, cfg.top_p) <= 1e-12
                              or draw_margin(x, cfg.temperature, cfg.top_k, cfg.top_p, r) <= 1e-12)
    if near:   # r or top_p within rounding of a running sum: either neighbour is a correct draw
        print(f"[sample] seed={seed} counter={counter}: boundary within 1e-12, token not compared")
        return res
    assert res.token_id == tok
    assert res.log_prob == pytest.approx(lp, abs=2e-6)
    return res


KAT = {  # Random123 known answers: (seed as key low | high << 32, counter row) -> output
    0: (0, (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    0xffffffff_ffffffff: (1, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    0x299f31d0_a4093822: (2, (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
}


def test_philox_device_matches_kat_and_oracle(hip):
    ctr = np.array([[0, 0, 0, 0], [0xffffffff] * 4, [0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344]],
                   np.uint32)
    rng = np.random.default_rng(5)
    ctr = np.concatenate([ctr, rng.integers(0, 2 ** 32, size=(997, 4), dtype=np.uint32)])
    for seed in (0, 0xffffffff_ffffffff, 0x299f31d0_a4093822, 123456789):
        c = Tensor(ctr.view(np.int32), dtype="int32")
        o = Tensor(np.zeros_like(ctr).view(np.int32), dtype="int32")
        kernels.philox4x32_10(seed, c.handle, o.handle)
        got = o.numpy().view(np.uint32)
        c.dispose()
        o.dispose()
        if seed in KAT:
            row, answer = KAT[seed]
            assert tuple(int(v) for v in got[row]) == answer
        want = np.array([philox4x32_10(row, (seed & 0xffffffff, seed >> 32)) for row in ctr], np.uint32)
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("cfg", [
    SamplerConfig(),                                          # plain softmax draw
    SamplerConfig(temperature=0.7, top_k=50),
    SamplerConfig(temperature=0.7, top_p=0.9),
    SamplerConfig(temperature=1.3, top_k=40, top_p=0.95),
    SamplerConfig(temperature=0.5, top_p=0.5),
    SamplerConfig(temperature=2.0, top_k=1),
], ids=["plain", "t0.7k50", "t0.7p0.9", "t1.3k40p0.95", "t0.5p0.5", "t2k1"])
def test_sample_matches_reference_full_vocab(hip, cfg):
    x = _logits(11)
    for seed, counter in ((0, 0), (42, 1), (42, 2), (2 ** 40 + 3, 77), (7, 123456)):
        _check(x, cfg, seed, counter)


def test_sample_peaked_and_flat_rows(hip):
    # a peaked row (top-p keeps few ids) and a flat one (the draw walks far into the vocabulary)
    peaked = _logits(12, scale=8.0)
    flat = _logits(13, scale=0.05)
    for seed in range(4):
        _check(peaked, SamplerConfig(top_p=0.8), seed, seed)
        _check(flat, SamplerConfig(temperature=1.5), seed, seed)
        _check(flat, SamplerConfig(top_k=1000, top_p=0.3), seed, seed)


@pytest.mark.parametrize("t", [1.0, 0.6, 1.7])
def test_greedy_matches_reference(hip, t):
    x = _logits(14)
    x[[100, 5000, 90000]] = x.max() + 1.0                      # a three-way tie for the maximum
    res = _check(x, SamplerConfig(temperature=t, do_sample=False), 0, 0)
    assert res.token_id == 100
    g = sample_greedy(Tensor(x, dtype="float32"), 5)
    assert g.token_id == 100 and g.top_k_token_ids[:3] == [100, 5000, 90000]


def test_small_vocab_ties_and_signed_zero(hip):
    x = np.array([1.0, 5.0, 5.0, 0.0, 5.0, -0.0, 0.0, -3.0], np.float32)
    for cfg in (SamplerConfig(top_k=2), SamplerConfig(top_p=0.5), SamplerConfig(temperature=0.3),
                SamplerConfig(do_sample=False)):
        for c in range(6):
            _check(x, cfg, 9, c, display_k=8)
    one = np.array([2.5], np.float32)
    res = _check(one, SamplerConfig(temperature=0.9, top_p=0.2), 1, 1, display_k=1)
    assert res.token_id == 0


@pytest.mark.parametrize("top_p", [-0.5, 0.0])
def test_nonpositive_top_p_keeps_one_token(hip, top_p):
    """top_p <= 0 keeps exactly the most probable token, as the reference loop does (its running
    sum passes top_p at the first id, sampling/index.ts:197-215): on the full-sort path (top-p
    alone) and on the selection path (with top-k), against the oracle."""
    x = _logits(61)
    for cfg in (SamplerConfig(temperature=0.8, top_p=top_p), SamplerConfig(temperature=0.8, top_k=50, top_p=top_p)):
        for seed in (1, 2, 3):
            res = _check(x, cfg, seed, seed)
            assert res.token_id == int(np.argmax(x))
            assert res.log_prob == pytest.approx(0.0, abs=1e-6)


def test_counter_read_on_device_and_2d_logits(hip):
    x = _logits(15, n=4096, scale=2.0)
    lg = Tensor(x.reshape(1, -1), dtype="float32")
    ctr = Tensor(np.array([3], np.int32), dtype="int32")
    tok = Tensor(np.zeros(1, np.int32), dtype="int32")
    sample_device(lg, SamplerConfig(temperature=0.8), 99, ctr, tok)
    want = sample_reference(x, 0.8, 0, 1.0, uniform24(99, 3), 0)[0]
    assert int(tok.numpy()[0]) == want
    for t in (lg, ctr, tok):
        t.dispose()


def test_sample_argument_errors(hip):
    lg = Tensor(_logits(16, n=64), dtype="float32")
    with pytest.raises(Exception, match="temperature"):
        sample(lg, SamplerConfig(temperature=0.0))
    lg.dispose()


# ---- generateStream (for_causal_lm.ts:354-440) on the device sampler -------------------------------

def _small_model(seed=5, max_seq=96):
    from kandle_amd.model_utils import Qwen3Config, Qwen3ForCausalLM, init_qwen3_weights

    cfg = Qwen3Config(vocab_size=4096, num_hidden_layers=2)
    w = init_qwen3_weights(cfg, seed=seed)
    return cfg, w, Qwen3ForCausalLM(cfg, w, max_seq_len=max_seq)


def _drive(gen, overrides=None):
    """Run a generate_stream generator to the end, sending overrides[i] after step i."""
    steps, send = [], None
    overrides = overrides or {}
    while True:
        try:
            st = gen.send(send) if steps else next(gen)
        except StopIteration:
            return steps
        steps.append(st)
        send = overrides.get(len(steps) - 1)


def test_generate_stream_sampled_steps_follow_reference(hip, monkeypatch):
    """Each step is sample() of the logits the oracle gives for the tokens actually fed (sampled or
    overridden), drawn with r = philox(seed, step)."""
    from kandle_amd import synthetic as syn
    from kandle_amd.model_utils import GeneratorConfig
    from kandle_amd.model_utils import sampling as S
    from oracle.qwen3 import Qwen3Oracle

    cfg, w, model = _small_model()
    prompt = syn.randint(6, (40,), 0, cfg.vocab_size)
    seen = []
    real = S.sample_device

    def spy(logits, config, seed, counter, *args, **kw):
        # eager steps only (use_graph=False): the logits and the counter as the draw reads them
        seen.append((logits.numpy().reshape(-1).copy(), seed, int(counter.numpy()[0])))
        return real(logits, config, seed, counter, *args, **kw)

    monkeypatch.setattr(S, "sample_device", spy)
    gc = GeneratorConfig(max_new_tokens=6, temperature=0.8, top_k=50, top_p=0.9, display_top_k=5)
    steps = _drive(model.generate_stream(prompt, gc, seed=7, use_graph=False), overrides={2: 123})
    model.dispose()
    assert len(steps) == 6 and len(seen) == 6
    fed = [s.token_id for s in steps]
    fed[2] = 123
    ref = Qwen3Oracle(cfg, w, max_seq_len=96, exact=True)
    rl = ref.forward(prompt, 0)
    for i, (st, (lg, seed, ctr)) in enumerate(zip(steps, seen)):
        assert (seed, ctr) == (7, i) and st.cache_position == 40 + i and st.generated_count == i + 1
        assert float(np.max(np.abs(lg - rl))) < 2e-2, i
        r = uniform24(7, i)
        tok, lp, ids, probs = sample_reference(lg, 0.8, 50, 0.9, r, 5)
        assert st.top_k_token_ids == [int(x) for x in ids]
        np.testing.assert_allclose(st.top_k_probs, probs, rtol=2e-6)
        if topp_margin(lg, 0.8, 50, 0.9) > 1e-12 and draw_margin(lg, 0.8, 50, 0.9, r) > 1e-12:
            assert st.token_id == tok and st.log_prob == pytest.approx(lp, abs=2e-6)
        if i + 1 < len(steps):
            rl = ref.forward([fed[i]], 40 + i)


def test_generate_stream_greedy_matches_generate_and_stops_at_eos(hip):
    from kandle_amd import synthetic as syn
    from kandle_amd.model_utils import GeneratorConfig

    cfg, w, model = _small_model(seed=8)
    prompt = syn.randint(9, (33,), 0, cfg.vocab_size)
    want = model.generate(prompt, 6)
    for use_graph in (False, True):
        steps = _drive(model.generate_stream(prompt, GeneratorConfig(max_new_tokens=6, do_sample=False),
                                             use_graph=use_graph))
        assert [s.token_id for s in steps] == want
        assert all(s.top_k_token_ids[0] == s.token_id for s in steps)
    eos = want[2]
    first = want.index(eos)
    steps = _drive(model.generate_stream(prompt, GeneratorConfig(max_new_tokens=6, do_sample=False,
                                                                 eos_token_ids=[eos])))
    model.dispose()
    assert len(steps) == first + 1 and steps[-1].is_eos and not any(s.is_eos for s in steps[:-1])


def test_generate_stream_graph_replay_matches_eager(hip):
    from kandle_amd import synthetic as syn
    from kandle_amd.model_utils import GeneratorConfig

    cfg, w, model = _small_model(seed=10)
    prompt = syn.randint(11, (24,), 0, cfg.vocab_size)
    gc = GeneratorConfig(max_new_tokens=8, temperature=1.1, top_p=0.95, display_top_k=4)
    a = _drive(model.generate_stream(prompt, gc, seed=3, use_graph=False))
    b = _drive(model.generate_stream(prompt, gc, seed=3, use_graph=True))
    c = _drive(model.generate_stream(prompt, gc, seed=4, use_graph=True))
    model.dispose()
    assert [s.token_id for s in a] == [s.token_id for s in b]
    for x, y in zip(a, b):
        assert x.top_k_token_ids == y.top_k_token_ids and np.array_equal(x.top_k_probs, y.top_k_probs)
    assert [s.token_id for s in c] != [s.token_id for s in a]   # another seed, another draw
    # top-p without top-k: the draw takes the full sort, which stays outside the captured graph
    gp = GeneratorConfig(max_new_tokens=5, temperature=0.9, top_p=0.8, display_top_k=3)
    cfg2, w2, model2 = _small_model(seed=12)
    d = _drive(model2.generate_stream(prompt, gp, seed=5, use_graph=False))
    e = _drive(model2.generate_stream(prompt, gp, seed=5, use_graph=True))
    model2.dispose()
    assert [s.token_id for s in d] == [s.token_id for s in e]
    assert all(np.array_equal(x.top_k_probs, y.top_k_probs) for x, y in zip(d, e))


# ---- the selection path (sorted prefix by LDS bitonic selection) against the full sort ------------

def _both_paths(x, cfg, seed, counter, display_k):
    outs = []
    for path in (1, 0):
        kernels.sample_set_path(path)
        try:
            lg = Tensor(x, dtype="float32")
            outs.append(sample(lg, cfg, display_k, seed=seed, counter=counter))
            lg.dispose()
        finally:
            kernels.sample_set_path(0)
    return outs


@pytest.mark.parametrize("n", [1, 100, 4095, 4096, 4097, 40000, VOCAB])
def test_selection_path_matches_sort_path_sizes(hip, n):
    x = _logits(20 + n, n=n, scale=2.5)
    dk = min(10, n)
    for cfg in (SamplerConfig(do_sample=False), SamplerConfig(), SamplerConfig(temperature=0.7, top_k=min(50, n)),
                SamplerConfig(temperature=1.2, top_k=min(20, n), top_p=0.8)):
        for c in range(3):
            a, b = _both_paths(x, cfg, 5, c, dk)
            assert a.top_k_token_ids == b.top_k_token_ids
            np.testing.assert_allclose(b.top_k_probs, a.top_k_probs, rtol=2e-6, atol=1e-30)
            _check(x, cfg, 5, c, dk)   # and both against the reference restatement


def test_selection_path_limits_and_ties(hip):
    x = _logits(30, n=50000, scale=1.0)
    # the longest prefix the selection path builds, and one past it (full sort)
    for k, dk in ((1024, 10), (1025, 10), (40, 1024), (40, 1025)):
        _check(x, SamplerConfig(temperature=0.9, top_k=k, top_p=0.97), 3, 1, dk)
    # all logits equal: the order is the ids, the prefix the lowest ids
    flat = np.full(20000, 1.5, np.float32)
    for cfg in (SamplerConfig(do_sample=False), SamplerConfig(top_k=300), SamplerConfig()):
        res = _check(flat, cfg, 2, 7, 16)
        assert res.top_k_token_ids == list(range(16))
    # ties straddling selection chunks: equal maxima at ids in different 4096-id chunks
    y = _logits(31, n=30000, scale=1.0)
    y[[29999, 4096, 4095, 12000]] = 9.0
    res = _check(y, SamplerConfig(top_k=3), 4, 0, 5)
    assert res.top_k_token_ids[:4] == [4095, 4096, 12000, 29999]
