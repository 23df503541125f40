"""Pins the CPU oracle (CPU only): torch golden vectors, closed forms, invariants and brute force.

Each oracle function is checked here by something other than a retyping of its own formula, chosen
so that a plausible slip (wrong mask direction, GQA index, missing eps, sign of rotate_half, wrong
half pairing, scale applied twice) fails at least one check.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")


# ---------------------------------------------------------------------------------------- bf16
def test_bf16_known_values():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40],
                 np.float32)
    bits = oracle.to_bf16_bits(x)
    # 1+2^-8 is a tie -> even (0x3f80); 1+3*2^-8 is a tie -> even (0x3f82)
    assert list(bits[:8]) == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x0000, 0x8000, 0x7F80, 0xFF80]
    assert bits[8] == 0x7F62  # 3.0e38 rounds within range
    nan_bits = oracle.to_bf16_bits(np.array([np.nan], np.float32))[0]
    assert (nan_bits & 0x7F80) == 0x7F80 and (nan_bits & 0x7F) != 0


def test_bf16_roundtrip_all_patterns():
    allb = np.arange(65536, dtype=np.uint16)
    f = oracle.from_bf16_bits(allb)
    back = oracle.to_bf16_bits(f)
    finite = ~np.isnan(f)
    assert np.array_equal(back[finite], allb[finite])
    # widening is exact: the low 16 bits are zero
    assert np.all((f.view(np.uint32) & 0xFFFF) == 0)


# ---------------------------------------------------------------------------------------- SDPA
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_matches_torch_golden(causal):
    o = oracle.sdpa(G["sdpa_q"], G["sdpa_k"], G["sdpa_v"], causal=causal)
    np.testing.assert_allclose(o, G[f"sdpa_c{int(causal)}_o"], rtol=1e-5, atol=1e-6)


def test_sdpa_rect_golden_explicit_scale():
    o = oracle.sdpa(G["sdpa_rect_q"], G["sdpa_rect_k"], G["sdpa_rect_v"], scale=0.3)
    np.testing.assert_allclose(o, G["sdpa_rect_o"], rtol=1e-5, atol=1e-6)


def test_sdpa_invariants():
    r = np.random.default_rng(0)
    # L = S = 1: output is V
    q, k, v = r.standard_normal((1, 2, 1, 8)), r.standard_normal((1, 1, 1, 8)), r.standard_normal((1, 1, 1, 8))
    np.testing.assert_allclose(oracle.sdpa(q, k, v), np.repeat(v, 2, axis=1), rtol=1e-6)
    # causal row 0 sees key 0 only
    q, k, v = (r.standard_normal((1, 4, 6, 8)).astype(np.float32), r.standard_normal((1, 2, 6, 8)),
               r.standard_normal((1, 2, 6, 8)))
    o = oracle.sdpa(q, k, v, causal=True)
    np.testing.assert_allclose(o[:, :, 0], np.repeat(v[:, :, 0], 2, axis=1), rtol=1e-6)
    # constant V rows give that constant
    vc = np.broadcast_to(np.arange(8, dtype=np.float32), (1, 2, 6, 8))
    np.testing.assert_allclose(oracle.sdpa(q, k, vc, causal=True), np.broadcast_to(np.arange(8.0), (1, 4, 6, 8)),
                               rtol=1e-6, atol=1e-6)
    # non-causal output is invariant to a permutation of the key/value rows
    p = r.permutation(6)
    np.testing.assert_allclose(oracle.sdpa(q, k, v), oracle.sdpa(q, k[:, :, p], v[:, :, p]), rtol=1e-5, atol=1e-6)
    # GQA equals explicit repeat of kv heads (repeat_interleave, gqa.ts:494-519)
    np.testing.assert_allclose(oracle.sdpa(q, k, v, causal=True),
                               oracle.sdpa(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), causal=True),
                               rtol=1e-6, atol=1e-7)


def test_sdpa_brute_force_numpy():
    r = np.random.default_rng(1)
    q, k, v = r.standard_normal((1, 2, 5, 4)), r.standard_normal((1, 1, 7, 4)), r.standard_normal((1, 1, 7, 4))
    scale = 0.7
    o = oracle.sdpa(q, k, v, scale=scale, causal=True)
    ref = np.zeros((1, 2, 5, 4))
    for h in range(2):
        for i in range(5):
            s = np.array([q[0, h, i] @ k[0, 0, j] * scale for j in range(7)])
            s[np.arange(7) > i] = -np.inf  # top-left causal: key j > query i masked
            p = np.exp(s - s.max())
            ref[0, h, i] = (p / p.sum()) @ v[0, 0]
    np.testing.assert_allclose(o, ref, rtol=1e-5, atol=1e-6)


def test_sdpa_kv_len_equals_truncation():
    r = np.random.default_rng(2)
    q, k, v = r.standard_normal((2, 2, 1, 8)), r.standard_normal((2, 1, 10, 8)), r.standard_normal((2, 1, 10, 8))
    o = oracle.sdpa(q, k, v, kv_len=[4, 10])
    np.testing.assert_allclose(o[0:1], oracle.sdpa(q[0:1], k[0:1, :, :4], v[0:1, :, :4]), rtol=1e-6)
    np.testing.assert_allclose(o[1:2], oracle.sdpa(q[1:2], k[1:2], v[1:2]), rtol=1e-6)


@pytest.mark.skipif(not oracle.node_available(), reason="node is not installed")
@pytest.mark.parametrize("causal", [False, True])
def test_flash_js_matches_oracle_and_torch_golden(causal):
    """The JavaScript restatement (the CPU baseline's JS leg) against the C oracle on ragged GQA
    shapes (37 rows: a partial Br = 8 block and Bc = 4 block) and against the torch golden vectors."""
    r = np.random.default_rng(4)
    q, k, v = (r.standard_normal((1, 4, 37, 16)).astype(np.float32), r.standard_normal((1, 2, 37, 16)),
               r.standard_normal((1, 2, 37, 16)))
    o, _ = oracle.flash_js(q, k, v, causal=causal)
    np.testing.assert_allclose(o, oracle.sdpa(q, k, v, causal=causal), rtol=1e-5, atol=1e-6)
    og, _ = oracle.flash_js(G["sdpa_q"], G["sdpa_k"], G["sdpa_v"], causal=causal)
    np.testing.assert_allclose(og, G[f"sdpa_c{int(causal)}_o"], rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------------------ SDPA with mask
def test_sdpa_masked_matches_torch_golden():
    o = oracle.sdpa_masked(G["sdpam_q"], G["sdpam_k"], G["sdpam_v"], G["sdpam_mask"])
    np.testing.assert_allclose(o, G["sdpam_o"], rtol=1e-5, atol=1e-6)
    # broadcast [L, S] mask holding the capture path's bottom-right causal pattern plus noise
    o = oracle.sdpa_masked(G["sdpamb_q"], G["sdpamb_k"], G["sdpamb_v"], G["sdpamb_mask"])
    np.testing.assert_allclose(o, G["sdpamb_o"], rtol=1e-5, atol=1e-6)


def test_sdpa_masked_invariants():
    r = np.random.default_rng(5)
    q, k, v = r.standard_normal((2, 4, 7, 8)), r.standard_normal((2, 2, 7, 8)), r.standard_normal((2, 2, 7, 8))
    # a zero mask is the unmasked (non-causal) attention
    np.testing.assert_allclose(oracle.sdpa_masked(q, k, v, np.zeros((7, 7))), oracle.sdpa(q, k, v),
                               rtol=1e-6, atol=1e-7)
    # -inf above the diagonal is the top-left causal attention
    tri = np.where(np.arange(7)[None, :] > np.arange(7)[:, None], -np.inf, 0.0)
    np.testing.assert_allclose(oracle.sdpa_masked(q, k, v, tri), oracle.sdpa(q, k, v, causal=True),
                               rtol=1e-6, atol=1e-7)
    # adding a constant per (batch, head, row) does not change the softmax
    m = r.standard_normal((2, 4, 7, 7))
    shift = r.standard_normal((2, 4, 7, 1)) * 5.0
    np.testing.assert_allclose(oracle.sdpa_masked(q, k, v, m), oracle.sdpa_masked(q, k, v, m + shift),
                               rtol=1e-5, atol=1e-6)
    # broadcasting over batch and heads equals the expanded mask
    m2 = r.standard_normal((7, 7))
    np.testing.assert_allclose(oracle.sdpa_masked(q, k, v, m2),
                               oracle.sdpa_masked(q, k, v, np.broadcast_to(m2, (2, 4, 7, 7)).copy()), rtol=1e-6)
    # explicit scale enters before the mask is added: scale s with mask M equals scale 1 on q*s
    np.testing.assert_allclose(oracle.sdpa_masked(q, k, v, m, scale=0.3),
                               oracle.sdpa_masked(q * 0.3, k, v, m, scale=1.0), rtol=1e-5, atol=1e-6)


def test_sdpa_masked_brute_force_and_reference_softmax_floor():
    r = np.random.default_rng(6)
    q, k, v = r.standard_normal((1, 1, 3, 4)), r.standard_normal((1, 1, 5, 4)), r.standard_normal((1, 1, 5, 4))
    m = r.standard_normal((3, 5))
    m[1, 2] = -np.inf
    o = oracle.sdpa_masked(q, k, v, m, scale=0.5)
    ref = np.zeros((3, 4))
    for i in range(3):
        x = np.array([q[0, 0, i] @ k[0, 0, j] * 0.5 + m[i, j] for j in range(5)])
        p = np.exp(x - x.max())
        ref[i] = (p / p.sum()) @ v[0, 0]
    np.testing.assert_allclose(o[0, 0], ref, rtol=1e-5, atol=1e-6)
    # The reference softmax starts its max at f32(-1e38) (shaderBuilder.ts:190-195): with q = 0 the
    # scores are the mask values themselves.
    z = np.zeros((1, 1, 4, 4))
    mk = np.array([[-1e38, -1e38, -1e38, -1e38],      # x = max floor: p = 1 each -> mean of V
                   [-3e38, -3e38, -3e38, -3e38],      # every p underflows: 0 / 0 = NaN
                   [-1.5e38, -1.2e38, -np.inf, -3e38],  # all below the floor: NaN (a plain softmax picks key 1)
                   [-np.inf, 0.0, -np.inf, -np.inf]], np.float32)  # one finite key -> that V row
    o = oracle.sdpa_masked(z, k[:, :, :4], v[:, :, :4], mk)
    np.testing.assert_allclose(o[0, 0, 0], v[0, 0, :4].mean(axis=0), rtol=1e-6)
    assert np.all(np.isnan(o[0, 0, 1])) and np.all(np.isnan(o[0, 0, 2]))
    np.testing.assert_allclose(o[0, 0, 3], v[0, 0, 1], rtol=1e-6)


def test_flash_f32_baseline_agrees_with_oracle():
    r = np.random.default_rng(3)
    q, k, v = (r.standard_normal((1, 4, 37, 16)).astype(np.float32), r.standard_normal((1, 2, 37, 16)),
               r.standard_normal((1, 2, 37, 16)))
    for causal in (False, True):
        np.testing.assert_allclose(oracle.flash_f32(q, k, v, causal=causal), oracle.sdpa(q, k, v, causal=causal),
                                   rtol=2e-5, atol=2e-6)


# ---------------------------------------------------------------------------------------- RMSNorm
def test_rms_norm_matches_torch_golden():
    np.testing.assert_allclose(oracle.rms_norm(G["rms_x"], G["rms_w"], 1e-6), G["rms_y"], rtol=1e-6, atol=1e-6)


def test_rms_norm_invariants():
    r = np.random.default_rng(4)
    x = r.standard_normal((3, 64)).astype(np.float32)
    eps = 1e-2
    y = oracle.rms_norm(x, None, eps)
    ms = (x.astype(np.float64) ** 2).mean(axis=1)
    np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(axis=1), ms / (ms + eps), rtol=1e-5)
    # scale invariance for c >> sqrt(eps)
    np.testing.assert_allclose(oracle.rms_norm(1000 * x, None, 1e-6), oracle.rms_norm(x, None, 1e-6), rtol=1e-5)


# ---------------------------------------------------------------------------------------- RoPE
def test_inv_freq_closed_form():
    inv = oracle.rope_inv_freq(128, 1e6)
    assert inv[0] == 1.0
    np.testing.assert_allclose(inv[32], 1e6 ** -0.5, rtol=1e-7)
    assert inv.dtype == np.float32 and inv.shape == (64,)


def test_rope_matches_complex_golden():
    inv = oracle.rope_inv_freq(16, float(G["rope_theta"]))
    np.testing.assert_array_equal(inv, G["rope_inv"])
    y = oracle.qk_norm_rope(G["rope_x"], None, G["rope_pos"], inv, do_norm=False)
    np.testing.assert_allclose(y, G["rope_y"], rtol=1e-5, atol=1e-6)


def test_rope_invariants():
    r = np.random.default_rng(5)
    D = 32
    inv = oracle.rope_inv_freq(D, 1e4)
    x = r.standard_normal((4, 2, D)).astype(np.float32)
    # position 0 is the identity
    np.testing.assert_allclose(oracle.qk_norm_rope(x, None, np.zeros(4), inv, do_norm=False), x, rtol=1e-6)
    # each (i, i + D/2) pair keeps its norm
    y = oracle.qk_norm_rope(x, None, np.array([3, 50, 999, 7]), inv, do_norm=False)
    h = D // 2
    np.testing.assert_allclose(x[..., :h] ** 2 + x[..., h:] ** 2, y[..., :h] ** 2 + y[..., h:] ** 2, rtol=1e-5)
    # <R(m) q, R(n) k> depends only on m - n (small positions: float32 angle rounding is negligible)
    q, k = x[:1], x[1:2]
    dots = []
    for m, n in ((5, 2), (9, 6), (13, 10)):
        qm = oracle.qk_norm_rope(q, None, [m], inv, do_norm=False)
        kn = oracle.qk_norm_rope(k, None, [n], inv, do_norm=False)
        dots.append(float((qm * kn).sum()))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-5)


def test_qk_norm_rope_is_norm_then_rope():
    r = np.random.default_rng(6)
    x = r.standard_normal((5, 3, 64)).astype(np.float32)
    w = r.uniform(0.5, 1.5, 64).astype(np.float32)
    pos = np.array([0, 1, 17, 300, 8191])
    inv = oracle.rope_inv_freq(64, 1e6)
    fused = oracle.qk_norm_rope(x, w, pos, inv, eps=1e-6)
    two_step = oracle.qk_norm_rope(oracle.rms_norm(x, w, 1e-6), None, pos, inv, do_norm=False)
    np.testing.assert_allclose(fused, two_step, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------------------- silu / linear / argmax
def test_silu_mul_golden_and_limits():
    np.testing.assert_allclose(oracle.silu_mul(G["silu_g"], G["silu_u"]), G["silu_y"], rtol=1e-6, atol=1e-7)
    s = oracle.silu_mul(np.array([0.0, 60.0, -100.0, 200.0], np.float32))
    assert s[0] == 0.0
    np.testing.assert_allclose(s[1], 60.0, rtol=1e-6)
    assert abs(s[2]) < 1e-30  # -100 / (1 + exp(88)) after the clamp
    assert s[3] == 200.0


def test_linear_golden_and_identity():
    np.testing.assert_allclose(oracle.linear(G["lin_a"], G["lin_w"], bias=G["lin_b"]), G["lin_y"], rtol=1e-6,
                               atol=1e-6)
    a = np.random.default_rng(7).standard_normal((4, 6)).astype(np.float32)
    np.testing.assert_array_equal(oracle.linear(a, np.eye(6, dtype=np.float32)), a)
    c = np.ones((4, 6), np.float32)
    np.testing.assert_allclose(oracle.linear(a, np.eye(6, dtype=np.float32), cin=c, alpha=2.0, beta=0.5),
                               2 * a + 0.5, rtol=1e-6)


def test_argmax_tie_and_nan_rules():
    x = np.array([[1.0, 3.0, 3.0, 2.0], [np.nan, 1.0, np.nan, 0.5], [-np.inf, -np.inf, -np.inf, -np.inf]],
                 np.float32)
    assert list(oracle.argmax(x)) == [1, 1, 0]


def test_argmax_tie_rule_differs_from_the_reference_kernel_only_on_ties():
    """The oracle (and the GPU kernel) return the lowest index among tied maxima; the reference's
    WGSL argmax, simulated thread by thread (oracle.argmax_workgroup_rule), depends on the
    workgroup size on ties: W = 4 with maxima at 1 and 2 gives 2, W = 256 with maxima at 1 and 256
    gives 256.  Without ties both rules agree (random rows, several workgroup sizes), and NaN /
    all -inf rows agree."""
    t4 = np.array([0.0, 5.0, 5.0, 1.0], np.float32)
    assert oracle.argmax(t4[None])[0] == 1 and oracle.argmax_workgroup_rule(t4, 4) == 2
    t = np.zeros(300, np.float32)
    t[1] = t[256] = 7.0
    assert oracle.argmax(t[None])[0] == 1 and oracle.argmax_workgroup_rule(t, 256) == 256
    rng = np.random.default_rng(3)
    rows = rng.normal(size=(6, 777)).astype(np.float32)
    for wg in (4, 64, 256):
        np.testing.assert_array_equal(oracle.argmax_workgroup_rule(rows, wg), oracle.argmax(rows))
    special = np.array([[np.nan, 1.0, np.nan, 0.5], [-np.inf] * 4], np.float32)
    np.testing.assert_array_equal(oracle.argmax_workgroup_rule(special, 4), oracle.argmax(special))


# ---------------------------------------------------------------------------------------- Qwen3 composition
def test_qwen3_oracle_matches_transformers_float32():
    """The model oracle without its bf16 rounding points reproduces Hugging Face transformers'
    Qwen3ForCausalLM (float32) on a tiny config: prefill logits, then the logits after each greedy
    token appended through the KV cache (tests/golden/make_qwen3_golden.py)."""
    from kandle_amd.model_utils.qwen3 import Qwen3Config
    from oracle.qwen3 import Qwen3Oracle

    Z = np.load(Path(__file__).resolve().parent / "golden" / "qwen3_tiny.npz")
    cfg = Qwen3Config(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6, rope_theta=1e6)
    weights = {k[2:]: Z[k] for k in Z.files if k.startswith("w:")}
    ids, P = [int(i) for i in Z["ids"]], int(Z["prompt_len"])
    ref = Qwen3Oracle(cfg, weights, max_seq_len=32, exact=True)
    steps = len(ids) - P
    toks, logits = ref.generate(ids[:P], steps + 1)
    assert toks[:steps] == ids[P:]
    for i in range(steps + 1):
        np.testing.assert_allclose(logits[i], Z["logits"][i], rtol=0, atol=2e-4 * np.abs(Z["logits"][i]).max())
