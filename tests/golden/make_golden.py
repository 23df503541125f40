"""Writes tests/golden/golden.npz: small input/output vectors from PyTorch (CPU, float64), an
implementation independent of both the reference and this repository's oracle.

The reference repository ships no golden vectors for this path (its test modules are absent from
the snapshot), so these torch vectors pin the oracle together with the closed-form and invariant
checks in tests/test_oracle.py.

  * sdpa: torch.nn.functional.scaled_dot_product_attention (causal = top-left lower-triangular mask,
    enable_gqa maps query head h to kv head h // (Hq / Hkv)), float64.
  * rms_norm: torch.nn.functional.rms_norm, float64.
  * rope: the rotation written as a complex multiplication (x_i + i x_{i+D/2}) * exp(i f_i) with
    torch.polar — a different formulation from the real rotate_half form the oracle uses; the angle
    f_i = float32(float32(pos) * inv_freq_i) is the reference's float32 product.
  * silu_mul: torch.nn.functional.silu(g) * u, float64.
  * linear: torch.nn.functional.linear, float64.
  * sdpam / sdpamb: scaled_dot_product_attention with a float attn_mask (added to the scaled scores),
    float64: a full [B,H,L,S] mask with -inf entries under GQA, and a broadcast [L,S] mask holding the
    bottom-right causal pattern of the reference's capture path plus noise.

Run: python tests/golden/make_golden.py   (CPU only; writes the .npz beside this file)
"""
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "golden.npz"


def main():
    g = torch.Generator().manual_seed(1234)
    d = {}

    def randn(*shape):
        return torch.randn(*shape, generator=g, dtype=torch.float32)

    # ---- SDPA: GQA 4/2 heads, L=S=9, D=16, causal and not; plus a non-square non-causal case ----
    q, k, v = randn(2, 4, 9, 16), randn(2, 2, 9, 16), randn(2, 2, 9, 16)
    for causal in (False, True):
        o = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=causal, enable_gqa=True)
        d[f"sdpa_c{int(causal)}_o"] = o.float().numpy()
    d["sdpa_q"], d["sdpa_k"], d["sdpa_v"] = q.numpy(), k.numpy(), v.numpy()
    q2, k2, v2 = randn(1, 2, 3, 8), randn(1, 1, 11, 8), randn(1, 1, 11, 8)
    d["sdpa_rect_q"], d["sdpa_rect_k"], d["sdpa_rect_v"] = q2.numpy(), k2.numpy(), v2.numpy()
    d["sdpa_rect_o"] = F.scaled_dot_product_attention(q2.double(), k2.double(), v2.double(), scale=0.3,
                                                      enable_gqa=True).float().numpy()

    # ---- RMSNorm ----
    x = randn(5, 24) * 3.0
    w = torch.rand(24, generator=g) + 0.5
    d["rms_x"], d["rms_w"] = x.numpy(), w.numpy()
    d["rms_y"] = F.rms_norm(x.double(), (24,), w.double(), eps=1e-6).float().numpy()

    # ---- RoPE (complex formulation) ----
    T, H, D, theta = 6, 3, 16, 10000.0
    xr = randn(T, H, D)
    pos = torch.tensor([0, 1, 2, 7, 100, 4095], dtype=torch.int32)
    half = D // 2
    inv = torch.tensor([1.0 / (theta ** (i / half)) for i in range(half)], dtype=torch.float64).float()
    ang = pos.float()[:, None] * inv[None, :]                      # float32 product
    rot = torch.polar(torch.ones_like(ang, dtype=torch.float64), ang.double())  # exp(i f)
    z = torch.complex(xr[..., :half].double(), xr[..., half:].double()) * rot[:, None, :]
    d["rope_x"], d["rope_pos"], d["rope_inv"] = xr.numpy(), pos.numpy(), inv.numpy()
    d["rope_theta"] = np.array(theta)
    d["rope_y"] = torch.cat([z.real, z.imag], dim=-1).float().numpy()

    # ---- silu * mul ----
    gt, ut = randn(4, 10) * 4.0, randn(4, 10)
    d["silu_g"], d["silu_u"] = gt.numpy(), ut.numpy()
    d["silu_y"] = (F.silu(gt.double()) * ut.double()).float().numpy()

    # ---- linear ----
    a, wt, b = randn(3, 7), randn(5, 7), randn(5)
    d["lin_a"], d["lin_w"], d["lin_b"] = a.numpy(), wt.numpy(), b.numpy()
    d["lin_y"] = F.linear(a.double(), wt.double(), b.double()).float().numpy()

    # ---- SDPA with an explicit additive float mask (GQA 4/2 heads; a full [B,H,L,S] mask with
    #      -inf entries, and a broadcast [L,S] bottom-right causal mask on a rectangular case) ----
    qm, km, vm = randn(2, 4, 9, 16), randn(2, 2, 9, 16), randn(2, 2, 9, 16)
    mm = randn(2, 4, 9, 9) * 2.0
    drop = torch.rand(2, 4, 9, 9, generator=g) < 0.3
    drop[..., 0] = False  # keep one finite score per row
    mm = mm.masked_fill(drop, float("-inf"))
    d["sdpam_q"], d["sdpam_k"], d["sdpam_v"], d["sdpam_mask"] = qm.numpy(), km.numpy(), vm.numpy(), mm.numpy()
    d["sdpam_o"] = F.scaled_dot_product_attention(qm.double(), km.double(), vm.double(), attn_mask=mm.double(),
                                                   enable_gqa=True).float().numpy()
    qr, kr, vr = randn(1, 2, 5, 8), randn(1, 2, 11, 8), randn(1, 2, 11, 8)
    L, S = 5, 11
    br = torch.zeros(L, S)
    for i in range(L):
        for j in range(S):
            if j > i + (S - L):
                br[i, j] = float("-inf")
    br = br + randn(L, S) * 0.5
    d["sdpamb_q"], d["sdpamb_k"], d["sdpamb_v"], d["sdpamb_mask"] = qr.numpy(), kr.numpy(), vr.numpy(), br.numpy()
    d["sdpamb_o"] = F.scaled_dot_product_attention(qr.double(), kr.double(), vr.double(),
                                                   attn_mask=br.double()).float().numpy()

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({len(d)} arrays)")


if __name__ == "__main__":
    main()
