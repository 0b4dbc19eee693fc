"""Synthetic inputs of the benchmark configurations, generated on the device.

Shapes and distributions follow the five configurations the attention path is
measured on (32 query heads, 8 KV heads, head_dim 64; decode KV cache fp16
[pos][8][64]; prefill Q already carries the 1/8 softmax scale, as the
reference's k_pf_qknr writes it, /root/reference/src/prefill.cu:1010).

Every random value comes from the seeded splitmix64 stream of its own seed,
with Box-Muller in float64 (lk_synth_f32 on the device; the same stream as the
oracle's sequential lko_sm_normal / lko_sm_uniform / lko_sm_student4), so the
inputs do not depend on a library's generator.  The seed of a tensor is
seed_of(config, layer, tensor) below.  What follows the draws -- per-head RMS
normalisation, gains, scales, the fp16 rounding -- is plain fp32 arithmetic in
torch.  Large configurations (2.7 GB of KV) take milliseconds on the device.
Parity tests compare against the CPU oracle by copying these tensors to the host.
"""
from __future__ import annotations

import torch

import lk_attn as lk

H, KV, D = 32, 8, 64
_CFG_ID = {"C1": 1, "C2": 2, "C3": 3, "C4": 4, "C5": 5}
# tensor tags
T_Q, T_K, T_V, T_GAIN, T_PEAK, T_CHAN = 1, 2, 3, 4, 5, 6
_M64 = (1 << 64) - 1
_GAMMA = 0x9E3779B97F4A7C15


def seed_of(cfg: str, layer: int, tensor: int, base: int = 0) -> int:
    """64-bit seed of one tensor: 0x5EED in the top bits, then the
    configuration, the layer and the tensor tag (and a caller's base)."""
    return (0x5EED << 48 | _CFG_ID[cfg] << 40 | (base & 0xFF) << 32 | (layer & 0xFFFF) << 8 | tensor) & _M64


def sm64_draws(seed: int, n: int) -> list:
    """The first n splitmix64 outputs of `seed` (host, for small choices)."""
    out, x = [], seed
    for _ in range(n):
        x = (x + _GAMMA) & _M64
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
        out.append(z ^ (z >> 31))
    return out


def _draw(kind, seed, shape, lo=0.0, hi=1.0, device="cuda"):
    t = torch.empty(*shape, dtype=torch.float32, device=device)
    lk.synth(kind, seed, t, lo, hi)
    return t


def _rmsnorm(x: torch.Tensor) -> torch.Tensor:
    return x * torch.rsqrt((x.float() ** 2).mean(-1, keepdim=True))


def decode_inputs(cfg: str, seed: int = 1, layers: int = 1, device="cuda", seq: int = None):
    """q fp32 [32][64] per layer, kc/vc fp16 [seq][8][64] per layer, seq.
    `seq` overrides the configuration's context length (same distributions),
    for the decode curve over context lengths.

    C1: ctx 4096, q/K/V N(0,1) RMS-normalised per head (q rounded to fp16).
    C2: ctx 32768, K N(0,1) RMS-normalised times a per-channel gain U(0.5, 2),
        V N(0,1), q RMS-normalised.
    C3: ctx 131072, K/V N(0,1); the positions whose uniform draw is below 0.01
        (about 1%, a seeded set) have their K and V rows scaled x8.
    """
    seq = seq or {"C1": 4096, "C2": 32768, "C3": 131072}[cfg]
    qs, kcs, vcs = [], [], []
    N, U = lk.SYNTH_NORMAL, lk.SYNTH_UNIFORM
    for layer in range(layers):
        q = _draw(N, seed_of(cfg, layer, T_Q, seed), (H, D), device=device)
        k = _draw(N, seed_of(cfg, layer, T_K, seed), (seq, KV, D), device=device)
        v = _draw(N, seed_of(cfg, layer, T_V, seed), (seq, KV, D), device=device)
        if cfg in ("C1", "C2"):
            q = _rmsnorm(q)
            k = _rmsnorm(k)
        if cfg == "C1":
            v = _rmsnorm(v)
            q = q.half().float()
        if cfg == "C2":
            k = k * _draw(U, seed_of(cfg, layer, T_GAIN, seed), (KV, D), 0.5, 2.0, device=device)
        if cfg == "C3":
            peak = _draw(U, seed_of(cfg, layer, T_PEAK, seed), (seq,), device=device) < 0.01
            k[peak] *= 8.0
            v[peak] *= 8.0
        qs.append(q.contiguous())
        kcs.append(k.half().contiguous())
        vcs.append(v.half().contiguous())
        del k, v
    return qs, kcs, vcs, seq


def outlier_channels(seed: int = 2) -> list:
    """C5's two outlier channels of 64: the first two distinct values of
    (draw mod 64) of the channel seed's stream."""
    ch = []
    for x in sm64_draws(seed_of("C5", 0, T_CHAN, seed), 16):
        c = x % D
        if c not in ch:
            ch.append(c)
        if len(ch) == 2:
            return ch
    raise RuntimeError("no two distinct channels in 16 draws")


def prefill_inputs(cfg: str, seed: int = 2, device="cuda"):
    """qh fp16 [S][2048] (x 1/8), kc/vc fp16 [S][8][64] for the whole prompt.

    C4: one 4096-token chunk at P = 0; Q = N(0,1)*1.5/8, K = N(0,1)*1.5,
        V = N(0,1) (the reference test recipe, test_prefill.cu:250-256).
    C5: a 131072-token prompt; Q and K Student-t (nu = 4) with the 2 channels
        of outlier_channels() scaled x20; V = N(0,1).
    """
    S = {"C4": 4096, "C5": 131072}[cfg]
    N, T4 = lk.SYNTH_NORMAL, lk.SYNTH_STUDENT4
    if cfg == "C4":
        q = _draw(N, seed_of(cfg, 0, T_Q, seed), (S, H * D), device=device) * 1.5
        k = _draw(N, seed_of(cfg, 0, T_K, seed), (S, KV, D), device=device) * 1.5
    else:
        q = _draw(T4, seed_of(cfg, 0, T_Q, seed), (S, H, D), device=device)
        k = _draw(T4, seed_of(cfg, 0, T_K, seed), (S, KV, D), device=device)
        ch = outlier_channels(seed)
        q[..., ch] *= 20.0
        k[..., ch] *= 20.0
        q = q.reshape(S, H * D)
    v = _draw(N, seed_of(cfg, 0, T_V, seed), (S, KV, D), device=device)
    qh = (q * 0.125).half().contiguous()
    del q
    return qh, k.half().contiguous(), v.half().contiguous(), S
