"""Synthetic inputs of the benchmark configurations, generated on the device.

Shapes and distributions follow the five configurations the attention path is
measured on (32 query heads, 8 KV heads, head_dim 64; decode KV cache fp16
[pos][8][64]; prefill Q already carries the 1/8 softmax scale, as the
reference's k_pf_qknr writes it, /root/reference/src/prefill.cu:1010).  Values
come from torch's seeded device generator: reproducible on one software stack,
and large configurations (2.7 GB of KV) are generated in milliseconds instead of
host minutes.  Parity tests compare against the CPU oracle by copying these
tensors to the host.
"""
from __future__ import annotations

import torch

H, KV, D = 32, 8, 64


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _rmsnorm(x: torch.Tensor) -> torch.Tensor:
    return x * torch.rsqrt((x.float() ** 2).mean(-1, keepdim=True))


def decode_inputs(cfg: str, seed: int = 1, layers: int = 1, device="cuda"):
    """q fp32 [32][64] per layer, kc/vc fp16 [seq][8][64] per layer, seq.

    C1: ctx 4096, q/K/V N(0,1) RMS-normalised per head.
    C2: ctx 32768, K N(0,1) RMS-normalised times a per-channel gain U(0.5, 2),
        V N(0,1), q RMS-normalised.
    C3: ctx 131072, K/V N(0,1), 1% of positions (seeded) with K scaled x8.
    """
    seq = {"C1": 4096, "C2": 32768, "C3": 131072}[cfg]
    g = _gen(seed, device)
    qs, kcs, vcs = [], [], []
    for _ in range(layers):
        q = torch.randn(H, D, generator=g, device=device)
        k = torch.randn(seq, KV, D, generator=g, device=device)
        v = torch.randn(seq, KV, D, generator=g, device=device)
        if cfg in ("C1", "C2"):
            q = _rmsnorm(q)
            k = _rmsnorm(k)
        if cfg == "C1":
            v = _rmsnorm(v)
            q = q.half().float()
        if cfg == "C2":
            gain = torch.rand(KV, D, generator=g, device=device) * 1.5 + 0.5
            k = k * gain
        if cfg == "C3":
            n_peak = seq // 100
            idx = torch.randperm(seq, generator=g, device=device)[:n_peak]
            k[idx] *= 8.0
        qs.append(q.contiguous())
        kcs.append(k.half().contiguous())
        vcs.append(v.half().contiguous())
        del k, v
    return qs, kcs, vcs, seq


def prefill_inputs(cfg: str, seed: int = 2, device="cuda"):
    """qh fp16 [S][2048] (x 1/8), kc/vc fp16 [S][8][64] for the whole prompt.

    C4: one 4096-token chunk at P = 0; Q = N(0,1)*1.5/8, K = N(0,1)*1.5,
        V = N(0,1) (the reference test recipe, test_prefill.cu:250-256).
    C5: a 131072-token prompt; Q and K Student-t (nu = 4) with 2 of the 64
        channels (seeded) scaled x20; V = N(0,1).
    """
    S = {"C4": 4096, "C5": 131072}[cfg]
    g = _gen(seed, device)
    if cfg == "C4":
        q = torch.randn(S, H * D, generator=g, device=device) * 1.5
        k = torch.randn(S, KV, D, generator=g, device=device) * 1.5
    else:
        def student4(shape):
            z = torch.randn(*shape, generator=g, device=device)
            c = (torch.randn(*shape, 4, generator=g, device=device) ** 2).sum(-1)
            return z / torch.sqrt(c / 4.0)
        q = student4((S, H, D))
        k = student4((S, KV, D))
        ch = torch.randperm(D, generator=g, device=device)[:2]
        q[..., ch] *= 20.0
        k[..., ch] *= 20.0
        q = q.reshape(S, H * D)
    v = torch.randn(S, KV, D, generator=g, device=device)
    qh = (q * 0.125).half().contiguous()
    return qh, k.half().contiguous(), v.half().contiguous(), S
