"""Attention-input producers on the GPU, through the C ABI: per-head RMS norm +
NEOX RoPE + fp16 KV-cache write for one decode token (lk_qk_norm_rope) and
for a prefill chunk (lk_pf_qknr, optionally emitting the int8 K copy).

Bit-exact against the oracle restatement (the transcendental values are
correctly rounded on both sides), and -- the reference's own gate,
tests/test_prefill.cu:463-504 -- the prefill kernel's Q / K / V equal the decode
kernel's per token, byte for byte.  The fused int8 K rows equal lk_pf_k8's.
"""
import numpy as np
import pytest
import torch

from gpu_util import dev, dev_h, host, host_h, note

pytestmark = pytest.mark.gpu


def _weights(rng):
    return rng.uniform(0.5, 1.5, 64).astype(np.float32), rng.uniform(0.5, 1.5, 64).astype(np.float32)


@pytest.mark.parametrize("pos", [0, 1, 1000, 131071])
def test_decode_producer_bit_exact(lk, oracle, pos):
    rng = np.random.default_rng(300 + pos % 97)
    qn, kn = _weights(rng)
    q = (rng.standard_normal(2048) * 2.0).astype(np.float32)
    k = (rng.standard_normal(512) * 2.0).astype(np.float32)
    v = rng.standard_normal(512).astype(np.float32)
    note(f"qk_norm_rope decode pos={pos}")
    S = pos + 1
    kc = torch.zeros(S, 8, 64, dtype=torch.float16, device="cuda")
    vc = torch.zeros(S, 8, 64, dtype=torch.float16, device="cuda")
    qd, kd = dev(q), dev(k)
    lk.qk_norm_rope(qd, kd, dev(v), dev(qn), dev(kn), torch.tensor([pos], dtype=torch.int32, device="cuda"), kc, vc)
    torch.cuda.synchronize()
    # oracle on the rows only (a full-length host cache is not needed)
    qrows = [oracle.norm_rope_row(q[h * 64:(h + 1) * 64], qn, pos) for h in range(32)]
    krows = [oracle.norm_rope_row(k[h * 64:(h + 1) * 64], kn, pos) for h in range(8)]
    qo, ko = np.concatenate(qrows), np.concatenate(krows)
    assert np.array_equal(host(qd).view(np.uint32), qo.view(np.uint32))
    assert np.array_equal(host(kd).view(np.uint32), ko.view(np.uint32))
    assert np.array_equal(host_h(kc[pos]).reshape(-1), ko.astype(np.float16).view(np.uint16))
    assert np.array_equal(host_h(vc[pos]).reshape(-1), v.astype(np.float16).view(np.uint16))
    if pos > 0:
        assert not bool(kc[:pos].any()) and not bool(vc[:pos].any())


@pytest.mark.parametrize("m,P", [(6, 1000), (300, 0), (70, 130000)])
def test_prefill_producer_bit_exact_and_equals_decode(lk, oracle, m, P):
    rng = np.random.default_rng(400 + m)
    qn, kn = _weights(rng)
    Y = (rng.standard_normal((m, 3072)) * 3.0).astype(np.float32)
    S = P + m
    note(f"pf_qknr m={m} P={P}")
    kc = torch.zeros(S, 8, 64, dtype=torch.float16, device="cuda")
    vc = torch.zeros(S, 8, 64, dtype=torch.float16, device="cuda")
    qh = torch.zeros(m, 2048, dtype=torch.float16, device="cuda")
    Yd, qnd, knd = dev(Y), dev(qn), dev(kn)
    lk.pf_qknr(Yd, qnd, knd, m, P, qh, kc, vc)
    torch.cuda.synchronize()
    kco = np.zeros((S, 8, 64), np.uint16)
    vco = np.zeros((S, 8, 64), np.uint16)
    qho = oracle.pf_qknr(Y, qn, kn, m, P, kco.reshape(-1), vco.reshape(-1))
    assert np.array_equal(host_h(qh), qho)
    assert np.array_equal(host_h(kc[P:]), kco[P:]) and np.array_equal(host_h(vc[P:]), vco[P:])
    # the decode kernel, token by token, into a second cache
    kc1 = torch.zeros_like(kc)
    vc1 = torch.zeros_like(vc)
    d_pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    for t in range(min(m, 8)):
        qf, kf, vf = Yd[t, :2048].clone(), Yd[t, 2048:2560].clone(), Yd[t, 2560:].clone()
        d_pos.fill_(P + t)
        lk.qk_norm_rope(qf, kf, vf, qnd, knd, d_pos, kc1, vc1)
        torch.cuda.synchronize()
        assert torch.equal((qf * 0.125).half().view(torch.int16), qh[t].view(torch.int16)), t
        assert torch.equal(kc1[P + t].view(torch.int16), kc[P + t].view(torch.int16)), t
        assert torch.equal(vc1[P + t].view(torch.int16), vc[P + t].view(torch.int16)), t


@pytest.mark.parametrize("smooth", [False, True])
def test_prefill_producer_fused_k8_equals_pf_k8(lk, oracle, smooth):
    rng = np.random.default_rng(500 + int(smooth))
    qn, kn = _weights(rng)
    m, P = 200, 4000
    S = P + m
    ks = lk.kstride_for(S)
    Y = (rng.standard_normal((m, 3072)) * 3.0).astype(np.float32)
    note(f"pf_qknr fused k8 smooth={smooth}")
    kc = torch.zeros(S, 8, 64, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    qh = torch.zeros(m, 2048, dtype=torch.float16, device="cuda")
    cm = dev(rng.standard_normal((8, 64)).astype(np.float32) * 0.3) if smooth else None
    k8a = torch.zeros(S * 512, dtype=torch.int8, device="cuda")
    ksa = torch.zeros(8 * ks + 4, device="cuda")
    lk.pf_qknr(dev(Y), dev(qn), dev(kn), m, P, qh, kc, vc, k8a, ksa, ks, cm)
    k8b = torch.zeros_like(k8a)
    ksb = torch.zeros_like(ksa)
    lk.pf_k8(kc, P, S, cm, ks, k8b, ksb)
    torch.cuda.synchronize()
    assert torch.equal(k8a, k8b)
    assert torch.equal(ksa.view(torch.int32), ksb.view(torch.int32))
    assert bool(k8a.view(S, 512)[P:].any()) and not bool(k8a.view(S, 512)[:P].any())
