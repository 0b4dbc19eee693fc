"""Q4_0 x planar Q8_1 GEMM (the consumer of the prefill attention output) on
the GPU, through the C ABI.

The kernel accumulates every (token, row) over the blocks in order with the
reference's fma sequence (k_pf_mmq, PF_EPI2), so every case is checked bit for
bit against the oracle: the attention-output shape (2048 x 2048) and others
(K staged through LDS 4 blocks per stage, token counts off the 128-token workgroup tile, the
residual add, the per-token scale), and the chain from lk_pf_attn8_q81's
planar Q8_1 output -- also against the float64 product of the dequantised
weights and the float64 attention output as a sanity bound.
"""
import numpy as np
import pytest
import torch

from gpu_util import dev, dev_h, host, note

pytestmark = pytest.mark.gpu


def _weights(rng, N, bpr):
    qs = rng.integers(0, 256, (N, bpr, 16), dtype=np.uint8)
    d = rng.uniform(0.002, 0.02, (N, bpr)).astype(np.float16).view(np.uint16)
    return qs, d


def _run(lk, qs, d, N, bpr, aqs, asc, ntok, out0, add, scale):
    out = dev(out0.astype(np.float32))
    lk.pf_gemm_q4_0(dev(qs.reshape(-1)), dev(d.reshape(-1).view(np.int16)), N, bpr, dev(aqs.reshape(-1)),
                    dev(asc.reshape(-1)), ntok, out, out0.shape[1], add, None if scale is None else dev(scale))
    torch.cuda.synchronize()
    return host(out)


SHAPES = [(2048, 64, 256), (128, 64, 100), (128, 8, 1), (384, 72, 65), (128, 16, 3), (256, 96, 130)]


@pytest.mark.parametrize("N,bpr,ntok", SHAPES, ids=[f"N{a}_b{b}_t{c}" for a, b, c in SHAPES])
@pytest.mark.parametrize("mode", ["plain", "residual_scale"])
def test_pf_gemm_bit_exact(lk, oracle, N, bpr, ntok, mode):
    rng = np.random.default_rng(N + 7 * bpr + ntok)
    qs, d = _weights(rng, N, bpr)
    aqs, asc = oracle.pf_quant_rows(rng.standard_normal((ntok, bpr * 32)).astype(np.float32), ntok, bpr * 32, bpr)
    out_ld = N + (4 if mode == "residual_scale" else 0)
    out0 = rng.standard_normal((ntok, out_ld)).astype(np.float32)
    add = mode == "residual_scale"
    scale = rng.uniform(0.5, 2.0, ntok).astype(np.float32) if add else None
    note(f"pf gemm q4_0 N={N} bpr={bpr} ntok={ntok} {mode}")
    got = _run(lk, qs, d, N, bpr, aqs, asc, ntok, out0, add, scale)
    want = oracle.pf_gemm_q4_0(qs, d, N, bpr, aqs, asc, ntok, scale=scale, out=out0, out_ld=out_ld, add=add)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_attention_output_chain(lk, oracle):
    """A 300-token chunk at P = 700: int8 attention straight to planar Q8_1
    (lk_pf_attn8_q81), then the attention-output GEMM with the residual add
    (engine.cu:1126-1131)."""
    rng = np.random.default_rng(77)
    m, P = 300, 700
    S = P + m
    K, V, Q = oracle.mt_prefill_case(4242, m, P, 0.0, False)
    ks = lk.kstride_for(S)
    kc, vc, qh = dev_h(K), dev_h(V), dev_h(Q)
    q8 = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
    qsc = torch.zeros(m, 32, device="cuda"); qcs = torch.zeros(m, 32, device="cuda")
    k8 = torch.zeros(S * 512, dtype=torch.int8, device="cuda"); ksc = torch.zeros(8 * ks + 4, device="cuda")
    aqs = torch.zeros(m, 2048, dtype=torch.int8, device="cuda"); asc = torch.zeros(m, 64, 2, device="cuda")
    note(f"prefill attention -> planar Q8_1 -> attn_output GEMM, m={m} P={P}")
    lk.pf_q8(qh, m, None, q8, qsc, qcs)
    lk.pf_k8(kc, 0, S, None, ks, k8, ksc)
    lk.pf_attn8_q81(q8, qsc, qcs, qh, m, P, k8, ksc, ks, kc, vc, 96, 1, None, aqs, asc)
    qsw, dw = _weights(rng, 2048, 64)
    x0 = rng.standard_normal((m, 2048)).astype(np.float32)
    x = dev(x0)
    lk.pf_gemm_q4_0(dev(qsw.reshape(-1)), dev(dw.reshape(-1).view(np.int16)), 2048, 64, aqs, asc, m, x, 2048, True)
    torch.cuda.synchronize()
    got = host(x)
    want = oracle.pf_gemm_q4_0(qsw, dw, 2048, 64, host(aqs), host(asc), m, out=x0, add=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # sanity: float64 dequantised weights times the float64 attention output (sampled rows)
    rows = np.array([0, 1, 150, 299])
    o = oracle.pf_ref(Q, m, P, K, V, rows=rows)[rows]
    w = (np.concatenate([(qsw & 0x0F), (qsw >> 4)], axis=2).astype(np.float64) - 8.0) \
        * dw.view(np.float16).astype(np.float64)[:, :, None]
    ref = o @ w.reshape(2048, 2048).T
    delta = got[rows].astype(np.float64) - x0[rows]
    assert np.max(np.abs(delta - ref)) / np.max(np.abs(ref)) < 5e-2
