"""Q4_0 x Q8_1 GEMV (the consumer of the decode attention output) on the GPU,
through the C ABI.

Mirrors the reference's gate G2 (tests/test_quant.cu: real weight blocks from
ref/quant_fixture.bin against their expected dot products, 5e-3 / 5e-2
relative) and its GEMV isolation test (tests/test_gemv.cu: quantise a known
input, GEMV, compare), with synthetic weights where the model's are not
available.  The kernel follows the oracle's arithmetic exactly (lane sums in
block order, the 32-lane xor-butterfly, contraction off), so every synthetic
case is checked bit for bit; the attention -> combine Q8_1 -> GEMV chain is
checked bit for bit on the GPU's own Q8_1 blocks and, as a sanity bound,
against the float64 product of the dequantised weights and the float64
attention output.
"""
import os

import numpy as np
import pytest
import torch

from gpu_util import d_pos_for, dev, dev_h, host, note

pytestmark = pytest.mark.gpu

GOLDEN_Q4 = os.path.join(os.path.dirname(__file__), "golden", "q4_0_dot.npz")


def _weights(rng, rows, bpr):
    qs = rng.integers(0, 256, (rows, bpr, 16), dtype=np.uint8)
    d = rng.uniform(0.002, 0.02, (rows, bpr)).astype(np.float16).view(np.uint16)
    return qs, d


def _run(lk, qs, d, xq, rows, bpr, y0=None, add=False, ssq=None, eps=1e-5):
    y = dev(np.zeros(rows, np.float32) if y0 is None else y0.astype(np.float32))
    lk.gemv_q4_0(dev(qs.reshape(-1)), dev(d.reshape(-1).view(np.int16)), dev(xq.reshape(-1)), rows, bpr, y,
                 add, None if ssq is None else dev(ssq), eps)
    torch.cuda.synchronize()
    return host(y)


SHAPES = [(2048, 64), (100, 8), (33, 1), (7, 40), (64, 256), (9, 96), (1, 64)]


@pytest.mark.parametrize("rows,bpr", SHAPES, ids=[f"r{r}_b{b}" for r, b in SHAPES])
@pytest.mark.parametrize("mode", ["plain", "residual", "norm"])
def test_gemv_bit_exact(lk, oracle, rows, bpr, mode):
    rng = np.random.default_rng(rows * 1000 + bpr)
    qs, d = _weights(rng, rows, bpr)
    xq = oracle.quantize_q8_1_blocks(rng.standard_normal(bpr * 32).astype(np.float32))
    y0 = rng.standard_normal(rows).astype(np.float32) if mode == "residual" else None
    ssq = rng.uniform(0.0, 30.0, 64).astype(np.float32) if mode == "norm" else None
    note(f"gemv q4_0 rows={rows} bpr={bpr} {mode}")
    got = _run(lk, qs, d, xq, rows, bpr, y0, mode == "residual", ssq)
    want = oracle.gemv_q4_0(qs, d, xq, rows, bpr, y=y0, add=(mode == "residual"), ssq=ssq)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemv_reference_fixture(lk, oracle):
    """ref/quant_fixture.bin's Q4_0 cases (real attn_q weight blocks) as one-row
    GEMVs: against the reference's expected values with its own bounds, and bit
    for bit against the oracle."""
    z = np.load(GOLDEN_Q4)
    for i in range(int(z["n"])):
        qs, d, x, (exact, fp32) = z[f"qs{i}"], z[f"d{i}"], z[f"x{i}"], z[f"expected{i}"]
        bpr = qs.shape[0]
        xq = oracle.quantize_q8_1_blocks(x)
        note(f"gemv fixture case {i} bpr={bpr}")
        got = _run(lk, qs.reshape(1, bpr, 16), d.reshape(1, bpr), xq, 1, bpr)[0]
        want = oracle.gemv_q4_0(qs.reshape(1, bpr, 16), d.reshape(1, bpr), xq, 1, bpr)[0]
        assert got == want
        assert abs(got - exact) / abs(exact) < 5e-3 and abs(got - fp32) / abs(fp32) < 5e-2


def test_attention_output_chain(lk, oracle):
    """Decode attention at 4096 positions -> the combine's Q8_1 blocks -> the
    attention-output GEMV with the residual add (engine.cu:640-657)."""
    rng = np.random.default_rng(2024)
    seq = 4096
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    qs, d = _weights(rng, 2048, 64)
    x0 = rng.standard_normal(2048).astype(np.float32)
    note("decode attention -> Q8_1 -> attn_output GEMV, seq 4096")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    out = torch.empty(32, 64, device="cuda")
    yq8 = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")
    lk.attn_decode(dev(q), dev_h(kc.view(np.uint16)), dev_h(vc.view(np.uint16)), d_pos_for(seq), part, out, yq8)
    x = dev(x0)
    lk.gemv_q4_0(dev(qs.reshape(-1)), dev(d.reshape(-1).view(np.int16)), yq8, 2048, 64, x, True)
    torch.cuda.synchronize()
    got, yb = host(x), host(yq8).reshape(64, 36)
    # bit for bit on the GPU's own Q8_1 blocks
    want = oracle.gemv_q4_0(qs, d, yb, 2048, 64, y=x0, add=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # sanity: the float64 product of the dequantised weights and the float64
    # attention output (the gap is the Q8_1 rounding of the activation)
    o = oracle.decode_ref(q, kc.view(np.uint16), vc.view(np.uint16), seq).reshape(-1)
    w = (np.concatenate([(qs & 0x0F), (qs >> 4)], axis=2).astype(np.float64) - 8.0) \
        * d.view(np.float16).astype(np.float64)[:, :, None]
    ref = x0.astype(np.float64) + w.reshape(2048, 2048) @ o
    delta = got.astype(np.float64) - x0
    assert np.max(np.abs(delta - (ref - x0))) / np.max(np.abs(ref - x0)) < 5e-2
