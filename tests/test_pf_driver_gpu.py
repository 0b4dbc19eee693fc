"""The prefill chunk driver (lk_pf_ctx: the attention slice of the engine's
pf_chunk, reference engine.cu:1064-1124, 1080, 1251) on the GPU: a prompt in
two chunks with decode steps in between, for two layers.  Every chunk's
attention output against the oracle run end to end on the same inputs
(producers -> int8 K over [0, pos0+m) -> Q quantiser -> same-algorithm float64
attention), the context's int8 K copy bit-exact (including the rows decode
appended, caught up through k8_valid), and the smoothing variant."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import dev, host, host_h, note

pytestmark = pytest.mark.gpu


def _copy_out(ptr, nbytes):
    """Device buffer owned by the library -> host bytes (hipMemcpy through torch)."""
    out = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ptr), ctypes.c_size_t(nbytes), 3) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("smooth", [False, True])
def test_prefill_driver_two_chunks_with_decode_between(lk, oracle, smooth):
    rng = np.random.default_rng(700 + int(smooth))
    layers, cap, mc = 2, 1024, 256
    near, sink = 96, 1
    chunks = [(0, 256), (259, 200)]                  # decode appends 256..258 in between
    note(f"prefill driver smooth={smooth}")
    ctx = lk.PrefillCtx(layers, mc, cap, attn8=True, ksmooth=smooth, near=near, sink=sink)
    W = [(rng.uniform(0.5, 1.5, 64).astype(np.float32), rng.uniform(0.5, 1.5, 64).astype(np.float32))
         for _ in range(layers)]
    kc = [torch.zeros(cap, 8, 64, dtype=torch.float16, device="cuda") for _ in range(layers)]
    vc = [torch.zeros_like(kc[0]) for _ in range(layers)]
    Kh = [np.zeros((cap, 8, 64), np.uint16) for _ in range(layers)]   # host mirrors (oracle side)
    Vh = [np.zeros((cap, 8, 64), np.uint16) for _ in range(layers)]
    cm_h = [None] * layers
    k8_valid = 0
    for ci, (pos0, m) in enumerate(chunks):
        if ci == 1:                                   # three decode steps write K/V rows
            for pos in range(256, 259):
                for l in range(layers):
                    q = (rng.standard_normal(2048) * 2).astype(np.float32)
                    k = (rng.standard_normal(512) * 2).astype(np.float32)
                    v = rng.standard_normal(512).astype(np.float32)
                    lk.qk_norm_rope(dev(q), dev(k), dev(v), dev(W[l][0]), dev(W[l][1]),
                                    torch.tensor([pos], dtype=torch.int32, device="cuda"), kc[l], vc[l])
                    kq = np.concatenate([oracle.norm_rope_row(k[h * 64:(h + 1) * 64], W[l][1], pos) for h in range(8)])
                    Kh[l][pos] = kq.reshape(8, 64).astype(np.float16).view(np.uint16)
                    Vh[l][pos] = v.reshape(8, 64).astype(np.float16).view(np.uint16)
        for l in range(layers):
            Y = (rng.standard_normal((m, 3072)) * 3).astype(np.float32)
            o = torch.full((m, 2048), float("nan"), device="cuda")
            aqs = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
            asc = torch.zeros(m, 64, 2, device="cuda")
            ctx.chunk_attn(l, dev(Y), dev(W[l][0]), dev(W[l][1]), m, pos0, kc[l], vc[l], o, aqs, asc)
            torch.cuda.synchronize()
            qso, sco = oracle.pf_quant_rows(host(o), m, 2048, 64)   # the fused Q8_1 planes
            assert np.array_equal(host(aqs), qso) and np.array_equal(host(asc).view(np.uint32), sco.view(np.uint32))
            # oracle, end to end
            qh = oracle.pf_qknr(Y, W[l][0], W[l][1], m, pos0, Kh[l].reshape(-1), Vh[l].reshape(-1))
            S = pos0 + m
            if smooth and pos0 == 0:
                cm_h[l] = oracle.pf_kmean(Kh[l].reshape(-1), m)
            cmv = cm_h[l] if smooth else None
            bufs = ctx.buffers(l)
            ks = bufs["kstride"]
            k8, ksc = oracle.pf_k8(Kh[l].reshape(-1), 0, S, ks, cmv)
            q8, qsc, qcs = oracle.pf_q8(qh, m, cmv)
            rows = np.array(sorted({0, 1, 63, 64, m // 2, m - 1}), np.int32)
            ref8 = oracle.pf_ref8(q8, qsc, qcs, qh, m, pos0, k8, ksc, ks,
                                  Kh[l].reshape(-1), Vh[l].reshape(-1), near, sink, rows=rows)
            rel = oracle.rel_err(host(o)[rows], ref8[rows])
            note(f"  chunk {ci} layer {l}: rel vs same-algorithm float64 {rel:.3e}")
            assert rel <= 2e-3
            assert np.array_equal(host_h(kc[l][:S]), Kh[l][:S]) and np.array_equal(host_h(vc[l][:S]), Vh[l][:S])
            # the context's int8 K copy over [0, S): bit-exact, rows decode wrote included
            k8_dev = _copy_out(bufs["k8"], S * 512).view(np.int8)
            assert np.array_equal(k8_dev, k8[:S * 512]), (ci, l)
            ksc_dev = _copy_out(bufs["ksc"], 8 * ks * 4).view(np.float32).reshape(8, ks)
            assert np.array_equal(ksc_dev[:, :S].view(np.uint32), ksc.reshape(8, ks)[:, :S].view(np.uint32))
            if smooth:
                cm_dev = _copy_out(bufs["cm"], 512 * 4).view(np.float32)
                assert np.array_equal(cm_dev.view(np.uint32), cm_h[l].reshape(-1).view(np.uint32))
            assert bufs["k8_valid"] == k8_valid
        ctx.chunk_done(pos0 + m)
        k8_valid = pos0 + m
    assert ctx.buffers(0)["k8_valid"] == 459
    ctx.close()
