"""Online-softmax range handling on the GPU, through the C ABI.

Random inputs rarely move the running max by more than the kernels' headroom
after the first tile, so the rescale branch and the overflow test are driven
here on purpose, each case against the float64 reference of the same
algorithm (prefill: tests/test_prefill.cu:263-282 and the int8 restatement;
decode: tests/test_attn.cu:46-74):

* ramp  -- every key scores far above the previous ones (the max moves past the
  headroom on every tile, so every tile rescales);
* spike -- one key 43 log2 units above the rest (every other p underflows once
  the spike is seen, but not before it);
* jump  -- one key ~290 log2 units above the rest, so 2^(x - m) overflows fp32
  on the tile that holds it (inf is caught by the overflow test);
* step  -- the second half of the keys scores 7-9 log2 units above the first:
  one decode rescale per row, after which the earlier keys still carry a
  visible share of the weight;
* step14 / step21 -- the same with +14.4 / +21.6 log2 units: the prefill
  kernels raise their exponent offset only once some p reaches 2^15 (20 log2
  units above the offset's max), so step14 runs on with p up to 2^9.4 and
  step21 rescales just past that limit.

Prefill runs unsplit, auto-split, in parts of 2 tiles (the combine then
merges parts whose maxima differ by hundreds of log2 units) and as the paired
launch (two 4-wave groups per workgroup, merged in LDS).
"""
import numpy as np
import pytest
import torch

from gpu_util import abs_err, d_pos_for, dev, dev_h, host, note

pytestmark = pytest.mark.gpu


def _prefill_case(kind, m, P, seed):
    S = P + m
    rng = np.random.default_rng(seed)
    Q = (rng.standard_normal((m, 32, 64)) * 0.2).astype(np.float32)
    K = (rng.standard_normal((S, 8, 64)) * 0.5).astype(np.float32)
    V = rng.standard_normal((S, 8, 64)).astype(np.float32)
    Q[:, :, 0] = 1.0
    if kind == "ramp":
        K[:, :, 0] = 0.25 * np.arange(S, dtype=np.float32)[:, None]     # +23 log2 units per tile
    elif kind == "spike":
        K[S // 2, :, 0] = 30.0
    elif kind == "jump":
        K[S // 2, :, 0] = 200.0
    elif kind == "step":
        K[S // 2:, :, 0] += 5.0                                         # +7.2 log2 units
    elif kind == "step14":
        K[S // 2:, :, 0] += 10.0                                        # +14.4 log2 units
    elif kind == "step21":
        K[S // 2:, :, 0] += 15.0                                        # +21.6 log2 units
    f16 = lambda a: a.astype(np.float16).view(np.uint16).reshape(-1)
    return f16(K), f16(V), f16(Q)


CASES = [("ramp", 200, 300, 96), ("spike", 200, 300, 96), ("jump", 200, 300, 96),
         ("step", 200, 300, 96), ("step", 100, 2000, 0), ("ramp", 130, 0, 1024), ("jump", 64, 1000, 0),
         ("step14", 200, 300, 96), ("step21", 200, 300, 96), ("step21", 300, 0, 1024), ("step14", 256, 1000, 0)]


@pytest.mark.parametrize("kind,m,P,near", CASES, ids=[f"{c[0]}_m{c[1]}_P{c[2]}_n{c[3]}" for c in CASES])
@pytest.mark.parametrize("split", [-1, 0, 2, "pair"], ids=["unsplit", "auto", "parts2", "paired"])
def test_prefill_range(lk, oracle, kind, m, P, near, split):
    K, V, Q = _prefill_case(kind, m, P, seed=m + P)
    S = P + m
    sink = int(near > 0)
    note(f"pf softmax range {kind} m={m} P={P} near={near} split={split}")
    ks = lk.kstride_for(S)
    kc, vc, qh = dev_h(K), dev_h(V), dev_h(Q)
    q8 = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
    qsc = torch.zeros(m, 32, device="cuda")
    qcs = torch.zeros(m, 32, device="cuda")
    k8 = torch.zeros(S * 512, dtype=torch.int8, device="cuda")
    ksc = torch.zeros(8 * ks + 4, device="cuda")
    lk.pf_q8(qh, m, None, q8, qsc, qcs)
    lk.pf_k8(kc, 0, S, None, ks, k8, ksc)
    o8 = torch.full((m, 2048), float("nan"), device="cuda")
    o16 = torch.full((m, 2048), float("nan"), device="cuda")
    if split == "pair":
        lk.pf_pair_override(1)
    else:
        lk.pf_split_override(split)
    try:
        lk.pf_attn8(q8, qsc, qcs, qh, m, P, k8, ksc, ks, kc, vc, near, sink, o8)
        lk.pf_attn(qh, m, P, kc, vc, o16)
        torch.cuda.synchronize()
    finally:
        lk.pf_split_override(0)
        lk.pf_pair_override(0)
    o8, o16 = host(o8), host(o16)
    assert np.isfinite(o8).all() and np.isfinite(o16).all()
    ref8 = oracle.pf_ref8(host(q8), host(qsc), host(qcs), Q, m, P, host(k8), host(ksc), ks, K, V, near, sink)
    ref = oracle.pf_ref(Q, m, P, K, V)
    r8, r16 = oracle.rel_err(o8, ref8), oracle.rel_err(o16, ref)
    note(f"  int8 kernel vs same-algorithm float64 rel {r8:.3e}; fp16 kernel vs float64 rel {r16:.3e}")
    assert r8 <= 2e-3 and r16 <= 2e-3


DEC_CASES = [("ramp", 2000), ("ramp", 33000), ("spike", 5000), ("jump", 5000), ("jump", 40000),
             ("step", 5000), ("step", 40000)]


@pytest.mark.parametrize("kind,seq", DEC_CASES, ids=[f"{c[0]}_seq{c[1]}" for c in DEC_CASES])
def test_decode_range(lk, oracle, kind, seq):
    rng = np.random.default_rng(seq)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    k = rng.standard_normal((seq, 8, 64)).astype(np.float32)
    v = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    q[:, 0] = 1.0
    if kind == "ramp":
        # +11.5 log2 units per 16-position tile, restarting every 4096 positions
        k[:, :, 0] = 4.0 * (np.arange(seq) % 4096)[:, None]
    elif kind == "spike":
        k[seq // 3, :, 0] = 240.0                                 # +43 log2 units
    elif kind == "step":
        k[seq // 2:, :, 0] += 50.0                                # +9 log2 units
    else:
        k[seq // 3, :, 0] = 1600.0                                # +290 log2 units
    kc = k.astype(np.float16)
    part = torch.full((lk.part_bytes() // 4,), float("nan"), device="cuda")
    out = torch.full((32, 64), float("nan"), device="cuda")
    note(f"decode softmax range {kind} seq={seq}")
    lk.attn_decode(dev(q), dev_h(kc.view(np.uint16)), dev_h(v.view(np.uint16)), d_pos_for(seq), part, out, None)
    torch.cuda.synchronize()
    ref = oracle.decode_ref(q, kc.view(np.uint16), v.view(np.uint16), seq)
    o = host(out)
    assert np.isfinite(o).all()
    rel = oracle.rel_err(o, ref)
    note(f"  split vs float64 rel {rel:.3e}")
    assert abs_err(o, ref) <= 1e-3 and rel <= 2e-3
