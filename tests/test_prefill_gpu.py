"""Prefill attention parity on the GPU, through the C ABI.

Mirrors the reference's prefill gates (tests/test_prefill.cu:244-364, 849-866):
the fp16 kernel against float64 causal attention at (m, P) = (64, 0),
(100, 150), (37, 1000) with its 4e-3 absolute bound (and the north-star 2e-3
relative bound); the int8 kernel on the lossless grid (within 1.01x of the fp16
kernel's error), with every tile exact and smoothing on (the q.c shift must
cancel), with mixed tiles and smoothing (2e-1), and -- stricter than the
reference, which only reports random-data int8 error -- against the float64
restatement of the same int8 algorithm (2e-3 relative) on every case.  The int8
quantisers, the K mean and the int32 Q.K^T sums are checked bit-exactly.
"""
import numpy as np
import pytest
import torch

from gpu_util import abs_err, dev, dev_h, host, host_h, note

pytestmark = pytest.mark.gpu

SEED = 12345


def _inputs(oracle, m, P, koff=0.0, with_off=False):
    K, V, Q = oracle.mt_prefill_case(SEED, m, P, koff, with_off)
    return K, V, Q


class _Dev:
    """Device copies of one case plus the int8 operands computed ON THE GPU."""

    def __init__(self, lk, K, V, Q, m, P, smooth):
        S = P + m
        self.m, self.P, self.S = m, P, S
        self.kstride = lk.kstride_for(S)
        self.kc, self.vc, self.qh = dev_h(K), dev_h(V), dev_h(Q)
        self.cm = torch.zeros(8, 64, device="cuda")
        if smooth:
            lk.pf_kmean(self.kc, S, self.cm)
        cm = self.cm if smooth else None
        self.q8 = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
        self.qsc = torch.zeros(m, 32, device="cuda")
        self.qcs = torch.zeros(m, 32, device="cuda")
        self.k8 = torch.zeros(S * 512, dtype=torch.int8, device="cuda")
        self.ksc = torch.zeros(8 * self.kstride + 4, device="cuda")
        lk.pf_q8(self.qh, m, cm, self.q8, self.qsc, self.qcs)
        lk.pf_k8(self.kc, 0, S, cm, self.kstride, self.k8, self.ksc)
        torch.cuda.synchronize()

    def attn8(self, lk, near, sink):
        o = torch.full((self.m, 2048), float("nan"), device="cuda")
        lk.pf_attn8(self.q8, self.qsc, self.qcs, self.qh, self.m, self.P, self.k8, self.ksc,
                    self.kstride, self.kc, self.vc, near, sink, o)
        torch.cuda.synchronize()
        return host(o)

    def attn16(self, lk):
        o = torch.full((self.m, 2048), float("nan"), device="cuda")
        lk.pf_attn(self.qh, self.m, self.P, self.kc, self.vc, o)
        torch.cuda.synchronize()
        return host(o)


# ---- bit-exact pieces ------------------------------------------------------------------
@pytest.mark.parametrize("smooth", [False, True])
def test_quantisers_bit_exact(lk, oracle, smooth):
    m, P = 100, 150
    K, V, Q = _inputs(oracle, m, P, 3.0, True)
    note(f"pf quantisers smooth={smooth}")
    d = _Dev(lk, K, V, Q, m, P, smooth)
    cm = oracle.pf_kmean(K, P + m) if smooth else None
    if smooth:
        assert np.array_equal(host(d.cm).view(np.uint32), cm.view(np.uint32))   # same order, same bits
    q8, qsc, qcs = oracle.pf_q8(Q, m, cm)
    assert np.array_equal(host(d.q8), q8)
    assert np.array_equal(host(d.qsc).view(np.uint32), qsc.view(np.uint32))
    assert np.array_equal(host(d.qcs).view(np.uint32), qcs.view(np.uint32))
    k8, ksc = oracle.pf_k8(K, 0, P + m, d.kstride, cm)
    assert np.array_equal(host(d.k8), k8)
    assert np.array_equal(host(d.ksc)[:8 * d.kstride].view(np.uint32), ksc.view(np.uint32))


def test_k8_incremental_range(lk, oracle):
    # the engine re-quantises only [lo, pos0 + m) (reference engine.cu:1077-1084)
    S, kstride = 300, 300
    rng = np.random.default_rng(31)
    K = (rng.standard_normal((S, 8, 64)) * 2).astype(np.float16).view(np.uint16)
    kc = dev_h(K)
    k8 = torch.full((S * 512,), 99, dtype=torch.int8, device="cuda")
    ksc = torch.full((8 * kstride,), -1.0, device="cuda")
    note("pf k8 incremental ranges")
    lk.pf_k8(kc, 0, 37, None, kstride, k8, ksc)
    lk.pf_k8(kc, 37, 37, None, kstride, k8, ksc)           # empty range: no-op
    lk.pf_k8(kc, 37, 211, None, kstride, k8, ksc)
    torch.cuda.synchronize()
    rk8, rksc = oracle.pf_k8(K, 0, 211, kstride)
    g8, gs = host(k8).reshape(S, 512), host(ksc).reshape(8, kstride)
    assert np.array_equal(g8[:211], rk8.reshape(S, 512)[:211])
    assert (g8[211:] == 99).all() and (gs[:, 211:] == -1.0).all()
    assert np.array_equal(gs[:, :211].view(np.uint32), rksc.reshape(8, kstride)[:, :211].view(np.uint32))


def test_qk_int32_bit_exact(lk, oracle):
    rng = np.random.default_rng(32)
    m, n = 48, 80
    q8 = rng.integers(-127, 128, (m, 2048)).astype(np.int8)
    k8 = rng.integers(-127, 128, (n, 8, 64)).astype(np.int8)
    # extreme sums: the kernel reads the MFMA result as the fp32 1.5 * 2^23 + sum,
    # exact while |sum| < 2^22; int8 operands reach at most 64 * 128 * 128 = 2^20
    k8[0, :, :] = -127; q8[0, :] = -127                        # +1032256 (quantiser range)
    k8[1, :, :] = -128; q8[1, :] = -128                        # +2^20, the int8 maximum
    q8[2, :] = 127                                             # 127 * -128 * 64 = -1040384
    k8[3, :, :] = 127; q8[3, :] = -128                         # -1040384 again, other operand
    k8[4, :, :] = 1                                            # sums near 0, both signs
    q8[4, :] = np.tile(np.array([1, -1], np.int8), 1024)
    s = torch.zeros(32, m, n, dtype=torch.int32, device="cuda")
    note("pf int32 QK^T")
    lk.pf_qk_i32(dev(q8), m, dev(k8), n, s)
    torch.cuda.synchronize()
    ref = oracle.qk_i32(q8, m, k8, n)
    assert ref.max() == 1 << 20 and ref.min() == -1040384     # the extremes are exercised
    got = host(s)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, (f"{len(bad)} sums differ, first {bad[:8].tolist()}: "
                           f"got {[int(got[tuple(i)]) for i in bad[:8]]} want {[int(ref[tuple(i)]) for i in bad[:8]]}")


# ---- fp16 kernel ---------------------------------------------------------------------------
@pytest.mark.parametrize("m,P", [(64, 0), (100, 150), (37, 1000), (1, 0), (1, 77), (130, 0), (200, 333)])
def test_attn_fp16(lk, oracle, m, P):
    K, V, Q = _inputs(oracle, m, P)
    note(f"pf attn fp16 m={m} P={P}")
    d = _Dev(lk, K, V, Q, m, P, False)
    o = d.attn16(lk)
    ref = oracle.pf_ref(Q, m, P, K, V)
    e, rel = abs_err(o, ref), oracle.rel_err(o, ref)
    note(f"  abs {e:.3e} rel {rel:.3e}")
    assert e < 4e-3 and rel <= 2e-3


def test_attn_first_row_is_v0(lk, oracle):
    m, P = 40, 0
    K, V, Q = _inputs(oracle, m, P)
    note("pf attn: query 0 sees only key 0")
    d = _Dev(lk, K, V, Q, m, P, False)
    v0 = np.repeat(oracle.h2f(V[:512]).reshape(8, 64), 4, axis=0).reshape(-1)
    assert np.array_equal(d.attn16(lk)[0], v0)
    # the int8 kernel's exponent is fma(x, sq, -m*sq): for x == m the rounding
    # residual of m*sq leaves p within an ulp or so of 1
    np.testing.assert_allclose(d.attn8(lk, 0, 0)[0], v0, rtol=1e-6, atol=0)


# ---- int8 kernel -----------------------------------------------------------------------------
CASES8 = [
    # (m, P, koff, smooth, near, gate) -- the reference's cases (test_prefill.cu:853-866)
    (64, 0, -1.0, False, 0, "lossless"),
    (100, 150, -1.0, False, 0, "lossless"),
    (100, 150, 3.0, True, 1 << 20, "allexact"),
    (37, 1000, 3.0, True, 1 << 20, "allexact"),
    (37, 1000, 3.0, True, 256, "mixed"),
    (100, 150, 0.0, False, 0, "info"),
    (37, 1000, 3.0, False, 0, "info"),
    (37, 1000, 3.0, True, 0, "info"),
    # wider: several 64-row blocks, mixed exact/int8 inside a block, sink on
    (300, 700, 0.0, False, 96, "info"),
    (129, 2000, 1.0, False, 1024, "info"),
]


@pytest.mark.parametrize("m,P,koff,smooth,near,gate", CASES8,
                         ids=[f"m{c[0]}_P{c[1]}_k{c[2]}_{'sm' if c[3] else 'ns'}_n{c[4]}" for c in CASES8])
def test_attn8(lk, oracle, m, P, koff, smooth, near, gate):
    K, V, Q = _inputs(oracle, m, P, koff, True)
    sink = int(near > 0)
    note(f"pf attn8 m={m} P={P} koff={koff} smooth={smooth} near={near}")
    d = _Dev(lk, K, V, Q, m, P, smooth)
    o8 = d.attn8(lk, near, sink)
    o16 = d.attn16(lk)
    ref = oracle.pf_ref(Q, m, P, K, V)
    e8, e16 = abs_err(o8, ref), abs_err(o16, ref)
    # the float64 restatement of the same int8 algorithm, on the GPU's int8 operands
    ref8 = oracle.pf_ref8(host(d.q8), host(d.qsc), host(d.qcs), Q, m, P, host(d.k8), host(d.ksc),
                          d.kstride, K, V, near, sink)
    rel8 = oracle.rel_err(o8, ref8)
    note(f"  int8 err {e8:.3e} (fp16 kernel {e16:.3e}); vs same-algorithm float64 rel {rel8:.3e}")
    assert rel8 <= 2e-3
    if gate in ("lossless", "allexact"):
        assert e8 <= e16 * 1.01 + 1e-6
    elif gate == "mixed":
        assert e8 < 2e-1


def test_attn8_deterministic(lk, oracle):
    m, P = 200, 500
    K, V, Q = _inputs(oracle, m, P, 1.0, True)
    d = _Dev(lk, K, V, Q, m, P, True)
    note("pf attn8 determinism")
    a = d.attn8(lk, 128, 1)
    for _ in range(3):
        assert np.array_equal(d.attn8(lk, 128, 1).view(np.uint32), a.view(np.uint32))


# ---- split-K work items (forced part sizes) --------------------------------------------------
SPLIT_CASES = [
    # (m, P, near, tiles per part)
    (300, 0, 96, 1),
    (300, 700, 96, 2),
    (129, 2000, 1024, 5),
    (500, 0, 0, 3),
    (64, 0, 0, 1),
]


@pytest.mark.parametrize("m,P,near,L", SPLIT_CASES, ids=[f"m{c[0]}_P{c[1]}_n{c[2]}_L{c[3]}" for c in SPLIT_CASES])
def test_attn_split_parts(lk, oracle, m, P, near, L):
    K, V, Q = _inputs(oracle, m, P, 1.0, True)
    sink = int(near > 0)
    note(f"pf split parts m={m} P={P} near={near} L={L}")
    d = _Dev(lk, K, V, Q, m, P, False)
    try:
        lk.pf_split_override(-1)
        whole8, whole16 = d.attn8(lk, near, sink), d.attn16(lk)
        lk.pf_split_override(L)
        part8, part16 = d.attn8(lk, near, sink), d.attn16(lk)
        again8 = d.attn8(lk, near, sink)
    finally:
        lk.pf_split_override(0)
    ref8 = oracle.pf_ref8(host(d.q8), host(d.qsc), host(d.qcs), Q, m, P, host(d.k8), host(d.ksc),
                          d.kstride, K, V, near, sink)
    ref = oracle.pf_ref(Q, m, P, K, V)
    r8, r16 = oracle.rel_err(part8, ref8), oracle.rel_err(part16, ref)
    d8, d16 = oracle.rel_err(part8, whole8), oracle.rel_err(part16, whole16)
    note(f"  split: int8 rel {r8:.3e}, fp16 rel {r16:.3e}; vs unsplit rel {d8:.3e} / {d16:.3e}")
    assert r8 <= 2e-3 and r16 <= 2e-3 and abs_err(part16, ref) <= 4e-3
    # parts round p against their own running max: same tolerance class as above
    assert d8 <= 1e-3 and d16 <= 1e-3
    assert np.array_equal(again8.view(np.uint32), part8.view(np.uint32))


# ---- paired workgroups (blocks i and nq-1-i in one 8-wave workgroup) ----------------------------
PAIR_CASES = [
    # (m, P, near): nq 2 (adjacent blocks); nq 3 ragged (the middle block alone);
    # nq 4 with P % 64 != 0 (the adjacent middle pair's later tiles all on one
    # group); nq 5 ragged; nq 8 deep; mixed exact/int8 tiles, sink on
    (128, 0, 0),
    (130, 0, 96),
    (256, 1, 96),
    (300, 37, 96),
    (500, 700, 1024),
    (129, 2000, 1024),
]


@pytest.mark.parametrize("m,P,near", PAIR_CASES, ids=[f"m{c[0]}_P{c[1]}_n{c[2]}" for c in PAIR_CASES])
def test_attn_pair(lk, oracle, m, P, near):
    """Paired launches, forced: both kernels against their float64 references
    and against the unpaired launch (bj's key range is cut in two parts and
    merged, so the same tolerance class as split parts), bit-identical on
    repeat, and the fused Q8_1 planes equal to quantising the float output."""
    K, V, Q = _inputs(oracle, m, P, 1.0, True)
    sink = int(near > 0)
    note(f"pf pair m={m} P={P} near={near}")
    d = _Dev(lk, K, V, Q, m, P, False)
    aqs = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
    asc = torch.zeros(m, 64, 2, device="cuda")
    try:
        lk.pf_pair_override(-1)
        whole8, whole16 = d.attn8(lk, near, sink), d.attn16(lk)
        lk.pf_pair_override(1)
        pair8, pair16 = d.attn8(lk, near, sink), d.attn16(lk)
        again8, again16 = d.attn8(lk, near, sink), d.attn16(lk)
        o = torch.full((m, 2048), float("nan"), device="cuda")
        lk.pf_attn_q81(d.qh, m, P, d.kc, d.vc, o, aqs, asc)
        torch.cuda.synchronize()
    finally:
        lk.pf_pair_override(0)
    ref8 = oracle.pf_ref8(host(d.q8), host(d.qsc), host(d.qcs), Q, m, P, host(d.k8), host(d.ksc),
                          d.kstride, K, V, near, sink)
    ref = oracle.pf_ref(Q, m, P, K, V)
    r8, r16 = oracle.rel_err(pair8, ref8), oracle.rel_err(pair16, ref)
    d8, d16 = oracle.rel_err(pair8, whole8), oracle.rel_err(pair16, whole16)
    note(f"  pair: int8 rel {r8:.3e}, fp16 rel {r16:.3e}; vs unpaired rel {d8:.3e} / {d16:.3e}")
    assert r8 <= 2e-3 and r16 <= 2e-3 and abs_err(pair16, ref) <= 4e-3
    assert d8 <= 1e-3 and d16 <= 1e-3
    assert np.isfinite(pair8).all() and np.isfinite(pair16).all()
    assert np.array_equal(again8.view(np.uint32), pair8.view(np.uint32))
    assert np.array_equal(again16.view(np.uint32), pair16.view(np.uint32))
    assert np.array_equal(host(o).view(np.uint32), pair16.view(np.uint32))
    qso, sco = oracle.pf_quant_rows(host(o), m, 2048, 64)
    assert np.array_equal(host(aqs), qso) and np.array_equal(host(asc).view(np.uint32), sco.view(np.uint32))


# ---- the rescale path: scores that climb past the running offset in every tile -----------------
RESCALE_CASES = [(600, 0, 96), (256, 300, 1024), (333, 100, 0)]


def _climbing_case(m, P, seed=7):
    """Keys along one direction u per kv head with a length growing by 1/8 per
    position, queries along the same u (length 2): the score q.k climbs by
    about 16 natural-log units (23 log2 units) per 64-key tile, so every tile
    raises some query's running max past the 2^15 limit of p and takes the
    rescale path; the softmax stays well conditioned (consecutive keys differ
    by 0.25 in score, so about four keys carry each row)."""
    rng = np.random.default_rng(seed)
    S = P + m
    u = rng.standard_normal((8, 64))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    beta = 0.5 + np.arange(S) * 0.125
    K = beta[:, None, None] * u[None] + 0.05 * rng.standard_normal((S, 8, 64))
    V = rng.standard_normal((S, 8, 64))
    Q = 2.0 * np.repeat(u, 4, axis=0)[None] + 0.05 * rng.standard_normal((m, 32, 64))
    f16 = lambda a: np.ascontiguousarray(a.astype(np.float16)).view(np.uint16).reshape(-1)
    return f16(K), f16(V), f16(Q)


@pytest.mark.parametrize("m,P,near", RESCALE_CASES, ids=[f"m{c[0]}_P{c[1]}_n{c[2]}" for c in RESCALE_CASES])
def test_attn_rescale_every_tile(lk, oracle, m, P, near):
    """The offset raise (a score more than 20 log2 units past the running
    offset) in every key tile, through the paired, unpaired and split
    launches: the fp16 kernel against float64, the int8 kernel against the
    float64 restatement of its algorithm, both within 2e-3 relative."""
    K, V, Q = _climbing_case(m, P)
    sink = int(near > 0)
    note(f"pf rescale every tile m={m} P={P} near={near}")
    d = _Dev(lk, K, V, Q, m, P, False)
    ref = oracle.pf_ref(Q, m, P, K, V)
    ref8 = oracle.pf_ref8(host(d.q8), host(d.qsc), host(d.qcs), Q, m, P, host(d.k8), host(d.ksc),
                          d.kstride, K, V, near, sink)
    forms = {}
    try:
        for name, pair, split in (("paired", 1, 0), ("unpaired", -1, 0), ("split", -1, 1)):
            lk.pf_pair_override(pair)
            lk.pf_split_override(split)
            forms[name] = (d.attn8(lk, near, sink), d.attn16(lk))
    finally:
        lk.pf_pair_override(0)
        lk.pf_split_override(0)
    for name, (o8, o16) in forms.items():
        r8, r16 = oracle.rel_err(o8, ref8), oracle.rel_err(o16, ref)
        note(f"  {name}: int8 rel {r8:.3e}, fp16 rel {r16:.3e}")
        assert np.isfinite(o8).all() and np.isfinite(o16).all(), name
        assert r8 <= 2e-3 and r16 <= 2e-3, name


# ---- the automatic (cost-model) split plan ------------------------------------------------------
AUTO_CASES = [(1000, 0, 256), (777, 0, 1024), (1500, 300, 96), (2048, 777, 1024), (4096, 4096, 1024),
              (512, 8000, 1024), (300, 20000, 256)]          # short chunks deep in a prompt: few blocks


@pytest.mark.parametrize("m,P,near", AUTO_CASES, ids=[f"m{c[0]}_P{c[1]}_n{c[2]}" for c in AUTO_CASES])
def test_attn_auto_split(lk, oracle, m, P, near):
    """Chunks the automatic plan cuts into parts (unequal key ranges, costliest
    first): the output matches the unsplit launch and, on sampled rows, the
    float64 restatement of the int8 algorithm; repeated launches are
    bit-identical."""
    assert any(it[3] >= 0 for it in lk.pf_plan_items(m, P, near, 1, True)), "the plan splits"
    K, V, Q = _inputs(oracle, m, P, 1.0, True)
    note(f"pf auto split m={m} P={P} near={near}")
    d = _Dev(lk, K, V, Q, m, P, False)
    auto8 = d.attn8(lk, near, 1)
    again8 = d.attn8(lk, near, 1)
    try:
        lk.pf_split_override(-1)
        whole8 = d.attn8(lk, near, 1)
    finally:
        lk.pf_split_override(0)
    assert np.array_equal(again8.view(np.uint32), auto8.view(np.uint32))
    dw = oracle.rel_err(auto8, whole8)
    rows = np.array(sorted({0, 1, 63, 64, 65, m // 2, m - 2, m - 1}), np.int32)
    ref8 = oracle.pf_ref8(host(d.q8), host(d.qsc), host(d.qcs), Q, m, P, host(d.k8), host(d.ksc),
                          d.kstride, K, V, near, 1, rows=rows)
    r8 = oracle.rel_err(auto8, ref8)
    note(f"  vs unsplit rel {dw:.3e}; rows {len(rows)} vs same-algorithm float64 rel {r8:.3e}")
    assert dw <= 1e-3 and r8 <= 2e-3
    assert np.isfinite(auto8).all()


# ---- BASELINE prefill configurations (sampled rows against the float64 oracle) -----------------
def _config_rows(m, long_ctx):
    if long_ctx:
        # every 64-row block edge, and the middle of the chunk
        rows = {r for b in range(0, m, 64) for r in (b, b + 63) if r < m} | {1023, 2048}
    else:
        # every 64-row block boundary (the kernel's query blocks, and so the
        # split-K parts' edges), the 32-row exactness tiles around the window
        # edge, and a seeded spread: 256+ rows in all
        rows = {r for b in range(0, m, 64) for r in (b, b + 63) if r < m}
        rows |= {1, 31, 32, 33, 65, 1000, 1023, 1024, 1025, 2047, 2048, m // 2 + 17, m - 2}
        rows |= set(np.random.default_rng(4).choice(m, 96, replace=False).tolist())
    return np.array(sorted(r for r in rows if r < m), np.int32)


def _config_check(lk, oracle, qh, kc, vc, P, m, near, sink, pure_rows=None):
    """The int8 kernel on chunk [P, P+m) of a prompt against the float64
    restatement of the same int8 algorithm (2e-3); with pure_rows, also the
    int8 kernel and the fp16 kernel against plain float64 attention on those
    rows (the reference reports this error for its int8 scoring,
    tests/test_prefill.cu:862-866), returned as (rel_rms, max_rel) pairs."""
    S = P + m
    kstride = lk.kstride_for(S)
    q8 = torch.empty(m, 2048, dtype=torch.int8, device="cuda")
    qsc = torch.empty(m, 32, device="cuda")
    qcs = torch.empty(m, 32, device="cuda")
    k8 = torch.empty(S * 512, dtype=torch.int8, device="cuda")
    ksc = torch.empty(8 * kstride + 4, device="cuda")
    qchunk = qh[P:P + m].contiguous()
    lk.pf_q8(qchunk, m, None, q8, qsc, qcs)
    lk.pf_k8(kc, 0, S, None, kstride, k8, ksc)
    o = torch.empty(m, 2048, device="cuda")
    lk.pf_attn8(q8, qsc, qcs, qchunk, m, P, k8, ksc, kstride, kc, vc, near, sink, o)
    torch.cuda.synchronize()
    rows = _config_rows(m, P > 0)
    Kh = host_h(kc[:S]).reshape(-1)
    Vh = host_h(vc[:S]).reshape(-1)
    Qh = host_h(qchunk)
    ref8 = oracle.pf_ref8(host(q8), host(qsc), host(qcs), Qh, m, P, host(k8), host(ksc),
                          kstride, Kh, Vh, near, sink, rows=rows)
    rel = oracle.rel_err(host(o), ref8)
    note(f"  rows {len(rows)}: rel vs same-algorithm float64 {rel:.3e}")
    assert rel <= 2e-3
    assert bool(torch.isfinite(o).all())
    if pure_rows is None:
        return None
    o16 = torch.empty(m, 2048, device="cuda")
    lk.pf_attn(qchunk, m, P, kc, vc, o16)
    torch.cuda.synchronize()
    pr = np.asarray(pure_rows, np.int32)
    ref = oracle.pf_ref(Qh, m, P, Kh, Vh, rows=pr)[pr]
    out = {}
    for name, got in (("int8", host(o)[pr]), ("fp16", host(o16)[pr])):
        e = got.astype(np.float64) - ref
        out[name] = (float(np.sqrt(np.mean(e * e)) / np.sqrt(np.mean(ref * ref))),
                     float(np.max(np.abs(e)) / np.max(np.abs(ref))))
    note(f"  vs plain float64 attention on {len(pr)} rows: int8 rel-RMS {out['int8'][0]:.3e} "
         f"max-rel {out['int8'][1]:.3e}; fp16 rel-RMS {out['fp16'][0]:.3e} max-rel {out['fp16'][1]:.3e}")
    return out


def test_config_c4(lk, oracle):
    import lk_configs
    note("prefill config C4 (m=4096, P=0, near 1024, sink)")
    qh, kc, vc, S = lk_configs.prefill_inputs("C4")
    _config_check(lk, oracle, qh, kc, vc, 0, S, 1024, 1)


# int8 against plain float64 on the sampled rows, measured on MI355X with the
# seeded splitmix64 inputs: (rel-RMS, max-rel) = (0.107, 1.14) at P = 65536 and
# (0.037, 0.29) at P = 126976.  Bounds sit 25% above, so a regression shows.
C5_INT8_BOUND = {65536: (0.135, 1.45), 126976: (0.046, 0.36)}


@pytest.mark.parametrize("P", [65536, 126976], ids=["mid_chunk", "last_chunk"])
def test_config_c5_chunk(lk, oracle, P):
    """C5 (heavy-tailed Q/K with x20 outlier channels, the stress case of the
    int8 scoring): a mid chunk and the last chunk against the same-algorithm
    restatement, and the int8 error against plain float64 attention -- an
    information figure in the reference (test_prefill.cu:862-866), bounded
    loosely here, beside the fp16 kernel's error (held to 2e-3)."""
    import lk_configs
    note(f"prefill config C5, 4096 chunk at P={P} (heavy-tailed Q/K)")
    qh, kc, vc, S = lk_configs.prefill_inputs("C5")
    err = _config_check(lk, oracle, qh, kc, vc, P, 4096, 1024, 1, pure_rows=[0, 1000, 2047, 3000, 4095])
    assert err["fp16"][1] <= 2e-3
    # The x20 channels set every row's absmax scale, so the other 62 channels
    # keep 1-3 int8 levels: this is the reference algorithm's own error on
    # outlier channels (the same-algorithm check above holds it to 2e-3).
    rms_max, rel_max = C5_INT8_BOUND[P]
    assert err["int8"][0] <= rms_max and err["int8"][1] <= rel_max


def test_config_c5_every_chunk(lk, oracle):
    """All 32 chunks of the C5 prompt as bench.py runs them (the int8 K copy
    extended chunk by chunk, Q quantised inside the attention kernel, the
    automatic launch choice: paired, split or unsplit), each checked on
    sampled rows against the float64 restatement of the same int8 algorithm
    (2e-3).  The rows move with the chunk: its first and last row, two 64-row
    block edges and one seeded row."""
    import lk_configs
    note("prefill config C5, all 32 chunks of 4096 (sampled rows)")
    qh, kc, vc, S = lk_configs.prefill_inputs("C5")
    m = 4096
    ks = lk.kstride_for(S)
    k8 = torch.empty(S * 512, dtype=torch.int8, device="cuda")
    ksc = torch.empty(8 * ks + 4, device="cuda")
    o = torch.empty(m, 2048, device="cuda")
    rng = np.random.default_rng(55)
    outs, rows_of = {}, {}
    for c, P in enumerate(range(0, S, m)):
        lk.pf_k8(kc, P, P + m, None, ks, k8, ksc)
        qchunk = qh[P:P + m].contiguous()
        lk.pf_attn8(None, None, None, qchunk, m, P, k8, ksc, ks, kc, vc, 1024, 1, o)
        b = 64 * ((c * 7) % 63)
        rows = np.array(sorted({0, b + 63, b + 64, int(rng.integers(0, m)), m - 1}), np.int32)
        rows_of[P] = rows
        outs[P] = host(o)[rows]
    torch.cuda.synchronize()
    Kh, Vh = host_h(kc).reshape(-1), host_h(vc).reshape(-1)
    K8, KSC = host(k8), host(ksc)
    Qall = host_h(qh)
    worst = 0.0
    for P, rows in rows_of.items():
        Qc = np.ascontiguousarray(Qall[P:P + m])
        q8, qsc, qcs = oracle.pf_q8(Qc, m)
        ref8 = oracle.pf_ref8(q8, qsc, qcs, Qc, m, P, K8, KSC, ks, Kh, Vh, 1024, 1, rows=rows)[rows]
        rel = oracle.rel_err(outs[P], ref8)
        worst = max(worst, rel)
        assert rel <= 2e-3, f"chunk at P={P}: rel {rel:.3e} on rows {rows.tolist()}"
    note(f"  worst chunk rel vs same-algorithm float64: {worst:.3e}")


# ---- planar Q8_1 of the attention output (reference k_pf_quant_rows) ----------------------------
def test_quant_rows_bit_exact(lk, oracle):
    rng = np.random.default_rng(81)
    rows, ld, kb = 37, 2048, 64
    X = (rng.standard_normal((rows, ld)) * rng.uniform(0.01, 5.0, (rows, 1))).astype(np.float32)
    X[3, 64:96] = 0.0
    note("pf quant_rows bit-exact")
    qs = torch.zeros(rows, kb * 32, dtype=torch.int8, device="cuda")
    sc = torch.zeros(rows, kb, 2, device="cuda")
    lk.pf_quant_rows(dev(X), rows, ld, kb, qs, sc)
    torch.cuda.synchronize()
    qso, sco = oracle.pf_quant_rows(X, rows, ld, kb)
    assert np.array_equal(host(qs), qso)
    assert np.array_equal(host(sc).view(np.uint32), sco.view(np.uint32))


@pytest.mark.parametrize("m,P,near,L,int8", [(300, 700, 96, -1, True), (300, 0, 96, 2, True),
                                             (129, 2000, 1024, 0, True), (300, 0, 0, 2, False)])
def test_attn_fused_q81_equals_quant_rows(lk, oracle, m, P, near, L, int8):
    K, V, Q = _inputs(oracle, m, P, 1.0, True)
    sink = int(near > 0)
    note(f"pf attn fused Q8_1 m={m} P={P} near={near} split={L} int8={int8}")
    d = _Dev(lk, K, V, Q, m, P, False)
    o = torch.full((m, 2048), float("nan"), device="cuda")
    aqs = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
    asc = torch.zeros(m, 64, 2, device="cuda")
    try:
        lk.pf_split_override(L)
        if int8:
            lk.pf_attn8_q81(d.q8, d.qsc, d.qcs, d.qh, m, P, d.k8, d.ksc, d.kstride, d.kc, d.vc, near, sink,
                            o, aqs, asc)
        else:
            lk.pf_attn_q81(d.qh, m, P, d.kc, d.vc, o, aqs, asc)
        # Q8_1 only (o = NULL) must give the same planes
        aqs2 = torch.zeros_like(aqs)
        asc2 = torch.zeros_like(asc)
        if int8:
            lk.pf_attn8_q81(d.q8, d.qsc, d.qcs, d.qh, m, P, d.k8, d.ksc, d.kstride, d.kc, d.vc, near, sink,
                            None, aqs2, asc2)
        else:
            lk.pf_attn_q81(d.qh, m, P, d.kc, d.vc, None, aqs2, asc2)
    finally:
        lk.pf_split_override(0)
    qs = torch.zeros_like(aqs)
    sc = torch.zeros_like(asc)
    lk.pf_quant_rows(o, m, 2048, 64, qs, sc)
    torch.cuda.synchronize()
    assert torch.equal(aqs, qs) and torch.equal(asc.view(torch.int32), sc.view(torch.int32))
    assert torch.equal(aqs2, aqs) and torch.equal(asc2.view(torch.int32), asc.view(torch.int32))
    qso, sco = oracle.pf_quant_rows(host(o), m, 2048, 64)
    assert np.array_equal(host(aqs), qso) and np.array_equal(host(asc).view(np.uint32), sco.view(np.uint32))


# ---- Q quantised inside the attention kernel (q8 = qsc = qcs = NULL) ------------------------------
INQ_CASES = [(4096, 0, 1024, 0), (300, 700, 96, -1), (300, 0, 96, 2), (129, 2000, 1024, 0),
             (200, 333, 0, 0), (64, 0, 1024, 0), (513, 64, 1024, 0), (1, 77, 96, 0)]


@pytest.mark.parametrize("m,P,near,L", INQ_CASES, ids=[f"m{c[0]}_P{c[1]}_n{c[2]}_L{c[3]}" for c in INQ_CASES])
@pytest.mark.parametrize("pair", [0, -1, 1], ids=["auto", "unpaired", "paired"])
def test_attn8_in_kernel_q8_is_bit_identical(lk, oracle, m, P, near, L, pair):
    """lk_pf_attn8 with q8/qsc/qcs NULL quantises Q from the fp16 block it
    stages anyway (lk_pf_q8's arithmetic, no smoothing): outputs and the fused
    Q8_1 planes equal the two-kernel path's bit for bit, whatever the launch
    form (paired, unpaired, split)."""
    K, V, Q = _inputs(oracle, m, P, 1.0, True)
    sink = int(near > 0)
    note(f"pf attn8 in-kernel q8 m={m} P={P} near={near} split={L} pair={pair}")
    d = _Dev(lk, K, V, Q, m, P, False)
    outs = []
    try:
        lk.pf_split_override(L)
        lk.pf_pair_override(pair)
        for q8, qsc in ((d.q8, d.qsc), (None, None)):
            o = torch.full((m, 2048), float("nan"), device="cuda")
            aqs = torch.zeros(m, 2048, dtype=torch.int8, device="cuda")
            asc = torch.zeros(m, 64, 2, device="cuda")
            lk.pf_attn8(q8, qsc, None if q8 is None else d.qcs, d.qh, m, P, d.k8, d.ksc, d.kstride,
                        d.kc, d.vc, near, sink, o)
            lk.pf_attn8_q81(q8, qsc, None if q8 is None else d.qcs, d.qh, m, P, d.k8, d.ksc, d.kstride,
                            d.kc, d.vc, near, sink, None, aqs, asc)
            torch.cuda.synchronize()
            outs.append((host(o), host(aqs), host(asc)))
    finally:
        lk.pf_split_override(0)
        lk.pf_pair_override(0)
    (o1, a1, s1), (o2, a2, s2) = outs
    assert np.isfinite(o2).all()
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(a1, a2) and np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_attn8_in_kernel_q8_argument_rules(lk):
    """q8 and qsc go together; without them qcs (smoothing) must be NULL."""
    import ctypes
    lib = lk.load()
    p = ctypes.c_void_p(0x1000)
    assert lib.lk_pf_attn8(None, p, None, p, 4, 0, p, p, 4, p, p, 0, 0, p, None) == 1
    assert lib.lk_pf_attn8(p, None, None, p, 4, 0, p, p, 4, p, p, 0, 0, p, None) == 1
    assert lib.lk_pf_attn8(None, None, p, p, 4, 0, p, p, 4, p, p, 0, 0, p, None) == 1
    assert b"qcs" in lib.lk_last_error()


# ---- the shared split-K partial buffer: one stream at a time ----------------------------------
def test_split_scratch_refuses_a_second_stream_while_pending(lk, oracle):
    """Split launches share the library's partial buffer on a device.  A split
    launch on stream B while one on stream A is still pending is refused with
    hipErrorNotReady (600) and a message; once A has completed, B is accepted;
    launches ordered on one stream are always accepted.  A's result is intact."""
    m, P = 1024, 0
    K, V, Q = _inputs(oracle, m, P)
    d = _Dev(lk, K, V, Q, m, P, False)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    oa = torch.full((m, 2048), float("nan"), device="cuda")
    ob = torch.full((m, 2048), float("nan"), device="cuda")
    note("pf split scratch guard: two streams")
    try:
        lk.pf_split_override(2)                     # this chunk splits
        with torch.cuda.stream(sa):
            torch.cuda._sleep(200_000_000)          # keep stream A busy (about 0.1 s)
        lk.pf_attn(d.qh, m, P, d.kc, d.vc, oa, stream=sa)
        lk.pf_attn(d.qh, m, P, d.kc, d.vc, oa, stream=sa)          # same stream: accepted
        with pytest.raises(lk.LkError) as ei:
            lk.pf_attn(d.qh, m, P, d.kc, d.vc, ob, stream=sb)
        assert "hipError 600" in str(ei.value) and "another stream" in str(ei.value)
        sa.synchronize()
        lk.pf_attn(d.qh, m, P, d.kc, d.vc, ob, stream=sb)          # A is done: accepted
        sb.synchronize()
    finally:
        lk.pf_split_override(0)
    assert np.array_equal(host(oa).view(np.uint32), host(ob).view(np.uint32))
    assert oracle.rel_err(host(oa), oracle.pf_ref(Q, m, P, K, V)) <= 2e-3
