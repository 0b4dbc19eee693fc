"""Pins of the CPU oracle (oracle/lk_oracle.cpp) -- CPU only.

The reference holds no attention golden vectors (its attention tests are
seeded-random float64 comparisons), so each oracle function is pinned against
something that is not itself: a library routine (numpy's IEEE fp16 conversion,
torch's float64 scaled_dot_product_attention, numpy integer matmul), a closed
form (seq = 1, constant keys, the lossless int8 grid the reference's own
test_attn8 relies on, tie-breaking of the two rounding rules), numbers printed
in the reference's sources, or a published test vector.  Each check is chosen
so that a plausible slip (wrong rounding rule, dropped scale, transposed
operand, wrong GQA head mapping, off-by-one tile boundary) fails it.
"""
import math

import numpy as np
import pytest
import torch


# ---- fp16 conversions -----------------------------------------------------------
def test_h2f_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = oracle.h2f(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_matches_numpy_rne(oracle):
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
        # exact ties between neighbouring halves (normal and subnormal), overflow edge
        (np.arange(1, 4000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        (np.arange(0, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        np.array([65504, 65519.99, 65520, 70000, -65520, 6.1e-5, 5.96e-8, 2.98e-8,
                  2.99e-8, 0.0, -0.0, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = oracle.f2h(x)
    assert np.array_equal(got, ref)


# ---- split-K slice rule -------------------------------------------------------------
@pytest.mark.parametrize("seq,ns,chunk", [
    # the reference operating point SPLIT=128, TARGET_N=64, SPLIT_MIN=8 and the
    # chunk sizes its sources state (test_attn.cu:224-228, kernels.cuh:623-625)
    (16384, 128, 128), (32768, 128, 256), (65536, 128, 512), (100003, 128, 782),
    (131072, 128, 1024), (4096, 64, 64), (8192, 128, 64), (1, 8, 1), (5, 8, 1),
])
def test_slice_rule_reference_points(oracle, seq, ns, chunk):
    assert oracle.attn_slices(seq, 128, 64, 8) == (ns, chunk)


def test_slice_rule_covers_sequence(oracle):
    for cap, tn, mn in [(128, 64, 8), (256, 128, 8), (512, 256, 16)]:
        for seq in [1, 2, 7, 63, 64, 65, 511, 4097, 32768, 100003, 131072]:
            ns, ch = oracle.attn_slices(seq, cap, tn, mn)
            assert mn <= ns <= cap and ch * ns >= seq and ch * (ns - 1) < seq or ns == mn
            nv = -(-seq // ch)
            assert nv <= ns and (nv - 1) * ch < seq <= nv * ch


# ---- decode float64 reference ----------------------------------------------------------
def _rand_kv(rng, seq):
    k = rng.uniform(-1, 1, (seq, 8, 64)).astype(np.float16)
    v = rng.uniform(-1, 1, (seq, 8, 64)).astype(np.float16)
    return k, v


def test_decode_ref_seq1_is_v(oracle):
    rng = np.random.default_rng(1)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    k, v = _rand_kv(rng, 1)
    out = oracle.decode_ref(q, k.view(np.uint16), v.view(np.uint16), 1)
    want = np.repeat(v[0].astype(np.float64), 4, axis=0)       # head h uses kv h // 4
    assert np.array_equal(out, want)


def test_decode_ref_constant_keys_average_v(oracle):
    rng = np.random.default_rng(2)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    seq = 37
    k = np.broadcast_to(rng.uniform(-1, 1, (1, 8, 64)), (seq, 8, 64)).astype(np.float16)
    v = rng.uniform(-1, 1, (seq, 8, 64)).astype(np.float16)
    out = oracle.decode_ref(q, np.ascontiguousarray(k).view(np.uint16), v.view(np.uint16), seq)
    want = np.repeat(v.astype(np.float64).mean(0), 4, axis=0)
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-14)


def test_decode_ref_matches_torch_sdpa(oracle):
    rng = np.random.default_rng(3)
    seq = 301
    q = (rng.standard_normal((32, 64)) * 1.5).astype(np.float32)
    k, v = _rand_kv(rng, seq)
    out = oracle.decode_ref(q, k.view(np.uint16), v.view(np.uint16), seq)
    qt = torch.from_numpy(q.astype(np.float64)).view(1, 32, 1, 64)
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).repeat_interleave(4, 0)[None]
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).repeat_interleave(4, 0)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=0.125)
    np.testing.assert_allclose(out, ref.view(32, 64).numpy(), rtol=0, atol=1e-13)


# ---- Q8_1 (combine epilogue) ---------------------------------------------------------------
def _unpack_q8_1(y):
    d = np.frombuffer(y[:2].tobytes(), np.float16)[0]
    s = np.frombuffer(y[2:4].tobytes(), np.float16)[0]
    return float(d), float(s), y[4:].view(np.int8).copy()


def test_q8_1_zero_block(oracle):
    d, s, q = _unpack_q8_1(oracle.quantize_q8_1(np.zeros(32, np.float32)))
    assert d == 0.0 and s == 0.0 and not q.any()


def test_q8_1_integer_grid_and_sum(oracle):
    rng = np.random.default_rng(4)
    k = rng.integers(-127, 128, 32)
    k[5] = -127                       # |max| = 127 -> d = 1 exactly
    d, s, q = _unpack_q8_1(oracle.quantize_q8_1(k.astype(np.float32)))
    assert d == float(np.float16(np.float32(127.0) / np.float32(127.0)))
    assert np.array_equal(q, k.astype(np.int8))
    assert s == float(np.float16(k.sum()))      # small integers: the sum is exact in any order


def test_q8_1_rounds_half_away_from_zero(oracle):
    # am = 127 -> d = 1, so q = roundf(x): halves go AWAY from zero (roundf),
    # unlike the prefill quantiser's round-to-nearest-even.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [0.5, 1.5, 2.5, -0.5, -2.5, 126.5]
    _, _, q = _unpack_q8_1(oracle.quantize_q8_1(x))
    assert list(q[:7]) == [127, 1, 2, 3, -1, -3, 127]


def test_q8_1_error_bound(oracle):
    rng = np.random.default_rng(5)
    for _ in range(200):
        x = (rng.standard_normal(32) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
        d, s, q = _unpack_q8_1(oracle.quantize_q8_1(x))
        dd = np.float32(np.abs(x).max()) / np.float32(127.0)
        assert np.all(np.abs(q.astype(np.int32)) <= 127)
        assert np.all(np.abs(x - q * dd) <= dd * (0.5 + 1e-5))
        assert abs(s - x.astype(np.float64).sum()) <= 1e-3 * (abs(x).sum() + 1)


# ---- prefill int8 quantiser ------------------------------------------------------------------
def test_q8_row_lossless_grid(oracle):
    # reference test_prefill.cu:301-309: integers with |max| = 127 times a power
    # of two quantise losslessly.
    rng = np.random.default_rng(6)
    for j in range(-12, 6):
        k = rng.integers(-127, 128, 64)
        k[0] = 127
        v = (k * 2.0 ** j).astype(np.float32)
        q, sc = oracle.q8_row(v, mul=1.0)
        assert np.array_equal(q, k.astype(np.int8))
        assert sc == np.float32(np.float32(127 * 2.0 ** j) / np.float32(127.0))


def test_q8_row_ties_to_even(oracle):
    v = np.zeros(64, np.float32)
    v[0] = 127.0                                   # id = 1 exactly
    v[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 125.5, 126.5]
    q, sc = oracle.q8_row(v, mul=2.0)
    assert list(q[:9]) == [127, 0, 2, 2, 0, -2, -2, 126, 126]
    assert sc == np.float32(2.0)


def test_q8_row_zero_and_bound(oracle):
    q, sc = oracle.q8_row(np.zeros(64, np.float32))
    assert not q.any() and sc == 0.0
    rng = np.random.default_rng(8)
    for _ in range(300):
        v = (rng.standard_t(4, 64) * 10.0 ** rng.uniform(-4, 3)).astype(np.float32)
        q, sc = oracle.q8_row(v)
        assert np.abs(q.astype(np.int32)).max() == 127          # the max element maps to +-127
        assert np.all(np.abs(v - q * sc) <= sc * 0.5 * (1 + 1e-5))


def test_pf_q8_layout_and_scales(oracle):
    rng = np.random.default_rng(9)
    m = 3
    qh = (rng.standard_normal((m, 2048)) * 0.2).astype(np.float16)
    cm = rng.standard_normal((8, 64)).astype(np.float32)
    q8, qsc, qcs = oracle.pf_q8(qh.view(np.uint16), m, cm)
    q8n, qscn, qcsn = oracle.pf_q8(qh.view(np.uint16), m, None)
    assert np.array_equal(q8, q8n) and np.array_equal(qsc, qscn) and not qcsn.any()
    l2e = np.float32(1.4426950408889634)
    for t in range(m):
        for h in range(32):
            row = qh[t, h * 64:(h + 1) * 64].astype(np.float32)
            q, sc = oracle.q8_row(row, mul=float(l2e))
            assert np.array_equal(q8[t, h * 64:(h + 1) * 64], q) and qsc[t, h] == sc
            want = row.astype(np.float64) @ cm[h // 4].astype(np.float64) * float(l2e)
            assert abs(qcs[t, h] - want) <= 1e-5 * (1 + abs(want))


def _warp_qc_reference_order(row, c):
    """q.c as the reference's k_pf_q8 computes it (prefill.cu:1279-1284),
    simulated lane by lane in float32: lane l holds values 2l and 2l+1, forms
    v[2l]*c[2l] + v[2l+1]*c[2l+1], then __shfl_xor_sync with offsets 16..1."""
    f = np.float32
    s = [f(f(row[2 * l] * c[2 * l]) + f(row[2 * l + 1] * c[2 * l + 1])) for l in range(32)]
    o = 16
    while o:
        s = [f(s[l] + s[l ^ o]) for l in range(32)]
        o >>= 1
    return s[0]


def _other_order_qc(row, c):
    """The same sum in a different, plausible order (value strides 32 .. 1)."""
    f = np.float32
    s = [f(row[i] * c[i]) for i in range(64)]
    o = 32
    while o:
        s = [f(s[i] + s[i ^ o]) for i in range(64)]
        o >>= 1
    return s[0]


def test_pf_q8_qc_reference_order(oracle):
    """qcs bit for bit against a lane-level simulation of the reference warp's
    reduction; and the simulation tells the orders apart on these inputs (so
    a kernel or oracle in another order would fail this test)."""
    rng = np.random.default_rng(19)
    m = 4
    qh = (rng.standard_normal((m, 2048)) * 0.7).astype(np.float16)
    cm = rng.standard_normal((8, 64)).astype(np.float32)
    _, _, qcs = oracle.pf_q8(qh.view(np.uint16), m, cm)
    l2e = np.float32(1.4426950408889634)
    differ = 0
    for t in range(m):
        for h in range(32):
            row = qh[t, h * 64:(h + 1) * 64].astype(np.float32)
            want = _warp_qc_reference_order(row, cm[h // 4])
            assert qcs[t, h].view(np.uint32) == np.float32(want * l2e).view(np.uint32), (t, h)
            differ += _other_order_qc(row, cm[h // 4]) != want
    assert differ > 0


def test_pf_k8_layout_and_smoothing(oracle):
    rng = np.random.default_rng(10)
    S, kstride = 13, 16
    kc = (rng.standard_normal((S, 8, 64)) * 1.5).astype(np.float16)
    cm = rng.standard_normal((8, 64)).astype(np.float32) * 0.3
    k8, ksc = oracle.pf_k8(kc.view(np.uint16), 3, 11, kstride, cm)
    k8 = k8.reshape(S, 8, 64)
    ksc = ksc.reshape(8, kstride)
    assert not k8[:3].any() and not k8[11:].any() and not ksc[:, :3].any() and not ksc[:, 11:].any()
    for p in range(3, 11):
        for h in range(8):
            q, sc = oracle.q8_row(kc[p, h].astype(np.float32) - cm[h])
            assert np.array_equal(k8[p, h], q) and ksc[h, p] == sc


def test_pf_kmean(oracle):
    rng = np.random.default_rng(11)
    n = 512
    # small integers: every fp32 partial sum is exact, and n is a power of two,
    # so the mean is exact whatever the summation order
    kc = rng.integers(-40, 41, (n, 8, 64)).astype(np.float16)
    cm = oracle.pf_kmean(kc.view(np.uint16), n)
    assert np.array_equal(cm, kc.astype(np.float64).mean(0).astype(np.float32))
    kc2 = rng.standard_normal((1000, 8, 64)).astype(np.float16)
    cm2 = oracle.pf_kmean(kc2.view(np.uint16), 777)
    np.testing.assert_allclose(cm2, kc2[:777].astype(np.float64).mean(0), rtol=0, atol=1e-6)


# ---- exact-tile predicate -------------------------------------------------------------------
def test_exact_tile_predicate(oracle):
    # near covering the context: every tile exact (test_prefill.cu:857-858)
    for P, m in [(150, 100), (1000, 37)]:
        for qt in range((m + 31) // 32):
            for kt in range((P + m + 63) // 64):
                assert oracle.pf_exact(P, qt, kt, 1 << 20, 1)
    # near = 0, no sink: exact iff the tile ends after the 32-query tile's first
    # position, i.e. exactly the tiles that touch the diagonal region
    P = 1000
    for qt in range(2):
        first = P + 32 * qt
        for kt in range(20):
            assert oracle.pf_exact(P, qt, kt, 0, 0) == (64 * kt + 63 >= first)
    # sink keeps tile 0 exact; near widens the window by exactly `near` keys
    assert oracle.pf_exact(4096, 5, 0, 0, 1) and not oracle.pf_exact(4096, 5, 0, 0, 0)
    P, qt, near = 8192, 3, 1024
    lo = P + 32 * qt - near
    for kt in range(200):
        assert oracle.pf_exact(P, qt, kt, near, 0) == (64 * kt + 64 > lo)


# ---- prefill references -----------------------------------------------------------------------
def _torch_causal(qh, kc, vc, m, P):
    q = torch.from_numpy(qh.astype(np.float64)).view(m, 32, 64).permute(1, 0, 2)[None]
    S = P + m
    k = torch.from_numpy(kc.astype(np.float64)).view(S, 8, 64).permute(1, 0, 2).repeat_interleave(4, 0)[None]
    v = torch.from_numpy(vc.astype(np.float64)).view(S, 8, 64).permute(1, 0, 2).repeat_interleave(4, 0)[None]
    mask = torch.arange(S)[None, :] <= (P + torch.arange(m))[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=1.0)
    return o[0].permute(1, 0, 2).reshape(m, 2048).numpy()


@pytest.mark.parametrize("m,P", [(5, 0), (37, 20), (64, 70)])
def test_pf_ref_matches_torch_sdpa(oracle, m, P):
    K, V, Q = oracle.mt_prefill_case(12345, m, P)
    o = oracle.pf_ref(Q, m, P, K, V)
    ref = _torch_causal(Q.view(np.float16), K.view(np.float16), V.view(np.float16), m, P)
    np.testing.assert_allclose(o, ref, rtol=0, atol=1e-12)


def _ref8_inputs(oracle, m, P, koff, with_off, smooth):
    K, V, Q = oracle.mt_prefill_case(12345, m, P, koff, with_off)
    S = P + m
    kstride = (S + 3) & ~3
    cm = oracle.pf_kmean(K, S) if smooth else None
    q8, qsc, qcs = oracle.pf_q8(Q, m, cm)
    k8, ksc = oracle.pf_k8(K, 0, S, kstride, cm)
    return K, V, Q, q8, qsc, qcs, k8, ksc, kstride


def test_pf_ref8_all_exact_equals_pf_ref(oracle):
    m, P = 40, 90
    K, V, Q, q8, qsc, qcs, k8, ksc, ks = _ref8_inputs(oracle, m, P, 3.0, True, True)
    o8 = oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8, ksc, ks, K, V, 1 << 20, 1)
    o = oracle.pf_ref(Q, m, P, K, V)
    # the q.c shift cancels; what remains is the fp32 log2(e) constant
    # (1.3e-8 relative) scaling the scores
    np.testing.assert_allclose(o8, o, rtol=0, atol=1e-6)


def test_pf_ref8_lossless_grid_int8_equals_exact(oracle):
    # lossless int8 grid (test_prefill.cu:301-309): every int8 tile scores exactly
    # what the fp16 tile would, so near = 0 must reproduce pf_ref.
    m, P = 50, 100
    K, V, Q, q8, qsc, qcs, k8, ksc, ks = _ref8_inputs(oracle, m, P, -1.0, True, False)
    o8 = oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8, ksc, ks, K, V, 0, 0)
    o = oracle.pf_ref(Q, m, P, K, V)
    np.testing.assert_allclose(o8, o, rtol=0, atol=1e-6)


def test_pf_ref8_int8_tiles_really_use_int8(oracle):
    # On random data the int8 tiles must differ from exact scoring (else the
    # classification is not being applied), and the tile-0 sink must matter.
    m, P = 32, 320
    K, V, Q, q8, qsc, qcs, k8, ksc, ks = _ref8_inputs(oracle, m, P, 0.0, True, False)
    o = oracle.pf_ref(Q, m, P, K, V)
    e_int8 = np.abs(oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8, ksc, ks, K, V, 0, 0) - o).max()
    e_sink = np.abs(oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8, ksc, ks, K, V, 0, 1) - o).max()
    e_all = np.abs(oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8, ksc, ks, K, V, 1 << 20, 0) - o).max()
    assert e_all < 1e-6 and e_int8 > 1e-4 and e_sink > 0 and e_sink != e_int8


def test_pf_ref8_int8_tile_formula(oracle):
    # one query, one key, int8 tile: s = sumi * ksc * qsc, a one-key softmax
    # returns V exactly; two keys give the closed-form two-way softmax.
    m, P = 1, 1
    K, V, Q, q8, qsc, qcs, k8, ksc, ks = _ref8_inputs(oracle, m, P, 0.0, True, False)
    o = oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8, ksc, ks, K, V, -1000, 0)   # no exact tiles
    Kq = k8.reshape(2, 8, 64).astype(np.int64)
    Vf = V.view(np.float16).reshape(2, 8, 64).astype(np.float64)
    for h in range(32):
        s = [float((q8[0, h * 64:(h + 1) * 64].astype(np.int64) * Kq[j, h // 4]).sum())
             * float(ksc[(h // 4) * ks + j]) * float(qsc[0, h]) for j in range(2)]
        w = np.exp2(np.array(s) - max(s))
        want = (w[:, None] * Vf[:, h // 4]).sum(0) / w.sum()
        np.testing.assert_allclose(o[0, h * 64:(h + 1) * 64], want, rtol=0, atol=1e-12)


def test_qk_i32_matches_integer_matmul(oracle):
    rng = np.random.default_rng(12)
    m, n = 16, 32
    q8 = rng.integers(-127, 128, (m, 2048)).astype(np.int8)
    k8 = rng.integers(-127, 128, (n, 8, 64)).astype(np.int8)
    s = oracle.qk_i32(q8, m, k8, n)
    qv = q8.reshape(m, 32, 64).astype(np.int64)
    kv = np.repeat(k8.astype(np.int64), 4, axis=1)           # head h -> kv h // 4
    want = np.einsum("ihd,jhd->hij", qv, kv)
    assert np.array_equal(s, want.astype(np.int32))


# ---- generators ---------------------------------------------------------------------------------
def test_xorshift_generator_matches_definition(oracle):
    # test_attn.cu:35-40: xorshift64 (13, 7, 17), top 53 bits / 2^53, then *2-1
    gen = oracle.XorShiftAttnCases()
    q, kc, vc = gen.next_case(cache_elems=4)
    s = oracle.XorShiftAttnCases.SEED
    M = (1 << 64) - 1

    def nxt(s):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        return s
    vals = []
    for _ in range(2048 + 8):
        s = nxt(s)
        vals.append(((s >> 11) & ((1 << 53) - 1)) / float(1 << 53) * 2.0 - 1.0)
    assert np.array_equal(q, (np.array(vals[:2048], np.float32) * np.float32(1.5)))
    kv = np.array(vals[2048:], np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(kc, kv[0::2]) and np.array_equal(vc, kv[1::2])
    assert gen.state.value == s


def test_splitmix_normal_stats(oracle):
    x = oracle.sm_normal(42, 400000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    u = oracle.sm_uniform(43, 200000, 0.5, 2.0)
    assert u.min() >= 0.5 and u.max() <= 2.0 and abs(u.mean() - 1.25) < 0.01
    t = oracle.sm_student4(44, 200000).astype(np.float64)
    # Student-t(4): median |x| = 0.7407
    assert abs(np.median(np.abs(t)) - 0.7407) < 0.01


def test_splitmix64_known_answers(oracle):
    """The integer stream the benchmark configurations are drawn from is
    splitmix64; its published test vector (seed 1234567, S. Vigna's
    splitmix64.c) pins the oracle's generator and the configs' host copy."""
    import lk_configs
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert oracle.sm64(1234567, 5).tolist() == want
    assert lk_configs.sm64_draws(1234567, 5) == want
    seed = lk_configs.seed_of("C5", 0, lk_configs.T_CHAN, 2)
    assert oracle.sm64(seed, 64).tolist() == lk_configs.sm64_draws(seed, 64)


def test_splitmix_box_muller_composition(oracle):
    """The normal, uniform and Student-t streams are built from the pinned
    integer stream exactly as documented: u = ((x >> 11) + 1) / 2^53, pair j of
    the normals from draws 2j+1, 2j+2 (r = sqrt(-2 ln u1); cos, then sin), the
    uniform from draw i+1, the Student-t element from draws 10i+1 .. 10i+10."""
    seed, n = 987654321, 1001
    x = oracle.sm64(seed, 10 * n + 2)
    u = ((x >> np.uint64(11)).astype(np.float64) + 1.0) / 9007199254740992.0
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    th = 2.0 * np.pi * u[1::2]
    want = np.empty(2 * len(th), np.float32)
    want[0::2] = (r * np.cos(th)).astype(np.float32)
    want[1::2] = (r * np.sin(th)).astype(np.float32)
    got = oracle.sm_normal(seed, n)
    assert np.mean(got == want[:n]) > 0.9999 and np.allclose(got, want[:n], rtol=1e-6, atol=1e-7)
    lo, hi = np.float32(0.5), np.float32(2.0)
    wu = lo + (hi - lo) * u[:n].astype(np.float32)
    assert np.array_equal(oracle.sm_uniform(seed, n, 0.5, 2.0), wu)
    g = np.sqrt(-2.0 * np.log(u[0:10 * n:2])) * np.cos(2.0 * np.pi * u[1:10 * n:2])
    g = g.reshape(n, 5)
    wt = (g[:, 0] / np.sqrt((g[:, 1] ** 2 + g[:, 2] ** 2 + g[:, 3] ** 2 + g[:, 4] ** 2) / 4.0)).astype(np.float32)
    gt = oracle.sm_student4(seed, n)
    assert np.mean(gt == wt) > 0.999 and np.allclose(gt, wt, rtol=1e-6, atol=1e-7)


def test_rel_err_metric(oracle):
    a = np.array([1.0, 2.0, 3.5])
    b = np.array([1.0, 2.0, 4.0])
    assert oracle.rel_err(a, b) == pytest.approx(0.5 / 4.0)


# ---- attention-input producers (kernels.cu:871-915, prefill.cu:975-1016) -------------------------
def _textbook_norm_rope(v, w, pos):
    """Independent float64 statement: RMS norm then NEOX rotation (first half
    paired with second half), theta 1e7, eps 1e-5."""
    v = v.astype(np.float64)
    y = v / np.sqrt(np.mean(v * v) + 1e-5) * w.astype(np.float64)
    i = np.arange(32, dtype=np.float64)
    ang = pos * 10000000.0 ** (-i / 32.0)
    c, s = np.cos(ang), np.sin(ang)
    return np.concatenate([y[:32] * c - y[32:] * s, y[:32] * s + y[32:] * c])


@pytest.mark.parametrize("pos", [0, 1, 7, 300])
def test_norm_rope_row_matches_textbook(oracle, pos):
    rng = np.random.default_rng(100 + pos)
    for _ in range(20):
        v = (rng.standard_normal(64) * rng.uniform(0.1, 30.0)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
        got = oracle.norm_rope_row(v, w, pos).astype(np.float64)
        want = _textbook_norm_rope(v, w, pos)
        # fp32 rounding of the steps, plus the fp32 angle (pos * f rounded)
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) <= 2e-6 + pos * 1.2e-7


def test_norm_rope_row_position_zero_is_pure_norm(oracle):
    rng = np.random.default_rng(7)
    v = rng.standard_normal(64).astype(np.float32)
    w = np.ones(64, np.float32)
    got = oracle.norm_rope_row(v, w, 0)
    y = v.astype(np.float64) / np.sqrt(np.mean(v.astype(np.float64) ** 2) + 1e-5)
    assert np.max(np.abs(got - y)) <= 4e-7 * np.max(np.abs(y))
    assert abs(np.mean(got.astype(np.float64) ** 2) - 1.0) < 1e-5 + 1e-5   # unit RMS (eps aside)


def test_norm_rope_row_rotation_keeps_pair_norms(oracle):
    # at a large position the angles are large, but each (i, i+32) pair is
    # only rotated: its norm equals the norm-only pair
    rng = np.random.default_rng(8)
    v = rng.standard_normal(64).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    y = oracle.norm_rope_row(v, w, 0).astype(np.float64)
    r = oracle.norm_rope_row(v, w, 131071).astype(np.float64)
    n0 = y[:32] ** 2 + y[32:] ** 2
    n1 = r[:32] ** 2 + r[32:] ** 2
    assert np.max(np.abs(n1 - n0) / n0) < 2e-6
    # frequency 0 turns by exactly `pos` radians
    assert abs(r[0] - (y[0] * math.cos(131071.0) - y[32] * math.sin(131071.0))) < 1e-5 * np.max(np.abs(y))


def test_decode_and_prefill_producers_agree(oracle):
    # the reference's own gate (test_prefill.cu:463-504): per token, decode's
    # in-place q/k and cache rows equal the prefill kernel's outputs
    rng = np.random.default_rng(9)
    M, P = 6, 1000
    S = P + M
    Y = (rng.standard_normal((M, 3072)) * 3.0).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    kc0 = np.zeros(S * 512, np.uint16)
    vc0 = np.zeros(S * 512, np.uint16)
    qh = oracle.pf_qknr(Y, qn, kn, M, P, kc0, vc0)
    kc1 = np.zeros(S * 512, np.uint16)
    vc1 = np.zeros(S * 512, np.uint16)
    for t in range(M):
        qf = Y[t, :2048].copy()
        kf = Y[t, 2048:2560].copy()
        vf = Y[t, 2560:].copy()
        oracle.qk_norm_rope(qf, kf, vf, qn, kn, P + t, kc1, vc1)
        assert np.array_equal(qh[t], (qf * np.float32(0.125)).astype(np.float16).view(np.uint16))
        for h in range(8):
            assert np.array_equal(kf[h * 64:(h + 1) * 64], oracle.norm_rope_row(Y[t, 2048 + h * 64:2048 + (h + 1) * 64], kn, P + t))
    assert np.array_equal(kc0, kc1) and np.array_equal(vc0, vc1)
    # V is copied unnormalised and unrotated; rows outside [P, P+M) untouched
    assert np.array_equal(vc0.reshape(S, 8, 64)[P:], Y[:, 2560:].reshape(M, 8, 64).astype(np.float16).view(np.uint16))
    assert not kc0.reshape(S, 512)[:P].any()


def test_pf_quant_rows_is_q8_1_widened(oracle):
    # the planar format holds exactly block_q8_1's values (prefill.cuh:20-31)
    rng = np.random.default_rng(11)
    X = (rng.standard_normal((3, 96)) * 4).astype(np.float32)
    X[1, 32:64] = 0.0                                 # an all-zero block
    qs, sc = oracle.pf_quant_rows(X, 3, 96, 3)
    for r in range(3):
        for b in range(3):
            blk = oracle.quantize_q8_1(X[r, 32 * b:32 * b + 32])
            assert np.array_equal(qs[r, 32 * b:32 * b + 32], blk[4:].view(np.int8))
            d, s = blk[:4].view(np.float16).astype(np.float32)
            assert sc[r, b, 0] == d and sc[r, b, 1] == np.float32(8.0) * s
    assert not qs[1, 32:64].any() and sc[1, 1, 0] == 0.0
    # the q values reconstruct x to half a quantisation step
    for r in range(3):
        for b in range(3):
            x = X[r, 32 * b:32 * b + 32]
            d = np.abs(x).max() / np.float32(127.0)
            if d > 0:
                assert np.max(np.abs(qs[r, 32 * b:32 * b + 32] * d - x)) <= 0.5 * d * (1 + 1e-6)


# ---- Q4_0 x Q8_1 dot and GEMV (the consumer of the decode attention output) -----------
GOLDEN_Q4 = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "q4_0_dot.npz")


def _golden_q4():
    z = np.load(GOLDEN_Q4)
    return [(z[f"qs{i}"], z[f"d{i}"], z[f"x{i}"], z[f"expected{i}"]) for i in range(int(z["n"]))]


@pytest.mark.parametrize("case", range(4))
def test_dot_q4_0_reference_fixture(oracle, case):
    """The reference's own golden vectors (ref/quant_fixture.bin: real attn_q
    weight blocks, tests/test_quant.cu's gate): the block dots summed in order
    against its expected_exact (ggml's integer convention in float64, with fp32
    d8 and raw sums, hence the reference's 5e-3 bound) and expected_fp32."""
    qs, d, x, (exact, fp32) = _golden_q4()[case]
    xq = oracle.quantize_q8_1_blocks(x)
    acc = np.float32(0.0)
    for b in range(qs.shape[0]):
        acc = np.float32(acc + np.float32(oracle.dot_q4_0_q8_1(qs[b], int(d[b]), xq[b])))
    assert abs(acc - exact) / abs(exact) < 5e-3
    assert abs(acc - fp32) / abs(fp32) < 5e-2
    # and, tighter: the same formula in float64 on the fp16-rounded fields the
    # Q8_1 block actually carries -- the oracle is then exact up to fp32 rounding
    d4 = d.view(np.float16).astype(np.float64)
    d8 = xq[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    s8 = xq[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    nib = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.int64)
    q8 = xq[:, 4:].view(np.int8).astype(np.int64)
    want = float(np.sum(d4 * (d8 * (nib * q8).sum(1) - 8.0 * s8)))
    assert abs(acc - want) <= 1e-5 * max(1.0, abs(want))


def test_dot_q4_0_closed_form(oracle):
    """Blocks whose Q8_1 fields are exact (d8 a power of two, sum representable):
    then sum8 = d8 * sum(q8) and the block dot is the dequantised product
    sum d4 * (nibble - 8) * d8 * q8 exactly.  Swapping the nibble halves, the
    sign of the offset term or dropping a scale fails it."""
    rng = np.random.default_rng(11)
    for _ in range(200):
        qs = rng.integers(0, 256, 16, dtype=np.uint8)
        q8 = rng.integers(-20, 21, 32).astype(np.int8)
        d8 = np.float16(2.0 ** int(rng.integers(-8, 0)))
        s8 = np.float16(float(d8) * int(q8.astype(np.int64).sum()))
        assert float(s8) == float(d8) * int(q8.astype(np.int64).sum())
        xq = np.concatenate([np.array([d8, s8], np.float16).view(np.uint8), q8.view(np.uint8)])
        d4 = np.float16(rng.uniform(0.001, 0.05))
        w = np.concatenate([(qs & 0x0F).astype(np.int64) - 8, (qs >> 4).astype(np.int64) - 8])
        want = float(d4) * float(d8) * float((w * q8.astype(np.int64)).sum())
        got = oracle.dot_q4_0_q8_1(qs, int(np.array(d4).view(np.uint16)), xq)
        assert abs(got - want) <= 2e-6 * max(1.0, abs(want)) + 1e-9


def test_gemv_q4_0_rows_and_norm_scale(oracle):
    """Each output row is the fp32 sum of its block dots (float64 within fp32
    rounding), the residual is added, and the norm scale is
    1/sqrt(sum(ssq)/2048 + eps)."""
    rng = np.random.default_rng(5)
    rows, bpr = 37, 70                       # bpr > 64: lanes take three blocks
    qs = rng.integers(0, 256, (rows, bpr, 16), dtype=np.uint8)
    d = rng.uniform(0.001, 0.02, (rows, bpr)).astype(np.float16).view(np.uint16)
    xq = oracle.quantize_q8_1_blocks(rng.standard_normal(bpr * 32).astype(np.float32))
    dots = np.array([[oracle.dot_q4_0_q8_1(qs[r, k], int(d[r, k]), xq[k]) for k in range(bpr)]
                     for r in range(rows)], np.float64)
    want = dots.sum(1)
    y = oracle.gemv_q4_0(qs, d, xq, rows, bpr)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-6)
    y0 = rng.standard_normal(rows).astype(np.float32)
    ya = oracle.gemv_q4_0(qs, d, xq, rows, bpr, y=y0, add=True)
    assert np.allclose(ya, y0.astype(np.float64) + want, rtol=1e-5, atol=1e-5)
    ssq = rng.uniform(0.0, 50.0, 64).astype(np.float32)
    yn = oracle.gemv_q4_0(qs, d, xq, rows, bpr, ssq=ssq, eps=1e-5)
    ninv = 1.0 / math.sqrt(float(ssq.astype(np.float64).sum()) / 2048.0 + 1e-5)
    assert np.allclose(yn, want * ninv, rtol=1e-5, atol=1e-6)


def test_pf_gemm_q4_0_reference_fixture(oracle):
    """The prefill GEMM restatement on the reference's golden Q4_0 blocks: one
    token, the input quantised to planar Q8_1 (lko_pf_quant_rows), against
    expected_exact / expected_fp32 with the reference's gate bounds."""
    for qs, d, x, (exact, fp32) in _golden_q4():
        bpr = qs.shape[0]
        aqs, asc = oracle.pf_quant_rows(x.reshape(1, -1), 1, bpr * 32, bpr)
        # the same row 64 times (N is a multiple of 64 in the GEMM's interface)
        got = float(oracle.pf_gemm_q4_0(np.tile(qs[None], (64, 1, 1)), np.tile(d[None], (64, 1)),
                                        64, bpr, aqs, asc, 1)[0, 0])
        assert abs(got - exact) / abs(exact) < 5e-3
        assert abs(got - fp32) / abs(fp32) < 5e-2


def test_pf_gemm_q4_0_block_formula(oracle):
    """Against float64 sum_b d4 * (d8 * sumi - s8): the only rounding the
    restatement adds beyond fp32 accumulation is the magic constant's (half a
    unit of sumi per block); a swapped nibble half, a transposed operand or a
    dropped offset term is off by far more.  Residual add and per-token scale."""
    rng = np.random.default_rng(9)
    N, bpr, ntok = 64, 5, 7
    qs = rng.integers(0, 256, (N, bpr, 16), dtype=np.uint8)
    d = rng.uniform(0.002, 0.02, (N, bpr)).astype(np.float16).view(np.uint16)
    aqs, asc = oracle.pf_quant_rows(rng.standard_normal((ntok, bpr * 32)).astype(np.float32), ntok, bpr * 32, bpr)
    nib = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.int64)                 # [N][bpr][32]
    xq = aqs.reshape(ntok, bpr, 32).astype(np.int64)
    sumi = np.einsum("rbk,tbk->trb", nib, xq).astype(np.float64)
    sc = asc.reshape(ntok, bpr, 2).astype(np.float64)
    d4 = d.view(np.float16).astype(np.float64)
    want = np.einsum("rb,trb->tr", d4, sc[:, None, :, 0] * sumi - sc[:, None, :, 1])
    got = oracle.pf_gemm_q4_0(qs, d, N, bpr, aqs, asc, ntok)
    # the constant c = fma(d8, 1.5*2^23, s8) rounds once per block (at most one
    # ulp of c, about one unit of sumi); fp32 accumulation adds ~1e-6 relative
    c = (sc[:, :, 0] * 12582912.0 + sc[:, :, 1]).astype(np.float32)                  # [ntok][bpr]
    bound = np.einsum("rb,tb->tr", np.abs(d4), np.spacing(np.abs(c)).astype(np.float64)) \
        + 1e-6 * np.einsum("rb,trb->tr", np.abs(d4), np.abs(sc[:, None, :, 0] * sumi - sc[:, None, :, 1]))
    assert np.all(np.abs(got - want) <= bound)
    assert np.max(bound) < 1e-3 * np.max(np.abs(want))          # the bound itself is tight
    y0 = rng.standard_normal((ntok, N)).astype(np.float32)
    s = rng.uniform(0.5, 2.0, ntok).astype(np.float32)
    got2 = oracle.pf_gemm_q4_0(qs, d, N, bpr, aqs, asc, ntok, scale=s, out=y0, add=True)
    assert np.allclose(got2, y0 + got * s[:, None], rtol=1e-6, atol=1e-6)
