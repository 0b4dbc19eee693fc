"""Decode attention parity on the GPU, through the C ABI.

Mirrors the reference's gate G6 (tests/test_attn.cu): the same xorshift64
inputs (seed 0x9e3779b97f4a7c15, state carried from case to case, the whole
131072-position cache filled per case), the same 12 lengths in the same order,
split+combine and the serial kernel each against the float64 reference, and
split against serial.  Tolerances: the reference's 1e-3 absolute (1e-4 split vs
serial) and the north-star 2e-3 max relative error; the combine's Q8_1 output is
checked bit-exactly.  Also: determinism, the hipGraph, the BASELINE decode
configurations and the error paths.
"""
import numpy as np
import pytest
import torch

from gpu_util import abs_err, d_pos_for, dev, dev_h, host, note, host_h

pytestmark = pytest.mark.gpu

REF_LENGTHS = [4096, 8192, 513, 512, 100, 5, 1, 16384, 32768, 65536, 100003, 131072]
CACHE = 131072 * 8 * 64


class _XsCases:
    """Generates test_attn.cu's cases in order, carrying the generator state."""

    def __init__(self, oracle):
        self.gen = oracle.XorShiftAttnCases()
        self.done = -1
        self.data = None

    def case(self, idx):
        assert idx >= self.done, "cases must be requested in reference order"
        while self.done < idx:
            self.data = self.gen.next_case(CACHE)
            self.done += 1
        return self.data


@pytest.fixture(scope="module")
def xs_cases(oracle):
    return _XsCases(oracle)


def _run_decode(lk, q, kc, vc, seq, yq8=False):
    d_pos = d_pos_for(seq)
    part = torch.empty(lk.part_bytes() // 4, dtype=torch.float32, device="cuda")
    out = torch.full((32, 64), float("nan"), device="cuda")
    y = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda") if yq8 else None
    lk.attn_decode(q, kc, vc, d_pos, part, out, y)
    torch.cuda.synchronize()
    return out, y


@pytest.mark.parametrize("idx", range(len(REF_LENGTHS)), ids=[f"seq{s}" for s in REF_LENGTHS])
def test_reference_cases(lk, oracle, xs_cases, idx):
    seq = REF_LENGTHS[idx]
    q, kc, vc = xs_cases.case(idx)
    note(f"decode reference case seq={seq}")
    qd, kd, vd = dev(q), dev_h(kc), dev_h(vc)
    out, y = _run_decode(lk, qd, kd, vd, seq, yq8=True)
    ref = oracle.decode_ref(q, kc, vc, seq)
    o = host(out)
    ep = abs_err(o, ref)
    rel = oracle.rel_err(o, ref)
    note(f"  split vs float64: abs {ep:.3e} rel {rel:.3e}")
    assert ep <= 1e-3 and rel <= 2e-3
    # the combine's Q8_1 epilogue, bit-exact against the oracle on the same values
    yb = host(y).reshape(64, 36)
    for b in range(64):
        assert np.array_equal(yb[b], oracle.quantize_q8_1(o.reshape(-1)[32 * b:32 * b + 32])), b
    if seq <= lk.DECODE_MAX_SEQ:
        os_ = torch.full((32, 64), float("nan"), device="cuda")
        lk.attention_decode(qd, kd, vd, d_pos_for(seq), os_, None)
        torch.cuda.synchronize()
        os_ = host(os_)
        es = abs_err(os_, ref)
        note(f"  serial vs float64: abs {es:.3e}; split vs serial {abs_err(os_, o):.3e}")
        assert es <= 1e-3 and abs_err(os_, o) <= 1e-4


def test_seq1_is_v_exactly(lk, oracle):
    rng = np.random.default_rng(21)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = rng.standard_normal((64, 8, 64)).astype(np.float16)
    vc = rng.standard_normal((64, 8, 64)).astype(np.float16)
    note("decode seq=1 closed form")
    out, _ = _run_decode(lk, dev(q), dev_h(kc.view(np.uint16)), dev_h(vc.view(np.uint16)), 1)
    assert np.array_equal(host(out), np.repeat(vc[0].astype(np.float32), 4, axis=0))


def test_constant_keys_average(lk, oracle):
    rng = np.random.default_rng(22)
    seq = 3000
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = np.ascontiguousarray(np.broadcast_to(rng.standard_normal((1, 8, 64)), (seq, 8, 64))).astype(np.float16)
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    note("decode constant keys")
    out, _ = _run_decode(lk, dev(q), dev_h(kc.view(np.uint16)), dev_h(vc.view(np.uint16)), seq)
    want = np.repeat(vc.astype(np.float64).mean(0), 4, axis=0)
    assert abs_err(host(out), want) <= 1e-5


def test_large_q_heads(lk, oracle):
    """q is fp32 in the interface; heads whose |q| reaches past fp16's range
    (the kernel's q = hi + lo fp16 split) are scaled by a power of 2 inside the
    kernel.  Mixed in one kv group with ordinary heads, against float64."""
    rng = np.random.default_rng(29)
    seq = 5000
    q = rng.standard_normal((32, 64)).astype(np.float32)
    q[1] *= 4e4                 # max |q| ~ 1e5 > 65504
    q[6] *= 1e9                 # one-hot softmax
    q[13] *= 3e4
    kc = (rng.standard_normal((seq, 8, 64)) * 2.5e-4).astype(np.float16)
    kc[:, 1] *= 4000.0          # kv head 1 (heads 4-7) at ordinary scale
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    note("decode large-|q| heads")
    out, _ = _run_decode(lk, dev(q), dev_h(kc.view(np.uint16)), dev_h(vc.view(np.uint16)), seq)
    ref = oracle.decode_ref(q, kc.view(np.uint16), vc.view(np.uint16), seq)
    o = host(out)
    assert np.isfinite(o).all()
    for h in range(32):
        assert oracle.rel_err(o[h], ref[h]) <= 2e-3, h


def test_bitwise_deterministic(lk, oracle):
    rng = np.random.default_rng(23)
    seq = 77777
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kd = torch.randn(seq, 8, 64, device="cuda").half()
    vd = torch.randn(seq, 8, 64, device="cuda").half()
    note("decode determinism seq=77777")
    outs = [host(_run_decode(lk, dev(q), kd, vd, seq, yq8=True)[0]) for _ in range(5)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


def test_null_outputs_and_q8_only(lk, oracle):
    rng = np.random.default_rng(24)
    seq = 1000
    q = dev(rng.standard_normal((32, 64)).astype(np.float32))
    kd = torch.randn(seq, 8, 64, device="cuda").half()
    vd = torch.randn(seq, 8, 64, device="cuda").half()
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    d_pos = d_pos_for(seq)
    note("decode nullable outputs")
    y1 = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")
    lk.attn_decode(q, kd, vd, d_pos, part, None, y1)
    out = torch.empty(32, 64, device="cuda")
    y2 = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")
    lk.attn_split(q, kd, vd, d_pos, part)
    lk.attn_combine(part, d_pos, out, y2)
    lk.attn_combine(part, d_pos, None, None)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("seq", [1, 9, 17, 100, 112, 113, 1025, 1031, 4100])
def test_dead_slices_write_neutral_records(lk, oracle, seq):
    """Slots whose slice holds no tile (fewer 16-position tiles than slices:
    seq <= 112, and every slot past the slice count) and lengths around that
    edge: the partial buffer starts as NaN everywhere, the combine merges all
    slots, and the result is the float64 reference's."""
    rng = np.random.default_rng(seq)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16)
    part = torch.full((lk.part_bytes() // 4,), float("nan"), device="cuda")
    out = torch.full((32, 64), float("nan"), device="cuda")
    note(f"decode dead slices seq={seq}")
    lk.attn_decode(dev(q), dev_h(kc.view(np.uint16)), dev_h(vc.view(np.uint16)), d_pos_for(seq), part, out, None)
    torch.cuda.synchronize()
    ref = oracle.decode_ref(q, kc.view(np.uint16), vc.view(np.uint16), seq)
    o = host(out)
    assert np.isfinite(o).all()
    assert abs_err(o, ref) <= 1e-3


@pytest.mark.parametrize("seq", [127, 128, 129, 4095, 4096, 4097, 4111, 4112, 4113, 8193, 12345])
def test_slice_and_tile_edges(lk, oracle, seq):
    """Lengths at the edges of the slice layout: the slice count reaching 8 and
    256, a last tile of 1, 15 and 16 positions, slices holding one or two
    tiles (at 4097 slice 0 holds tiles 0 and 256): split + combine against
    the float64 reference, and repeat bit-identity."""
    rng = np.random.default_rng(seq + 7)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = rng.standard_normal((seq, 8, 64)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16).view(np.uint16)
    note(f"decode slice/tile edges seq={seq}")
    qd, kd, vd = dev(q), dev_h(kc), dev_h(vc)
    o1, _ = _run_decode(lk, qd, kd, vd, seq)
    o2, _ = _run_decode(lk, qd, kd, vd, seq)
    ref = oracle.decode_ref(q, kc, vc, seq)
    o = host(o1)
    assert np.isfinite(o).all()
    assert abs_err(o, ref) <= 1e-3 and oracle.rel_err(o, ref) <= 2e-3
    assert torch.equal(o1.view(torch.int32), o2.view(torch.int32))


def test_serial_beyond_limit_writes_nothing(lk):
    seq = lk.DECODE_MAX_SEQ + 1
    q = torch.randn(32, 64, device="cuda")
    kd = torch.randn(seq, 8, 64, device="cuda").half()
    out = torch.full((32, 64), 7.0, device="cuda")
    note("serial decode beyond its limit")
    lk.attention_decode(q, kd, kd, d_pos_for(seq), out, None)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_graph_replay_matches_eager_and_is_position_independent(lk, oracle):
    layers, cap = 10, 6000
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    qs = [torch.randn(32, 64, device="cuda", generator=g) for _ in range(layers)]
    kcs = [torch.randn(cap, 8, 64, device="cuda", generator=g).half() for _ in range(layers)]
    vcs = [torch.randn(cap, 8, 64, device="cuda", generator=g).half() for _ in range(layers)]
    d_pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    outs = [torch.empty(32, 64, device="cuda") for _ in range(layers)]
    yq8s = [torch.zeros(64 * 36, dtype=torch.uint8, device="cuda") for _ in range(layers)]
    note("decode graph capture, 10 layers")
    graph = lk.DecodeGraph(qs, kcs, vcs, d_pos, part, outs, yq8s)
    assert graph.nodes() == 2 * layers
    eager_part = torch.empty_like(part)
    for seq in [1, 129, 4000, 5999, 4000]:
        d_pos.fill_(seq - 1)
        torch.cuda.synchronize()
        graph.launch()
        graph.stream.synchronize()
        for i in range(layers):
            o = torch.empty(32, 64, device="cuda")
            y = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")
            lk.attn_decode(qs[i], kcs[i], vcs[i], d_pos, eager_part, o, y)
            torch.cuda.synchronize()
            assert torch.equal(o.view(torch.int32), outs[i].view(torch.int32)), (seq, i)
            assert torch.equal(y, yq8s[i]), (seq, i)
        kh = kcs[3][:seq].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        vh = vcs[3][:seq].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        ref = oracle.decode_ref(host(qs[3]), kh, vh, seq)
        assert oracle.rel_err(host(outs[3]), ref) <= 2e-3
    graph.close()


def _check_config(lk, oracle, cfg, layers, check_layers):
    import lk_configs
    note(f"decode config {cfg} ({layers} layer(s))")
    qs, kcs, vcs, seq = lk_configs.decode_inputs(cfg, layers=layers)
    d_pos = d_pos_for(seq)
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    outs = [torch.empty(32, 64, device="cuda") for _ in range(layers)]
    graph = lk.DecodeGraph(qs, kcs, vcs, d_pos, part, outs)
    graph.launch()
    graph.stream.synchronize()
    for i in check_layers:
        kh = kcs[i].view(torch.int16).cpu().numpy().view(np.uint16)
        vh = vcs[i].view(torch.int16).cpu().numpy().view(np.uint16)
        ref = oracle.decode_ref(host(qs[i]), kh, vh, seq)
        o = host(outs[i])
        rel = oracle.rel_err(o, ref)
        note(f"  layer {i}: abs {abs_err(o, ref):.3e} rel {rel:.3e}")
        assert rel <= 2e-3 and abs_err(o, ref) <= 1e-3
    graph.close()


def test_config_c1(lk, oracle):
    _check_config(lk, oracle, "C1", 1, [0])


def test_config_c2(lk, oracle):
    _check_config(lk, oracle, "C2", 1, [0])


def test_config_c3_graph(lk, oracle):
    _check_config(lk, oracle, "C3", 10, [0, 9])


@pytest.mark.parametrize("P0,steps", [(1000, 5), (0, 3), (14, 4), (2047, 3), (4094, 4)])
def test_decode_step_graph_runs_steps_like_the_oracle(lk, oracle, P0, steps):
    """The decode step graph (per layer: qk norm + RoPE + cache append folded
    into the split, combine; d_pos += 1 in the last combine) replayed n times =
    n decode steps: cache
    rows, d_pos and every layer's output against the oracle, and the replay
    bit-identical to the same kernels called eagerly."""
    rng = np.random.default_rng(61)
    # from 4094 the slice count reaches 256 and the new row moves into the
    # second tile of slice 0
    layers, cap = 3, max(2048, P0 + steps) + 64
    note(f"decode step graph: {layers} layers, {steps} steps from position {P0}")
    Ls, host_in = [], []
    for i in range(layers):
        qs = (rng.standard_normal(2048) * 2).astype(np.float32)
        ks = (rng.standard_normal(512) * 2).astype(np.float32)
        vs = rng.standard_normal(512).astype(np.float32)
        qn = rng.uniform(0.5, 1.5, 64).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, 64).astype(np.float32)
        kc0 = np.zeros((cap, 8, 64), np.uint16)
        vc0 = np.zeros((cap, 8, 64), np.uint16)
        kc0[:P0] = rng.standard_normal((P0, 8, 64)).astype(np.float16).view(np.uint16)
        vc0[:P0] = rng.standard_normal((P0, 8, 64)).astype(np.float16).view(np.uint16)
        host_in.append((qs, ks, vs, qn, kn, kc0, vc0))
        Ls.append({"q_src": dev(qs), "k_src": dev(ks), "v_src": dev(vs),
                   "q": torch.empty(2048, device="cuda"), "k": torch.empty(512, device="cuda"),
                   "q_norm": dev(qn), "k_norm": dev(kn), "kc": dev_h(kc0), "vc": dev_h(vc0),
                   "out": torch.full((32, 64), float("nan"), device="cuda"),
                   "yq8": torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")})
    d_pos = torch.tensor([P0], dtype=torch.int32, device="cuda")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    g = lk.DecodeStepGraph(Ls, d_pos, part)
    assert g.nodes() == 2 * layers           # producer in the split node, advance in the last combine
    g.run(steps)
    g.stream.synchronize()
    assert int(d_pos.item()) == P0 + steps
    # eager replay of the same kernels on fresh copies must match bit for bit
    E = [{k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in L.items()} for L in Ls]
    for i, (qs, ks, vs, qn, kn, kc0, vc0) in enumerate(host_in):
        E[i]["kc"], E[i]["vc"] = dev_h(kc0), dev_h(vc0)
    dp = torch.tensor([P0], dtype=torch.int32, device="cuda")
    for s in range(steps):
        for L in E:
            L["q"].copy_(L["q_src"]); L["k"].copy_(L["k_src"])
            lk.qk_norm_rope(L["q"], L["k"], L["v_src"], L["q_norm"], L["k_norm"], dp, L["kc"], L["vc"])
            lk.attn_split(L["q"], L["kc"], L["vc"], dp, part)
            lk.attn_combine(part, dp, L["out"], L["yq8"])
        dp += 1
    torch.cuda.synchronize()
    for L, M in zip(Ls, E):
        assert torch.equal(L["out"].view(torch.int32), M["out"].view(torch.int32))
        assert torch.equal(L["yq8"], M["yq8"])
        assert torch.equal(L["kc"].view(torch.int16), M["kc"].view(torch.int16))
        assert torch.equal(L["vc"].view(torch.int16), M["vc"].view(torch.int16))
        # the working q / k rows of the last step, as the standalone producer writes them
        assert torch.equal(L["q"].view(torch.int32), M["q"].view(torch.int32))
        assert torch.equal(L["k"].view(torch.int32), M["k"].view(torch.int32))
    # against the oracle: appended rows and the last step's output
    last = P0 + steps - 1
    for (qs, ks, vs, qn, kn, kc0, vc0), L in zip(host_in, Ls):
        kc_h = host_h(L["kc"]).reshape(cap, 8, 64)
        vc_h = host_h(L["vc"]).reshape(cap, 8, 64)
        assert np.array_equal(kc_h[:P0], kc0[:P0]) and np.array_equal(vc_h[:P0], vc0[:P0])
        for s in range(steps):
            krow = np.concatenate([oracle.norm_rope_row(ks[h * 64:(h + 1) * 64], kn, P0 + s) for h in range(8)])
            assert np.array_equal(kc_h[P0 + s].reshape(-1), krow.astype(np.float16).view(np.uint16))
            assert np.array_equal(vc_h[P0 + s].reshape(-1), vs.astype(np.float16).view(np.uint16))
        q_rot = np.concatenate([oracle.norm_rope_row(qs[h * 64:(h + 1) * 64], qn, last) for h in range(32)])
        ref = oracle.decode_ref(q_rot.reshape(32, 64), kc_h[:last + 1].reshape(-1), vc_h[:last + 1].reshape(-1), last + 1)
        assert oracle.rel_err(host(L["out"]), ref) <= 2e-3
    g.close()


def test_decode_step_graph_with_output_projection(lk, oracle):
    """The step graph with the optional third node per layer (x += W_o . yq8,
    lk_gemv_q4_0): three nodes per layer, and after each replay every layer's
    residual stream equals the oracle's GEMV of that step's Q8_1 blocks added
    to the previous x, bit for bit."""
    rng = np.random.default_rng(62)
    layers, cap, P0, steps = 2, 1024, 500, 3
    note(f"decode step graph with the output projection: {layers} layers, {steps} steps")
    Ls, W = [], []
    for i in range(layers):
        wq = rng.integers(0, 256, (2048, 64, 16), dtype=np.uint8)
        wd = rng.uniform(0.002, 0.02, (2048, 64)).astype(np.float16).view(np.uint16)
        W.append((wq, wd))
        kc0 = np.zeros((cap, 8, 64), np.uint16)
        vc0 = np.zeros((cap, 8, 64), np.uint16)
        kc0[:P0] = rng.standard_normal((P0, 8, 64)).astype(np.float16).view(np.uint16)
        vc0[:P0] = rng.standard_normal((P0, 8, 64)).astype(np.float16).view(np.uint16)
        Ls.append({"q_src": dev((rng.standard_normal(2048) * 2).astype(np.float32)),
                   "k_src": dev((rng.standard_normal(512) * 2).astype(np.float32)),
                   "v_src": dev(rng.standard_normal(512).astype(np.float32)),
                   "q": torch.empty(2048, device="cuda"), "k": torch.empty(512, device="cuda"),
                   "q_norm": dev(rng.uniform(0.5, 1.5, 64).astype(np.float32)),
                   "k_norm": dev(rng.uniform(0.5, 1.5, 64).astype(np.float32)),
                   "kc": dev_h(kc0), "vc": dev_h(vc0), "out": None,
                   "yq8": torch.zeros(64 * 36, dtype=torch.uint8, device="cuda"),
                   "wo_qs": dev(wq.reshape(-1)), "wo_d": dev(wd.reshape(-1).view(np.int16)),
                   "x": dev(rng.standard_normal(2048).astype(np.float32))})
    d_pos = torch.tensor([P0], dtype=torch.int32, device="cuda")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    g = lk.DecodeStepGraph(Ls, d_pos, part)
    assert g.nodes() == 3 * layers
    for s in range(steps):
        x_before = [host(L["x"]).copy() for L in Ls]
        g.run(1)
        g.stream.synchronize()
        for (wq, wd), L, x0 in zip(W, Ls, x_before):
            want = oracle.gemv_q4_0(wq, wd, host(L["yq8"]).reshape(64, 36), 2048, 64, y=x0, add=True)
            assert np.array_equal(host(L["x"]).view(np.uint32), want.view(np.uint32)), s
    assert int(d_pos.item()) == P0 + steps
    g.close()


def test_read_probe_reads_and_leaves_sink(lk):
    """The measurement probe (not on the attention path) runs over a buffer and
    leaves its sink untouched; misaligned sizes are rejected."""
    buf = torch.ones(1 << 20, device="cuda")
    sink = torch.zeros(1, device="cuda")
    note("read probe")
    lk.read_probe(buf, sink)
    torch.cuda.synchronize()
    assert float(sink.item()) == 0.0
    with pytest.raises(Exception):
        lk.read_probe(torch.ones(3, dtype=torch.float16, device="cuda"), sink)
