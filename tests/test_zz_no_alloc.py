"""The allocation-free decode entry point (lk_attn_decode_noalloc), through the
C ABI: bit for bit against lk_attn_decode with a caller workspace, on two calls
in a row, the second over a shorter sequence (the static scratch then still
holds the first call's records, so stale slots would show), and against the
float64 oracle.  Runs alone or after the other GPU tests."""
import numpy as np
import pytest
import torch

from gpu_util import d_pos_for, dev, dev_h, host, note

pytestmark = pytest.mark.gpu


def _inputs(seq, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = rng.standard_normal((seq, 8, 64)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16).view(np.uint16)
    return q, kc, vc


def _with_part(lk, qd, kd, vd, seq):
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    out = torch.full((32, 64), float("nan"), device="cuda")
    y = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")
    lk.attn_decode(qd, kd, vd, d_pos_for(seq), part, out, y)
    torch.cuda.synchronize()
    return host(out), host(y)


def _no_alloc(lk, qd, kd, vd, seq):
    out = torch.full((32, 64), float("nan"), device="cuda")
    y = torch.zeros(64 * 36, dtype=torch.uint8, device="cuda")
    lk.attn_decode_noalloc(qd, kd, vd, d_pos_for(seq), out, y)
    torch.cuda.synchronize()
    return host(out), host(y)


def test_no_alloc_matches_workspace_entry(lk, oracle):
    # the first call fills every slot; the second (shorter) uses fewer live
    # slices, so its dead slots must be rewritten, not read stale
    for call, (seq, seed) in enumerate(((40000, 5), (777, 6))):
        note(f"lk_attn_decode_noalloc call {call}: seq={seq}")
        q, kc, vc = _inputs(seq, seed)
        qd, kd, vd = dev(q), dev_h(kc), dev_h(vc)
        o_ref, y_ref = _with_part(lk, qd, kd, vd, seq)
        o, y = _no_alloc(lk, qd, kd, vd, seq)
        assert np.array_equal(o.view(np.uint32), o_ref.view(np.uint32)), f"call {call}: out differs"
        assert np.array_equal(y, y_ref), f"call {call}: Q8_1 differs"
        ref = oracle.decode_ref(q, kc, vc, seq)
        assert oracle.rel_err(o, ref) <= 2e-3


def test_no_alloc_rejects_null(lk):
    rc = lk.load().lk_attn_decode_noalloc(None, None, None, None, None, None, None)
    assert rc == 1 and b"null" in lk.load().lk_last_error()


def test_no_alloc_refuses_a_second_stream_while_pending(lk):
    """Every call on a GPU shares its static array: a call on stream B while one
    on stream A is still pending is refused with hipErrorNotReady (600) and a
    message; calls ordered on one stream are accepted, and so is B once A has
    completed.  A's result is intact."""
    seq = 4096
    q, kc, vc = _inputs(seq, 9)
    qd, kd, vd = dev(q), dev_h(kc), dev_h(vc)
    o_ref, _ = _with_part(lk, qd, kd, vd, seq)
    pos = d_pos_for(seq)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    oa = torch.full((32, 64), float("nan"), device="cuda")
    ob = torch.full((32, 64), float("nan"), device="cuda")
    torch.cuda.synchronize()
    note("lk_attn_decode_noalloc: guard of the shared array across two streams")
    with torch.cuda.stream(sa):
        torch.cuda._sleep(200_000_000)              # keep stream A busy (about 0.1 s)
    lk.attn_decode_noalloc(qd, kd, vd, pos, oa, None, stream=sa)
    lk.attn_decode_noalloc(qd, kd, vd, pos, oa, None, stream=sa)    # same stream: accepted
    with pytest.raises(lk.LkError) as ei:
        lk.attn_decode_noalloc(qd, kd, vd, pos, ob, None, stream=sb)
    assert "hipError 600" in str(ei.value) and "another stream" in str(ei.value)
    sa.synchronize()
    lk.attn_decode_noalloc(qd, kd, vd, pos, ob, None, stream=sb)    # A is done: accepted
    sb.synchronize()
    assert np.array_equal(host(oa).view(np.uint32), o_ref.view(np.uint32))
    assert np.array_equal(host(ob).view(np.uint32), o_ref.view(np.uint32))
