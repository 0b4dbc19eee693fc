"""Prefill attention with a caller-owned split-K workspace, its graph capture,
and the paired kernel's bounded group barrier, through the C ABI.

The reference's kernels use only buffers the engine owns
(/root/reference/src/engine.cu:974-985); lk_pf_attn8_ws / lk_pf_attn_ws take
the split-K partial workspace from the caller: with a full workspace the output
is bit-identical to the static-scratch entry points, with a small one the
planner cuts coarser pieces (same float64 tolerance), and a launch that owns
its workspace can be captured into a hipGraph and replayed.  The group barrier
of the paired kernel gives up after a bounded number of polls; the failure is
forced from the host (a poll bound of 1) and must show as NaN outputs and a
non-zero fault count, with the kernel running to its end."""
import numpy as np
import pytest
import torch

from gpu_util import dev_h, host, note

pytestmark = pytest.mark.gpu

SEED = 777


class _Case:
    def __init__(self, lk, oracle, m, P):
        K, V, Q = oracle.mt_prefill_case(SEED, m, P)
        self.K, self.V, self.Q, self.m, self.P = K, V, Q, m, P
        S = P + m
        self.kstride = lk.kstride_for(S)
        self.kc, self.vc, self.qh = dev_h(K), dev_h(V), dev_h(Q)
        self.k8 = torch.zeros(S * 512, dtype=torch.int8, device="cuda")
        self.ksc = torch.zeros(8 * self.kstride + 4, device="cuda")
        lk.pf_k8(self.kc, 0, S, None, self.kstride, self.k8, self.ksc)
        torch.cuda.synchronize()

    def out(self):
        return torch.full((self.m, 2048), float("nan"), device="cuda")

    def run8(self, lk, o, work, near=256, sink=1, stream=None):
        lk.pf_attn8_ws(None, None, None, self.qh, self.m, self.P, self.k8, self.ksc, self.kstride,
                       self.kc, self.vc, near, sink, o, None, None, work, stream=stream)

    def ref8(self, oracle, near=256, sink=1):
        """Float64 restatement of the int8 algorithm on the oracle's own quantised operands."""
        S = self.P + self.m
        q8, qsc, qcs = oracle.pf_q8(self.Q, self.m)
        k8, ksc = oracle.pf_k8(self.K, 0, S, self.kstride)
        return oracle.pf_ref8(q8, qsc, qcs, self.Q, self.m, self.P, k8, ksc, self.kstride, self.K, self.V,
                              near, sink)


def _bits(a):
    return a.view(np.uint32)


@pytest.mark.parametrize("m,P,L", [(512, 0, 2), (256, 3000, 3), (1000, 200, 0)])
def test_workspace_matches_static_scratch(lk, oracle, m, P, L):
    c = _Case(lk, oracle, m, P)
    note(f"pf workspace m={m} P={P} split={L}")
    try:
        lk.pf_pair_override(-1)
        lk.pf_split_override(L if L else 0)
        o_static = c.out()
        lk.pf_attn8(None, None, None, c.qh, m, P, c.k8, c.ksc, c.kstride, c.kc, c.vc, 256, 1, o_static)
        work = torch.empty(lk.pf_part_bytes() // 4, device="cuda")
        o_ws = c.out()
        c.run8(lk, o_ws, work)
        # fp16 kernel too
        f_static, f_ws = c.out(), c.out()
        lk.pf_attn(c.qh, m, P, c.kc, c.vc, f_static)
        lk.pf_attn_ws(c.qh, m, P, c.kc, c.vc, f_ws, None, None, work)
        torch.cuda.synchronize()
    finally:
        lk.pf_split_override(0)
        lk.pf_pair_override(0)
    assert np.array_equal(_bits(host(o_ws)), _bits(host(o_static)))
    assert np.array_equal(_bits(host(f_ws)), _bits(host(f_static)))
    ref = oracle.pf_ref(c.Q, m, P, c.K, c.V)
    assert oracle.rel_err(host(f_ws), ref) <= 2e-3
    assert oracle.rel_err(host(o_ws), c.ref8(oracle)) <= 2e-3


@pytest.mark.parametrize("floats", [0, 40000, 200000])
def test_small_workspace_coarser_plan(lk, oracle, floats):
    """A workspace below lk_pf_part_bytes() bounds the parts the planner makes
    (0 bytes: no split at all); the result stays within the float64 bound."""
    m, P = 512, 0
    c = _Case(lk, oracle, m, P)
    note(f"pf small workspace {floats} floats")
    try:
        lk.pf_pair_override(-1)
        lk.pf_split_override(1)                   # ask for the finest split: the workspace limits it
        work = torch.empty(max(floats, 4), device="cuda")
        o = c.out()
        if floats == 0:
            lk.load()
            import ctypes
            rc = lk.load().lk_pf_attn_ws(lk._ptr(c.qh), m, P, lk._ptr(c.kc), lk._ptr(c.vc), lk._ptr(o), None,
                                         None, lk._ptr(work), ctypes.c_size_t(0), lk._stream(None))
            assert rc == 0
        else:
            lk.pf_attn_ws(c.qh, m, P, c.kc, c.vc, o, None, None, work)
        torch.cuda.synchronize()
    finally:
        lk.pf_split_override(0)
        lk.pf_pair_override(0)
    assert oracle.rel_err(host(o), oracle.pf_ref(c.Q, m, P, c.K, c.V)) <= 2e-3


def test_split_launch_with_workspace_in_a_graph(lk, oracle):
    """An engine that owns every buffer captures a split prefill launch (attention
    plus the merge kernel) into a graph; every replay, with eager work of the
    program in between, gives the eager result bit for bit."""
    m, P = 512, 1000
    c = _Case(lk, oracle, m, P)
    work = torch.empty(lk.pf_part_bytes() // 4, device="cuda")
    o_eager, o_graph = c.out(), c.out()
    note("pf split launch captured in a graph")
    s = torch.cuda.Stream()
    try:
        lk.pf_pair_override(-1)
        lk.pf_split_override(2)
        c.run8(lk, o_eager, work)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            c.run8(lk, o_graph, work, stream=s)
    finally:
        lk.pf_split_override(0)
        lk.pf_pair_override(0)
    want = _bits(host(o_eager)).copy()
    for rep in range(3):
        o_graph.fill_(float("nan"))               # eager work between the replays
        work.fill_(12345.0)                       # stale partials must not matter
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(host(o_graph)), want), f"replay {rep}"
    del g
    assert oracle.rel_err(host(o_eager), c.ref8(oracle)) <= 2e-3


def test_group_barrier_bound_reports_and_poisons(lk, oracle):
    """Forced from the host: with a poll bound of 1 the paired kernel's group
    barriers give up; the kernel still completes, the fault count is non-zero
    and the affected workgroups write NaN.  With the default bound the same
    launch is correct and counts nothing."""
    m, P = 1024, 0
    c = _Case(lk, oracle, m, P)
    lk.pf_gsync_faults(reset=True)
    note("pf paired kernel: forced group-barrier timeout (poll bound 1)")
    try:
        lk.pf_pair_override(1)
        lk.pf_gsync_limit(1)
        o_bad = c.out()
        c.run8(lk, o_bad, None)
        torch.cuda.synchronize()
        faults = lk.pf_gsync_faults(reset=True)
        lk.pf_gsync_limit(0)                       # the default bound again
        o_ok = c.out()
        c.run8(lk, o_ok, None)
        torch.cuda.synchronize()
        clean = lk.pf_gsync_faults(reset=True)
    finally:
        lk.pf_gsync_limit(0)
        lk.pf_pair_override(0)
    ob = host(o_bad)
    assert faults > 0
    assert np.isnan(ob).any(), "a barrier that gave up must poison its workgroup's output"
    assert clean == 0
    ok = host(o_ok)
    assert not np.isnan(ok).any()
    assert oracle.rel_err(ok, c.ref8(oracle)) <= 2e-3
