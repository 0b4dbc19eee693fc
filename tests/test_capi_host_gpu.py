"""The attention library driven from C++ through its C ABI alone
(tests/csrc/capi_host.cpp, built by tests/csrc/Makefile): the engine-side view
of the drop-in -- hipMalloc'ed buffers, one stream, the decode attention also
as a captured graph, the prefill attention with the caller's workspace, an
error return for a NULL operand.  The C++ side only moves data; the checks are
here, against the float64 oracle:

* decode (workspace, allocation-free and graph forms) bit-identical to each
  other and within 2e-3 relative of the float64 reference;
* lk_pf_k8 bit-exact against the oracle's quantiser;
* the int8 prefill attention with Q quantised in the kernel, through the
  static scratch and through the caller's workspace, bit-identical to each
  other and within 2e-3 relative of the float64 restatement of the int8
  algorithm on the oracle's own int8 operands.
"""
import ctypes
import os

import numpy as np
import pytest

from gpu_util import note

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "libcapi_host.so")


@pytest.mark.parametrize("seq,m,P,near,sink", [(3000, 300, 200, 96, 1), (777, 513, 4096, 0, 0)])
def test_cpp_caller(lk, oracle, seq, m, P, near, sink):
    assert os.path.exists(LIB), "tests/csrc/libcapi_host.so is not built (make -C tests/csrc)"
    lk.load()                                       # the same liblk_attn.so the C++ side links
    host = ctypes.CDLL(LIB)
    P_ = ctypes.c_void_p
    host.capi_host_run.argtypes = [P_, P_, P_, ctypes.c_int, P_, P_, P_, P_, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, P_, P_, P_, ctypes.c_char_p, ctypes.c_int]
    host.capi_host_run.restype = ctypes.c_int
    rng = np.random.default_rng(seq + m)
    q = rng.standard_normal((32, 64)).astype(np.float32)
    kc = rng.standard_normal((seq, 8, 64)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((seq, 8, 64)).astype(np.float16).view(np.uint16)
    K, V, Q = oracle.mt_prefill_case(seq, m, P, 1.0, True)
    S = P + m
    kstride = (S + 3) & ~3
    dec = np.full((3, 32, 64), np.nan, np.float32)
    pf = np.full((2, m, 2048), np.nan, np.float32)
    k8 = np.zeros(S * 512, np.int8)
    ksc = np.zeros(8 * kstride, np.float32)
    msg = ctypes.create_string_buffer(512)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    note(f"C++ caller: decode seq={seq}, prefill m={m} P={P} near={near} sink={sink}")
    rc = host.capi_host_run(ptr(q), ptr(kc), ptr(vc), seq, ptr(dec), ptr(Q), ptr(K), ptr(V), m, P, near, sink,
                            ptr(pf), ptr(k8), ptr(ksc), msg, len(msg))
    assert rc == 0, msg.value.decode()
    # decode: three entry points, one result
    assert np.array_equal(dec[0].view(np.uint32), dec[1].view(np.uint32))
    assert np.array_equal(dec[0].view(np.uint32), dec[2].view(np.uint32))
    ref = oracle.decode_ref(q, kc, vc, seq)
    assert oracle.rel_err(dec[0], ref) <= 2e-3
    # prefill: the int8 K, then the attention on the oracle's own int8 operands
    k8o, ksco = oracle.pf_k8(K, 0, S, kstride)
    assert np.array_equal(k8, k8o) and np.array_equal(ksc.view(np.uint32), ksco.view(np.uint32))
    assert np.array_equal(pf[0].view(np.uint32), pf[1].view(np.uint32))
    q8, qsc, qcs = oracle.pf_q8(Q, m)
    ref8 = oracle.pf_ref8(q8, qsc, qcs, Q, m, P, k8o, ksco, kstride, K, V, near, sink)
    r8 = oracle.rel_err(pf[0], ref8)
    note(f"  decode rel {oracle.rel_err(dec[0], ref):.3e}, prefill int8 rel {r8:.3e}")
    assert np.isfinite(pf[0]).all() and r8 <= 2e-3
