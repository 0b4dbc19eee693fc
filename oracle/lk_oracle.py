"""ctypes binding of the CPU oracle (oracle/_build/liblk_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the timed CPU baseline,
never by the product path.  Arrays are numpy; fp16 data travels as uint16 bit
patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liblk_oracle.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-B", "-C", HERE], check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    P, I, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_double
    U64, F, S = ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t
    sig = {
        "lko_h2f": ([ctypes.c_uint16], F),
        "lko_f2h": ([F], ctypes.c_uint16),
        "lko_h2f_n": ([P, P, S], None),
        "lko_f2h_n": ([P, P, S], None),
        "lko_attn_slices": ([I, I, I, I, P, P], None),
        "lko_decode_ref": ([P, P, P, I, P], None),
        "lko_quantize_q8_1": ([P, P], None),
        "lko_q8_row": ([P, P, P, F], None),
        "lko_pf_q8": ([P, I, P, P, P, P], None),
        "lko_pf_k8": ([P, I, I, P, I, P, P], None),
        "lko_pf_kmean": ([P, I, P], None),
        "lko_pf_exact": ([I, I, I, I, I], I),
        "lko_pf_ref": ([P, I, I, P, P, P, I, P], None),
        "lko_pf_ref8": ([P, P, P, P, I, I, P, P, I, P, P, I, I, P, I, P], None),
        "lko_qk_i32": ([P, I, P, I, P], None),
        "lko_norm_rope_row": ([P, P, I, P], None),
        "lko_pf_quant_rows": ([P, I, I, I, P, P], None),
        "lko_qk_norm_rope": ([P, P, P, P, P, I, P, P], None),
        "lko_pf_qknr": ([P, P, P, I, I, P, P, P], None),
        "lko_xs_fill_attn_case": ([P, S, P, P, P], None),
        "lko_sm_normal": ([U64, P, S], None),
        "lko_sm_uniform": ([U64, P, S, F, F], None),
        "lko_sm_student4": ([U64, P, S], None),
        "lko_mt_prefill_case": ([ctypes.c_uint32, I, I, F, I, P, P, P], None),
        "lko_rel_err": ([P, P, S], D),
        "lko_dot_q4_0_q8_1": ([P, ctypes.c_uint16, P], F),
        "lko_gemv_q4_0": ([P, P, P, I, I, P, F, P, I], None),
        "lko_pf_gemm_q4_0": ([P, P, I, I, P, P, I, P, P, I, I], None),
        "lko_set_threads": ([I], I),
        "lko_sm64_n": ([U64, P, S], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def set_threads(n: int = 0) -> int:
    """Threads of the float64 references (0: OpenMP's default); returns the count in effect."""
    return int(load().lko_set_threads(int(n)))


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---- fp16 ------------------------------------------------------------------------
def h2f(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    f = np.empty(h.shape, np.float32)
    load().lko_h2f_n(_p(h), _p(f), h.size)
    return f


def f2h(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    h = np.empty(f.shape, np.uint16)
    load().lko_f2h_n(_p(f), _p(h), f.size)
    return h


# ---- decode ------------------------------------------------------------------------
def attn_slices(seq, split_cap, target_n, split_min):
    ns, ch = ctypes.c_int(), ctypes.c_int()
    load().lko_attn_slices(seq, split_cap, target_n, split_min, ctypes.byref(ns), ctypes.byref(ch))
    return ns.value, ch.value


def decode_ref(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, seq: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.uint16)
    vc = np.ascontiguousarray(vc, np.uint16)
    assert q.size == 2048 and kc.size >= seq * 512 and vc.size >= seq * 512
    out = np.empty((32, 64), np.float64)
    load().lko_decode_ref(_p(q), _p(kc), _p(vc), seq, _p(out))
    return out


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """32 fp32 values -> 36-byte Q8_1 block (uint8)."""
    x = np.ascontiguousarray(x, np.float32)
    assert x.size == 32
    y = np.empty(36, np.uint8)
    load().lko_quantize_q8_1(_p(x), _p(y))
    return y


# ---- prefill quantisers --------------------------------------------------------------
def q8_row(v: np.ndarray, mul: float = 1.0):
    v = np.ascontiguousarray(v, np.float32)
    assert v.size == 64
    dst = np.empty(64, np.int8)
    sc = ctypes.c_float()
    load().lko_q8_row(_p(v), _p(dst), ctypes.byref(sc), mul)
    return dst, np.float32(sc.value)


def pf_q8(qh: np.ndarray, m: int, cm=None):
    qh = np.ascontiguousarray(qh, np.uint16)
    q8 = np.empty((m, 2048), np.int8)
    qsc = np.empty((m, 32), np.float32)
    qcs = np.empty((m, 32), np.float32)
    cmv = None if cm is None else np.ascontiguousarray(cm, np.float32)
    load().lko_pf_q8(_p(qh), m, _p(cmv), _p(q8), _p(qsc), _p(qcs))
    return q8, qsc, qcs


def pf_k8(kc: np.ndarray, p0: int, p1: int, kstride: int, cm=None, k8=None, ksc=None):
    kc = np.ascontiguousarray(kc, np.uint16)
    if k8 is None:
        k8 = np.zeros(kc.size, np.int8)
    if ksc is None:
        ksc = np.zeros(8 * kstride, np.float32)
    cmv = None if cm is None else np.ascontiguousarray(cm, np.float32)
    load().lko_pf_k8(_p(kc), p0, p1, _p(cmv), kstride, _p(k8), _p(ksc))
    return k8, ksc


def pf_kmean(kc: np.ndarray, n: int) -> np.ndarray:
    kc = np.ascontiguousarray(kc, np.uint16)
    cm = np.empty((8, 64), np.float32)
    load().lko_pf_kmean(_p(kc), n, _p(cm))
    return cm


def pf_exact(P, qt, kt, near, sink) -> bool:
    return bool(load().lko_pf_exact(P, qt, kt, near, sink))


def _rows(rows, m):
    if rows is None:
        return None, m
    r = np.ascontiguousarray(rows, np.int32)
    return r, r.size


def pf_ref(qh, m, P, kc, vc, rows=None) -> np.ndarray:
    """Float64 causal attention (test_prefill.cu:263-282).  Unlisted rows are NaN."""
    qh, kc, vc = (np.ascontiguousarray(a, np.uint16) for a in (qh, kc, vc))
    o = np.full((m, 2048), np.nan)
    r, n = _rows(rows, m)
    load().lko_pf_ref(_p(qh), m, P, _p(kc), _p(vc), _p(r), n, _p(o))
    return o


def pf_ref8(q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, rows=None) -> np.ndarray:
    """Float64 restatement of the int8-score attention algorithm.  Unlisted rows are NaN."""
    q8 = np.ascontiguousarray(q8, np.int8)
    k8 = np.ascontiguousarray(k8, np.int8)
    qsc = np.ascontiguousarray(qsc, np.float32)
    qcs = None if qcs is None else np.ascontiguousarray(qcs, np.float32)
    ksc = np.ascontiguousarray(ksc, np.float32)
    qh, kc, vc = (np.ascontiguousarray(a, np.uint16) for a in (qh, kc, vc))
    o = np.full((m, 2048), np.nan)
    r, n = _rows(rows, m)
    load().lko_pf_ref8(_p(q8), _p(qsc), _p(qcs), _p(qh), m, P, _p(k8), _p(ksc), kstride,
                       _p(kc), _p(vc), near, sink, _p(r), n, _p(o))
    return o


def qk_i32(q8, m, k8, n) -> np.ndarray:
    q8 = np.ascontiguousarray(q8, np.int8)
    k8 = np.ascontiguousarray(k8, np.int8)
    s = np.empty((32, m, n), np.int32)
    load().lko_qk_i32(_p(q8), m, _p(k8), n, _p(s))
    return s


def pf_quant_rows(X, rows, ld, kb):
    """Planar Q8_1 (qs int8 [rows][kb*32], sc fp32 [rows][kb][2])."""
    X = np.ascontiguousarray(X, np.float32)
    qs = np.empty((rows, kb * 32), np.int8)
    sc = np.empty((rows, kb, 2), np.float32)
    load().lko_pf_quant_rows(_p(X), int(rows), int(ld), int(kb), _p(qs), _p(sc))
    return qs, sc


# ---- attention-input producers (kernels.cu:871-915, prefill.cu:975-1016) ----------------
def norm_rope_row(v, w, pos) -> np.ndarray:
    v = np.ascontiguousarray(v, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty(64, np.float32)
    load().lko_norm_rope_row(_p(v), _p(w), int(pos), _p(out))
    return out


def qk_norm_rope(qf, kf, vf, qn, kn, pos, kc, vc):
    """In place on qf [32*64], kf [8*64] (fp32) and kc / vc (uint16 fp16 bits)."""
    for a, t in ((qf, np.float32), (kf, np.float32), (kc, np.uint16), (vc, np.uint16)):
        assert a.dtype == t and a.flags["C_CONTIGUOUS"]
    vf, qn, kn = (np.ascontiguousarray(a, np.float32) for a in (vf, qn, kn))
    load().lko_qk_norm_rope(_p(qf), _p(kf), _p(vf), _p(qn), _p(kn), int(pos), _p(kc), _p(vc))


def pf_qknr(Y, qn, kn, m, P, kc, vc) -> np.ndarray:
    """Returns qh (uint16 [m][2048]); writes rows P .. P+m-1 of kc / vc in place."""
    Y, qn, kn = (np.ascontiguousarray(a, np.float32) for a in (Y, qn, kn))
    assert kc.dtype == np.uint16 and vc.dtype == np.uint16
    qh = np.zeros((m, 2048), np.uint16)
    load().lko_pf_qknr(_p(Y), _p(qn), _p(kn), int(m), int(P), _p(qh), _p(kc), _p(vc))
    return qh


# ---- generators ---------------------------------------------------------------------
class XorShiftAttnCases:
    """tests/test_attn.cu's generator: one state carried across cases."""

    SEED = 0x9E3779B97F4A7C15
    CACHE = 131072 * 8 * 64          # the reference fills the full LK_ATTN_MAX_SEQ cache

    def __init__(self, seed: int = SEED):
        self.state = ctypes.c_uint64(seed)

    def next_case(self, cache_elems: int = CACHE):
        q = np.empty(2048, np.float32)
        kc = np.empty(cache_elems, np.uint16)
        vc = np.empty(cache_elems, np.uint16)
        load().lko_xs_fill_attn_case(ctypes.byref(self.state), cache_elems, _p(q), _p(kc), _p(vc))
        return q, kc, vc


def sm64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of the splitmix64 stream of `seed`."""
    out = np.empty(n, np.uint64)
    load().lko_sm64_n(seed, _p(out), n)
    return out


def sm_normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().lko_sm_normal(seed, _p(out), n)
    return out


def sm_uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().lko_sm_uniform(seed, _p(out), n, lo, hi)
    return out


def sm_student4(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().lko_sm_student4(seed, _p(out), n)
    return out


def mt_prefill_case(seed: int, m: int, P: int, koff: float = 0.0, with_off: bool = False):
    S = P + m
    K = np.empty(S * 512, np.uint16)
    V = np.empty(S * 512, np.uint16)
    Q = np.empty(m * 2048, np.uint16)
    load().lko_mt_prefill_case(seed, m, P, koff, int(with_off), _p(K), _p(V), _p(Q))
    return K, V, Q


def dot_q4_0_q8_1(qs16: np.ndarray, d: int, xq36: np.ndarray) -> float:
    """One Q4_0 x Q8_1 block dot (reference quant.cuh:131-158), fp32."""
    qs16 = np.ascontiguousarray(qs16, np.uint8)
    xq36 = np.ascontiguousarray(xq36, np.uint8)
    assert qs16.size == 16 and xq36.size == 36
    return float(load().lko_dot_q4_0_q8_1(_p(qs16), int(d), _p(xq36)))


def gemv_q4_0(qs, d, xq, rows, bpr, y=None, add=False, ssq=None, eps=1e-5) -> np.ndarray:
    """Q4_0 GEMV (reference k_gemv_q4_0): qs uint8 [rows][bpr][16], d uint16
    [rows][bpr], xq uint8 [bpr][36]; returns y float32 [rows]."""
    qs = np.ascontiguousarray(qs, np.uint8)
    d = np.ascontiguousarray(d, np.uint16)
    xq = np.ascontiguousarray(xq, np.uint8)
    assert qs.size == rows * bpr * 16 and d.size == rows * bpr and xq.size == bpr * 36
    out = np.zeros(rows, np.float32) if y is None else np.array(y, np.float32).copy()
    s = None if ssq is None else np.ascontiguousarray(ssq, np.float32)
    load().lko_gemv_q4_0(_p(qs), _p(d), _p(xq), rows, bpr, _p(s), float(eps), _p(out), int(add))
    return out


def pf_gemm_q4_0(qs, d, N, bpr, aqs, asc, ntok, scale=None, out=None, out_ld=None, add=False) -> np.ndarray:
    """Q4_0 x planar Q8_1 GEMM (reference k_pf_mmq EPI 0): qs uint8 [N][bpr][16],
    d uint16 [N][bpr], aqs int8 [ntok][bpr*32], asc float32 [ntok][bpr][2];
    returns out float32 [ntok][out_ld]."""
    out_ld = N if out_ld is None else out_ld
    qs = np.ascontiguousarray(qs, np.uint8); d = np.ascontiguousarray(d, np.uint16)
    aqs = np.ascontiguousarray(aqs, np.int8); asc = np.ascontiguousarray(asc, np.float32)
    assert qs.size == N * bpr * 16 and d.size == N * bpr and aqs.size >= ntok * bpr * 32 and asc.size >= ntok * bpr * 2
    o = np.zeros((ntok, out_ld), np.float32) if out is None else np.array(out, np.float32).reshape(ntok, out_ld).copy()
    sc = None if scale is None else np.ascontiguousarray(scale, np.float32)
    load().lko_pf_gemm_q4_0(_p(qs), _p(d), N, bpr, _p(aqs), _p(asc), ntok, _p(sc), _p(o), out_ld, int(add))
    return o


def quantize_q8_1_blocks(x: np.ndarray) -> np.ndarray:
    """fp32 [32 * n] -> Q8_1 blocks uint8 [n][36] (reference quant.cuh:106-121)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    return np.stack([quantize_q8_1(r) for r in x])


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """max|a-b| / max|b| (b = reference), NaN entries of b skipped."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    ok = ~np.isnan(b)
    a, b = a[ok], b[ok]
    r = np.max(np.abs(b)) if b.size else 0.0
    e = np.max(np.abs(a - b)) if b.size else 0.0
    return float(e / r) if r > 0 else float(e)
