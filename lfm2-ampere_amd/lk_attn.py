"""Python host mirror of the attention entry points (ctypes over liblk_attn.so).

The reference engine is C++ and launches its attention kernels directly
(/root/reference/src/engine.cu:638-641 for decode, :1082-1089 and :1122 for
prefill).  This module binds the C ABI of ``include/lk_attn.h`` under the
reference's kernel names (``attn_split`` for ``k_attn_split`` and so on) so
tests and the benchmark read like the reference's own harnesses.  PyTorch is
used only to own device memory and streams; every computation runs in the HIP
library.  There is no fallback: if the library is missing or fails, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblk_attn.so")

N_HEADS, N_KV_HEADS, HEAD_DIM = 32, 8, 64
PARTW = 4 + HEAD_DIM
DECODE_MAX_SEQ = 8192
Q8_1_BYTES = 36

# Every symbol the header declares; tests check the library exports them all.
EXPORTS = (
    "lk_attn_config", "lk_attn_part_bytes", "lk_last_error",
    "lk_attn_split", "lk_attn_combine", "lk_attn_decode", "lk_attention_decode",
    "lk_decode_graph_create", "lk_decode_graph_launch", "lk_decode_graph_nodes",
    "lk_decode_graph_destroy",
    "lk_pf_q8", "lk_pf_k8", "lk_pf_kmean", "lk_pf_attn8", "lk_pf_attn", "lk_pf_split_override", "lk_pf_pair_override",
    "lk_pf_qk_i32", "lk_pf_plan_items", "lk_read_probe", "lk_qk_norm_rope", "lk_pf_qknr",
    "lk_decode_step_graph_create", "lk_decode_graph_run",
    "lk_pf_ctx_create", "lk_pf_ctx_destroy", "lk_pf_chunk_attn", "lk_pf_chunk_done", "lk_pf_ctx_buffers",
    "lk_pf_attn8_q81", "lk_pf_attn_q81", "lk_pf_quant_rows", "lk_gemv_q4_0", "lk_pf_gemm_q4_0",
    "lk_attn_decode_noalloc", "lk_rope_freq_table",
    "lk_pf_part_bytes", "lk_pf_attn8_ws", "lk_pf_attn_ws", "lk_pf_gsync_limit", "lk_pf_gsync_faults",
    "lk_synth_f32",
)


class LkError(RuntimeError):
    """A C-ABI call returned a non-zero hipError_t."""


_lib: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load liblk_attn.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `make -C lfm2-ampere_amd` "
            "(or __graft_entry__.build()); there is no fallback path")
    # torch (whose tensors this module passes as device memory) carries its own
    # HIP runtime under the same soname; load it first so the process has one
    # runtime and torch's streams and allocations are valid for the library.
    import torch  # noqa: F401
    lib = ctypes.CDLL(path)
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    sig = {
        "lk_attn_config": ([P, P, P], I),
        "lk_attn_part_bytes": ([], S),
        "lk_rope_freq_table": ([P], I),
        "lk_last_error": ([], ctypes.c_char_p),
        "lk_attn_split": ([P, P, P, P, P, P], I),
        "lk_attn_combine": ([P, P, P, P, P], I),
        "lk_attn_decode": ([P, P, P, P, P, P, P, P], I),
        "lk_attn_decode_noalloc": ([P, P, P, P, P, P, P], I),
        "lk_attention_decode": ([P, P, P, P, P, P, P], I),
        "lk_decode_graph_create": ([I, P, P, P, P, P, P, P, P, P], I),
        "lk_decode_graph_launch": ([P, P], I),
        "lk_decode_graph_nodes": ([P, P], I),
        "lk_decode_graph_destroy": ([P], I),
        "lk_pf_q8": ([P, I, P, P, P, P, P], I),
        "lk_pf_k8": ([P, I, I, P, I, P, P, P], I),
        "lk_pf_kmean": ([P, I, P, P], I),
        "lk_pf_attn8": ([P, P, P, P, I, I, P, P, I, P, P, I, I, P, P], I),
        "lk_pf_attn": ([P, I, I, P, P, P, P], I),
        "lk_pf_split_override": ([I], I),
        "lk_pf_pair_override": ([I], I),
        "lk_pf_qk_i32": ([P, I, P, I, P, P], I),
        "lk_pf_plan_items": ([I, I, I, I, I, P, I], I),
        "lk_read_probe": ([P, S, P, P], I),
        "lk_gemv_q4_0": ([P, P, P, I, I, P, I, P, ctypes.c_float, P], I),
        "lk_pf_gemm_q4_0": ([P, P, I, I, P, P, I, P, P, I, I, P], I),
        "lk_qk_norm_rope": ([P, P, P, P, P, P, P, P, P], I),
        "lk_pf_qknr": ([P, P, P, I, I, P, P, P, P, P, I, P, P], I),
        "lk_decode_step_graph_create": ([I, P, P, P, P, P], I),
        "lk_decode_graph_run": ([P, I, P], I),
        "lk_pf_ctx_create": ([I, I, I, I, I, I, I, P], I),
        "lk_pf_ctx_destroy": ([P], I),
        "lk_pf_chunk_attn": ([P, I, P, P, P, I, I, P, P, P, P, P, P], I),
        "lk_pf_attn8_q81": ([P, P, P, P, I, I, P, P, I, P, P, I, I, P, P, P, P], I),
        "lk_pf_attn_q81": ([P, I, I, P, P, P, P, P, P], I),
        "lk_pf_quant_rows": ([P, I, I, I, P, P, P], I),
        "lk_pf_chunk_done": ([P, I], I),
        "lk_pf_ctx_buffers": ([P, I, P, P, P, P, P, P], I),
        "lk_pf_part_bytes": ([], S),
        "lk_pf_attn8_ws": ([P, P, P, P, I, I, P, P, I, P, P, I, I, P, P, P, P, S, P], I),
        "lk_pf_attn_ws": ([P, I, I, P, P, P, P, P, P, S, P], I),
        "lk_pf_gsync_limit": ([I], I),
        "lk_pf_gsync_faults": ([P, I], I),
        "lk_synth_f32": ([I, ctypes.c_uint64, S, ctypes.c_float, ctypes.c_float, P, P], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lk_last_error().decode(errors="replace")
        raise LkError(f"{what} failed (hipError {rc}): {msg}")


def _ptr(t) -> Optional[int]:
    """Device pointer of a tensor (None -> NULL).  Checks residency and layout."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("lk_attn: tensors must live in device memory")
    if not t.is_contiguous():
        raise ValueError("lk_attn: tensors must be contiguous")
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


def config() -> dict:
    a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(load().lk_attn_config(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)), "lk_attn_config")
    return {"split_cap": a.value, "target_n": b.value, "split_min": c.value}


def part_bytes() -> int:
    return int(load().lk_attn_part_bytes())


def attn_slices(seq: int) -> tuple:
    """The library's split-K slice rule (reference kernels.cuh:630-635)."""
    c = config()
    s = (seq + c["target_n"] - 1) // c["target_n"]
    s = max(c["split_min"], min(c["split_cap"], s))
    return s, (seq + s - 1) // s


# ---- decode (reference kernels.cuh:644-658) -------------------------------------
def attn_split(q, kc, vc, d_pos, part, stream=None) -> None:
    _check(load().lk_attn_split(_ptr(q), _ptr(kc), _ptr(vc), _ptr(d_pos), _ptr(part),
                                _stream(stream)), "lk_attn_split")


def attn_combine(part, d_pos, out=None, yq8=None, stream=None) -> None:
    _check(load().lk_attn_combine(_ptr(part), _ptr(d_pos), _ptr(out), _ptr(yq8),
                                  _stream(stream)), "lk_attn_combine")


def attn_decode(q, kc, vc, d_pos, part, out=None, yq8=None, stream=None) -> None:
    _check(load().lk_attn_decode(_ptr(q), _ptr(kc), _ptr(vc), _ptr(d_pos), _ptr(part),
                                 _ptr(out), _ptr(yq8), _stream(stream)), "lk_attn_decode")


def attn_decode_noalloc(q, kc, vc, d_pos, out=None, yq8=None, stream=None) -> None:
    """lk_attn_decode without a `part` workspace: the library's static
    per-device scratch holds the partials (calls overlapping on one GPU race)."""
    _check(load().lk_attn_decode_noalloc(_ptr(q), _ptr(kc), _ptr(vc), _ptr(d_pos),
                                         _ptr(out), _ptr(yq8), _stream(stream)), "lk_attn_decode_noalloc")


def attention_decode(q, kc, vc, d_pos, out=None, yq8=None, stream=None) -> None:
    _check(load().lk_attention_decode(_ptr(q), _ptr(kc), _ptr(vc), _ptr(d_pos), _ptr(out),
                                      _ptr(yq8), _stream(stream)), "lk_attention_decode")


class DecodeLayer(ctypes.Structure):
    """lk_decode_layer (include/lk_attn.h): one layer's buffers for the step graph."""
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("q_src", "k_src", "v_src", "q", "k", "q_norm", "k_norm", "kc", "vc", "out", "yq8",
                 "wo_qs", "wo_d", "x")]


class DecodeStepGraph:
    """The decode step's attention slice (per layer: qk norm + RoPE of the
    projection rows + cache append, split, combine; then d_pos += 1) captured
    into one hipGraph; run(n) replays it n times."""

    def __init__(self, layers: Sequence[dict], d_pos, part, stream=None):
        import torch
        n = len(layers)
        arr = (DecodeLayer * n)()
        for i, L in enumerate(layers):
            for f, _ in DecodeLayer._fields_:
                setattr(arr[i], f, _ptr(L.get(f)))
        self._keep = (layers, d_pos, part, arr)
        self._stream = stream if stream is not None else torch.cuda.Stream()
        h = ctypes.c_void_p()
        _check(load().lk_decode_step_graph_create(n, arr, _ptr(d_pos), _ptr(part),
                                                  self._stream.cuda_stream, ctypes.byref(h)),
               "lk_decode_step_graph_create")
        self._h = h

    @property
    def stream(self):
        return self._stream

    def nodes(self) -> int:
        n = ctypes.c_size_t()
        _check(load().lk_decode_graph_nodes(self._h, ctypes.byref(n)), "lk_decode_graph_nodes")
        return n.value

    def run(self, n_steps: int = 1) -> None:
        _check(load().lk_decode_graph_run(self._h, int(n_steps), self._stream.cuda_stream), "lk_decode_graph_run")

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().lk_decode_graph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DecodeGraph:
    """n_layers x (split, combine) captured into one hipGraph."""

    def __init__(self, qs: Sequence, kcs: Sequence, vcs: Sequence, d_pos, part,
                 outs: Optional[Sequence] = None, yq8s: Optional[Sequence] = None, stream=None):
        import torch
        n = len(qs)
        if not (len(kcs) == n and len(vcs) == n):
            raise ValueError("DecodeGraph: per-layer lists must have equal length")
        arr = ctypes.c_void_p * n
        self._keep = (qs, kcs, vcs, d_pos, part, outs, yq8s)
        self._stream = stream if stream is not None else torch.cuda.Stream()
        h = ctypes.c_void_p()
        o = arr(*[_ptr(t) for t in outs]) if outs is not None else None
        y = arr(*[_ptr(t) for t in yq8s]) if yq8s is not None else None
        _check(load().lk_decode_graph_create(
            n, arr(*[_ptr(t) for t in qs]), arr(*[_ptr(t) for t in kcs]),
            arr(*[_ptr(t) for t in vcs]), _ptr(d_pos), _ptr(part), o, y,
            self._stream.cuda_stream, ctypes.byref(h)), "lk_decode_graph_create")
        self._h = h

    @property
    def stream(self):
        return self._stream

    def nodes(self) -> int:
        n = ctypes.c_size_t()
        _check(load().lk_decode_graph_nodes(self._h, ctypes.byref(n)), "lk_decode_graph_nodes")
        return n.value

    def launch(self) -> None:
        _check(load().lk_decode_graph_launch(self._h, self._stream.cuda_stream), "lk_decode_graph_launch")

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().lk_decode_graph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- prefill (reference prefill.cuh:85-109) -------------------------------------
def pf_q8(qh, m, cm, q8, qsc, qcs, stream=None) -> None:
    _check(load().lk_pf_q8(_ptr(qh), m, _ptr(cm), _ptr(q8), _ptr(qsc), _ptr(qcs), _stream(stream)),
           "lk_pf_q8")


def pf_k8(kc, p0, p1, cm, kstride, k8, ksc, stream=None) -> None:
    _check(load().lk_pf_k8(_ptr(kc), p0, p1, _ptr(cm), kstride, _ptr(k8), _ptr(ksc), _stream(stream)),
           "lk_pf_k8")


def pf_kmean(kc, n, cm, stream=None) -> None:
    _check(load().lk_pf_kmean(_ptr(kc), n, _ptr(cm), _stream(stream)), "lk_pf_kmean")


def pf_attn8(q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, stream=None) -> None:
    """Int8-scored prefill attention (reference k_pf_attn8).  q8, qsc and qcs
    None: the kernel quantises qh itself (lk_pf_q8's arithmetic, no
    smoothing), with the same output as the two-kernel path."""
    _check(load().lk_pf_attn8(_ptr(q8), _ptr(qsc), _ptr(qcs), _ptr(qh), m, P, _ptr(k8), _ptr(ksc),
                              kstride, _ptr(kc), _ptr(vc), near, sink, _ptr(o), _stream(stream)),
           "lk_pf_attn8")


def pf_attn(qh, m, P, kc, vc, o, stream=None) -> None:
    _check(load().lk_pf_attn(_ptr(qh), m, P, _ptr(kc), _ptr(vc), _ptr(o), _stream(stream)), "lk_pf_attn")


def pf_attn8_q81(q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, aqs, asc, stream=None) -> None:
    _check(load().lk_pf_attn8_q81(_ptr(q8), _ptr(qsc), _ptr(qcs), _ptr(qh), int(m), int(P), _ptr(k8), _ptr(ksc),
                                  int(kstride), _ptr(kc), _ptr(vc), int(near), int(sink), _ptr(o), _ptr(aqs),
                                  _ptr(asc), _stream(stream)), "lk_pf_attn8_q81")


def pf_attn_q81(qh, m, P, kc, vc, o, aqs, asc, stream=None) -> None:
    _check(load().lk_pf_attn_q81(_ptr(qh), int(m), int(P), _ptr(kc), _ptr(vc), _ptr(o), _ptr(aqs), _ptr(asc),
                                 _stream(stream)), "lk_pf_attn_q81")


def pf_part_bytes() -> int:
    """Bytes of the largest split-K partial workspace a prefill launch uses."""
    return int(load().lk_pf_part_bytes())


def _nbytes(t) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def pf_attn8_ws(q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, aqs, asc, work,
                stream=None) -> None:
    """pf_attn8_q81 with a caller-owned split-K workspace (a device tensor; None:
    the library's static scratch)."""
    _check(load().lk_pf_attn8_ws(_ptr(q8), _ptr(qsc), _ptr(qcs), _ptr(qh), int(m), int(P), _ptr(k8), _ptr(ksc),
                                 int(kstride), _ptr(kc), _ptr(vc), int(near), int(sink), _ptr(o), _ptr(aqs),
                                 _ptr(asc), _ptr(work), _nbytes(work), _stream(stream)), "lk_pf_attn8_ws")


def pf_attn_ws(qh, m, P, kc, vc, o, aqs, asc, work, stream=None) -> None:
    _check(load().lk_pf_attn_ws(_ptr(qh), int(m), int(P), _ptr(kc), _ptr(vc), _ptr(o), _ptr(aqs), _ptr(asc),
                                _ptr(work), _nbytes(work), _stream(stream)), "lk_pf_attn_ws")


def pf_gsync_limit(polls: int) -> None:
    """Poll bound of the paired prefill kernel's group barriers (0: default)."""
    _check(load().lk_pf_gsync_limit(int(polls)), "lk_pf_gsync_limit")


def pf_gsync_faults(reset: bool = False) -> int:
    """Group barriers that gave up on this device since the last reset (synchronous)."""
    c = ctypes.c_uint()
    _check(load().lk_pf_gsync_faults(ctypes.byref(c), int(bool(reset))), "lk_pf_gsync_faults")
    return c.value


SYNTH_NORMAL, SYNTH_UNIFORM, SYNTH_STUDENT4 = 0, 1, 2


def synth(kind: int, seed: int, out, lo: float = 0.0, hi: float = 1.0, stream=None) -> None:
    """Fill the fp32 device tensor `out` with the seeded splitmix64 stream of
    `seed` (kind: SYNTH_NORMAL, SYNTH_UNIFORM in [lo, hi), SYNTH_STUDENT4)."""
    if out.dtype != __import__("torch").float32:
        raise ValueError("synth: out must be fp32")
    _check(load().lk_synth_f32(int(kind), int(seed) & ((1 << 64) - 1), out.numel(), float(lo), float(hi),
                               _ptr(out), _stream(stream)), "lk_synth_f32")


def pf_quant_rows(X, rows, ld, kb, qs, sc, stream=None) -> None:
    _check(load().lk_pf_quant_rows(_ptr(X), int(rows), int(ld), int(kb), _ptr(qs), _ptr(sc), _stream(stream)),
           "lk_pf_quant_rows")


def pf_pair_override(mode: int) -> None:
    """Paired prefill workgroups (blocks i and nq-1-i in one launch unit):
    -1 never, 0 automatic, 1 whenever the chunk has at least two 64-row blocks."""
    _check(load().lk_pf_pair_override(int(mode)), "lk_pf_pair_override")


def pf_split_override(tiles: int) -> None:
    """-1 never split prefill blocks, 0 automatic, n > 0 parts of <= n key tiles."""
    _check(load().lk_pf_split_override(int(tiles)), "lk_pf_split_override")


def read_probe(buf, sink, stream=None) -> None:
    """Plain streaming read of a device tensor (measurement reference)."""
    _check(load().lk_read_probe(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink),
                                _stream(stream)), "lk_read_probe")


def gemv_q4_0(qs, d, xq, out_rows: int, bpr: int, y, add_residual: bool = False, ssq=None,
              eps: float = 1e-5, stream=None) -> None:
    """Q4_0 x Q8_1 GEMV (reference k_gemv_q4_0): qs [out_rows][bpr] 16-byte
    blocks, d fp16 [out_rows][bpr], xq [bpr] Q8_1 blocks (36 bytes), y fp32
    [out_rows] (accumulated into when add_residual); ssq: 64 fp32 norm partials
    or None."""
    _check(load().lk_gemv_q4_0(_ptr(qs), _ptr(d), _ptr(xq), int(out_rows), int(bpr), _ptr(y),
                               int(bool(add_residual)), _ptr(ssq), float(eps), _stream(stream)),
           "lk_gemv_q4_0")


def pf_gemm_q4_0(qs, d, N: int, bpr: int, aqs, asc, ntok: int, out, out_ld: int = None,
                 add: bool = False, scale=None, stream=None) -> None:
    """Q4_0 x planar Q8_1 GEMM of a prefill chunk (reference pf_gemm_dense, one
    tensor, plain epilogue): out[t][r] (+)= scale[t] * W[r] . x[t]."""
    _check(load().lk_pf_gemm_q4_0(_ptr(qs), _ptr(d), int(N), int(bpr), _ptr(aqs), _ptr(asc), int(ntok),
                                  _ptr(scale), _ptr(out), int(N if out_ld is None else out_ld),
                                  int(bool(add)), _stream(stream)), "lk_pf_gemm_q4_0")


def pf_plan_items(m: int, P: int, near: int, sink: int, int8: bool = True, max_items: int = 1024):
    """The split work list of a prefill chunk, in dispatch order: a list of
    (query block, first key tile, end key tile, partial slot or -1); [] for an
    unsplit launch.  Host-side only."""
    import ctypes
    buf = (ctypes.c_int32 * (4 * max_items))()
    n = load().lk_pf_plan_items(int(m), int(P), int(near), int(sink), int(bool(int8)),
                                ctypes.addressof(buf), int(max_items))
    if n < 0:
        raise LkError("lk_pf_plan_items: bad arguments")
    return [tuple(buf[4 * i:4 * i + 4]) for i in range(min(n, max_items))]


def pf_qk_i32(q8, m, k8, n, s, stream=None) -> None:
    _check(load().lk_pf_qk_i32(_ptr(q8), m, _ptr(k8), n, _ptr(s), _stream(stream)), "lk_pf_qk_i32")


def kstride_for(S: int) -> int:
    """ksc row stride for S positions: rounded up to 4 (reference engine.cu:979)."""
    return (S + 3) & ~3


# ---- attention-input producers (reference kernels.cu:871-915, prefill.cu:975-1016) ----
def qk_norm_rope(qf, kf, vf, qn, kn, d_pos, kc, vc, stream=None) -> None:
    _check(load().lk_qk_norm_rope(_ptr(qf), _ptr(kf), _ptr(vf), _ptr(qn), _ptr(kn), _ptr(d_pos),
                                  _ptr(kc), _ptr(vc), _stream(stream)), "lk_qk_norm_rope")


def pf_qknr(Y, qn, kn, m, P, qh, kc, vc, k8=None, ksc=None, kstride=0, cm=None, stream=None) -> None:
    _check(load().lk_pf_qknr(_ptr(Y), _ptr(qn), _ptr(kn), int(m), int(P), _ptr(qh), _ptr(kc), _ptr(vc),
                             _ptr(k8), _ptr(ksc), int(kstride), _ptr(cm), _stream(stream)), "lk_pf_qknr")


class PrefillCtx:
    """lk_pf_ctx: the prefill chunk driver's state (int8 K copies, k8_valid)."""

    def __init__(self, n_layers, max_chunk, max_seq, attn8=True, ksmooth=False, near=1024, sink=1):
        h = ctypes.c_void_p()
        _check(load().lk_pf_ctx_create(int(n_layers), int(max_chunk), int(max_seq), int(bool(attn8)),
                                       int(bool(ksmooth)), int(near), int(sink), ctypes.byref(h)),
               "lk_pf_ctx_create")
        self._h = h

    def chunk_attn(self, layer, Y, qn, kn, m, pos0, kc, vc, o, aqs=None, asc=None, stream=None) -> None:
        _check(load().lk_pf_chunk_attn(self._h, int(layer), _ptr(Y), _ptr(qn), _ptr(kn), int(m), int(pos0),
                                       _ptr(kc), _ptr(vc), _ptr(o), _ptr(aqs), _ptr(asc), _stream(stream)),
               "lk_pf_chunk_attn")

    def chunk_done(self, pos_end) -> None:
        _check(load().lk_pf_chunk_done(self._h, int(pos_end)), "lk_pf_chunk_done")

    def buffers(self, layer) -> dict:
        qh, k8, ksc, cm = (ctypes.c_void_p() for _ in range(4))
        ks, kv = ctypes.c_int(), ctypes.c_int()
        _check(load().lk_pf_ctx_buffers(self._h, int(layer), ctypes.byref(qh), ctypes.byref(k8),
                                        ctypes.byref(ksc), ctypes.byref(cm), ctypes.byref(ks),
                                        ctypes.byref(kv)), "lk_pf_ctx_buffers")
        return {"qh": qh.value, "k8": k8.value, "ksc": ksc.value, "cm": cm.value,
                "kstride": ks.value, "k8_valid": kv.value}

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().lk_pf_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
