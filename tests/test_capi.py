"""The C-ABI library loads and exports every entry point include/lk_attn.h
declares; host-side argument checks reject bad calls without launching.
CPU only: no kernel is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "lk_attn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lk_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    import lk_attn
    assert _declared() == sorted(lk_attn.EXPORTS)


def test_library_exports_every_declared_symbol():
    import lk_attn
    lib = ctypes.CDLL(lk_attn.LIB_PATH)
    missing = [s for s in _declared() if not hasattr(lib, s)]
    assert not missing, missing


def test_rope_frequency_constants_match_host_pow():
    """The producers' rotary frequencies are compile-time constants; they must be
    (float) pow(1e7, -i/32) evaluated in fp64 and rounded once, the formula the
    oracle evaluates with the host's pow (Python's math.pow is the same C pow)."""
    import math
    import numpy as np
    import lk_attn
    lib = ctypes.CDLL(lk_attn.LIB_PATH)
    lib.lk_rope_freq_table.argtypes = [ctypes.c_void_p]
    out = np.zeros(32, dtype=np.float32)
    assert lib.lk_rope_freq_table(out.ctypes.data_as(ctypes.c_void_p)) == 0
    want = np.array([math.pow(10000000.0, -i / 32.0) for i in range(32)]).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    assert out[0] == 1.0 and np.all(np.diff(out) < 0)
    assert lib.lk_rope_freq_table(None) != 0


def test_config_and_part_size():
    import lk_attn
    c = lk_attn.config()
    assert c["split_min"] >= 1 and c["target_n"] >= 16 and c["split_cap"] >= c["split_min"]
    assert lk_attn.part_bytes() == 32 * c["split_cap"] * lk_attn.PARTW * 4


def test_slice_rule_binding_matches_oracle(oracle):
    import lk_attn
    c = lk_attn.config()
    for seq in [1, 5, 100, 513, 4096, 32768, 100003, 131072]:
        assert lk_attn.attn_slices(seq) == oracle.attn_slices(seq, c["split_cap"], c["target_n"], c["split_min"])


def test_host_argument_errors():
    import lk_attn
    lib = lk_attn.load()
    p = ctypes.c_void_p(0x1000)      # never dereferenced: every call below fails validation
    assert lib.lk_attn_split(None, p, p, p, p, None) == 1
    assert b"null" in lib.lk_last_error()
    assert lib.lk_attn_combine(None, p, None, None, None) == 1
    assert lib.lk_pf_k8(p, 0, 10, None, 6, p, p, None) == 1            # kstride not a multiple of 4
    assert b"kstride" in lib.lk_last_error()
    assert lib.lk_pf_k8(p, 5, 3, None, 8, p, p, None) == 1             # p1 < p0
    assert lib.lk_pf_attn8(p, p, p, p, 10, 0, p, p, 8, p, p, 0, 0, p, None) == 1   # kstride < P+m
    assert lib.lk_pf_qk_i32(p, 17, p, 16, p, None) == 1
    assert lib.lk_pf_kmean(p, 0, p, None) == 1
    assert lib.lk_qk_norm_rope(None, p, p, p, p, p, p, p, None) == 1
    assert lib.lk_pf_qknr(p, p, p, 4, 0, p, p, p, p, None, 8, None, None) == 1        # k8 without ksc
    assert lib.lk_pf_qknr(p, p, p, 4, 0, p, p, p, p, p, 6, None, None) == 1          # kstride % 4
    assert lib.lk_pf_qknr(None, None, None, 0, 0, None, None, None, None, None, 0, None, None) == 0
    q = ctypes.c_void_p(0x1008)      # 8-byte aligned only: the producers load and store 16 bytes
    assert lib.lk_qk_norm_rope(p, p, p, q, p, p, p, p, None) == 1
    assert b"16-byte" in lib.lk_last_error()
    assert lib.lk_pf_qknr(q, p, p, 4, 0, p, p, p, None, None, 0, None, None) == 1
    assert b"misaligned" in lib.lk_last_error()
    assert lib.lk_pf_qknr(p, p, p, 4, 0, p, p, p, ctypes.c_void_p(0x1004), p, 8, None, None) == 1   # k8 8 B
    hc = ctypes.c_void_p()
    assert lib.lk_pf_ctx_create(0, 16, 64, 1, 0, 0, 0, ctypes.byref(hc)) == 1
    assert lib.lk_pf_ctx_create(1, 128, 64, 1, 0, 0, 0, ctypes.byref(hc)) == 1    # max_seq < max_chunk
    assert lib.lk_pf_chunk_attn(None, 0, p, p, p, 4, 0, p, p, p, None, None, None) == 1
    assert lib.lk_pf_attn8_q81(p, p, p, p, 4, 0, p, p, 8, p, p, 0, 0, None, p, None, None) == 1  # asc missing
    assert lib.lk_pf_quant_rows(p, 2, 16, 1, p, p, None) == 1                                  # ld < 32 kb
    assert lib.lk_pf_quant_rows(None, 0, 64, 2, None, None, None) == 0
    assert lib.lk_pf_chunk_done(None, 4) == 1
    assert lib.lk_pf_ctx_destroy(None) == 0
    assert lib.lk_pf_split_override(-2) == 1
    assert lib.lk_pf_split_override(0) == 0
    # empty work is a successful no-op
    assert lib.lk_pf_q8(None, 0, None, None, None, None, None) == 0
    assert lib.lk_pf_attn(None, 0, 0, None, None, None, None) == 0
    assert lib.lk_pf_k8(None, 4, 4, None, 8, None, None, None) == 0
    h = ctypes.c_void_p()
    assert lib.lk_decode_graph_create(0, None, None, None, None, None, None, None, p, ctypes.byref(h)) == 1
    assert lib.lk_decode_graph_launch(None, None) == 1
    assert lib.lk_decode_graph_destroy(None) == 0
    assert lib.lk_decode_step_graph_create(0, None, p, p, p, ctypes.byref(h)) == 1
    assert lib.lk_decode_graph_run(None, 1, None) == 1
    assert lib.lk_read_probe(None, 64, p, None) == 1
    assert lib.lk_read_probe(p, 24, p, None) == 1                         # not a multiple of 16
    assert lib.lk_pf_plan_items(0, 0, 0, 0, 1, None, 0) == -1
    assert lib.lk_pf_plan_items(64, 0, 0, 0, 1, None, 4) == -1            # items NULL with room
    assert lib.lk_pf_plan_items(64, 0, 0, 0, 1, None, 0) == 0             # one block: unsplit
    F = ctypes.c_float
    assert lib.lk_gemv_q4_0(None, p, p, 8, 64, p, 0, None, F(1e-5), None) == 1        # null qs
    assert lib.lk_gemv_q4_0(p, p, p, 8, 0, p, 0, None, F(1e-5), None) == 1            # bpr < 1
    assert lib.lk_gemv_q4_0(p, p, p, 8, 257, p, 0, None, F(1e-5), None) == 1          # bpr > 256
    assert lib.lk_gemv_q4_0(p, p, p, -1, 64, p, 0, None, F(1e-5), None) == 1          # rows < 0
    q = ctypes.c_void_p(0x1008)                                                        # not 16-byte aligned
    assert lib.lk_gemv_q4_0(q, p, p, 8, 64, p, 0, None, F(1e-5), None) == 1
    assert lib.lk_gemv_q4_0(p, p, p, 8, 64, p, 0, ctypes.c_void_p(0x1002), F(1e-5), None) == 1  # ssq
    assert lib.lk_gemv_q4_0(None, None, None, 0, 64, None, 0, None, F(1e-5), None) == 0  # no rows
    assert lib.lk_pf_gemm_q4_0(p, p, 100, 64, p, p, 4, None, p, 128, 0, None) == 1   # N % 64
    assert lib.lk_pf_gemm_q4_0(p, p, 128, 64, p, p, 4, None, p, 64, 0, None) == 1    # out_ld < N
    assert lib.lk_pf_gemm_q4_0(p, p, 128, 0, p, p, 4, None, p, 128, 0, None) == 1    # bpr < 1
    assert lib.lk_pf_gemm_q4_0(p, p, 128, 12, p, p, 4, None, p, 128, 0, None) == 1   # bpr % 8
    assert lib.lk_pf_gemm_q4_0(p, None, 128, 64, p, p, 4, None, p, 128, 0, None) == 1  # null d
    assert lib.lk_pf_gemm_q4_0(q, p, 128, 64, p, p, 4, None, p, 128, 0, None) == 1   # qs misaligned
    # every operand is checked at the width the kernel loads it with
    assert lib.lk_pf_gemm_q4_0(p, ctypes.c_void_p(0x1004), 128, 64, p, p, 4, None, p, 128, 0, None) == 1  # d: 8 B
    assert lib.lk_pf_gemm_q4_0(p, p, 128, 64, q, p, 4, None, p, 128, 0, None) == 1   # aqs: 16 B
    assert lib.lk_pf_gemm_q4_0(p, p, 128, 64, p, q, 4, None, p, 128, 0, None) == 1   # asc: 16 B
    assert b"misaligned" in lib.lk_last_error()
    assert lib.lk_pf_gemm_q4_0(None, None, 128, 64, None, None, 0, None, None, 128, 0, None) == 0  # no tokens
    assert lib.lk_pf_gemm_q4_0(p, p, 128, 2048, p, p, 65536, None, p, 128, 0, None) == 1  # 4 GiB of activations
    assert b"4 GiB" in lib.lk_last_error()
    # the decode split reads q with 16-byte loads: every entry point that runs it checks q
    assert lib.lk_attn_split(q, p, p, p, p, None) == 1
    assert b"16-byte" in lib.lk_last_error()
    assert lib.lk_attn_decode(q, p, p, p, p, p, None, None) == 1
    assert b"16-byte" in lib.lk_last_error()
    assert lib.lk_attn_decode_noalloc(q, p, p, p, p, None, None) == 1
    assert b"16-byte" in lib.lk_last_error()
    assert lib.lk_decode_graph_create(1, ctypes.byref(q), ctypes.byref(p), ctypes.byref(p), p, p, None, None,
                                      p, ctypes.byref(h)) == 1
    assert b"16-byte" in lib.lk_last_error()
    # prefill workspaces are 16-byte aligned; their size is the static scratch's
    S = ctypes.c_size_t
    assert lib.lk_pf_attn8_ws(p, p, p, p, 4, 0, p, p, 8, p, p, 0, 0, p, None, None, q, S(4096), None) == 1
    assert b"workspace" in lib.lk_last_error()
    assert lib.lk_pf_attn_ws(p, 4, 0, p, p, p, None, None, q, S(4096), None) == 1
    assert lib.lk_pf_attn_ws(None, 0, 0, None, None, None, None, None, None, S(0), None) == 0
    assert lib.lk_pf_part_bytes() == 64 << 20
    assert lib.lk_pf_gsync_limit(-1) == 1
    assert lib.lk_pf_gsync_limit(0) == 0
    assert lib.lk_pf_gsync_faults(None, 0) == 1


def test_python_mirror_fails_loudly_without_library(tmp_path):
    import importlib
    import lk_attn
    mod = importlib.reload(lk_attn)
    try:
        mod._lib = None
        with pytest.raises(FileNotFoundError):
            mod.load(str(tmp_path / "missing.so"))
    finally:
        importlib.reload(lk_attn)
