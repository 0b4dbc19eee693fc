"""The device generator of the benchmark configurations (lk_synth_f32) draws
the same values as the oracle's sequential splitmix64 + Box-Muller streams
(whose integers are pinned by the published splitmix64 test vector in
tests/test_oracle.py).  Bit for bit, except where the device's and the host's
float64 log / cos / sin differ in the last place and the fp32 rounding falls
on the other side (a handful in a million at most)."""
import numpy as np
import pytest
import torch

from gpu_util import host, note

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind,seed,n", [(0, 12345, 100003), (0, 0x5EED020000000102, 4096), (1, 777, 50001),
                                         (2, 4242, 30001)])
def test_synth_matches_host_stream(lk, oracle, kind, seed, n):
    note(f"lk_synth_f32 kind {kind} seed {seed:#x} n {n}")
    out = torch.full((n,), float("nan"), device="cuda")
    lk.synth(kind, seed, out, 0.5, 2.0)
    torch.cuda.synchronize()
    got = host(out)
    want = {0: lambda: oracle.sm_normal(seed, n), 1: lambda: oracle.sm_uniform(seed, n, 0.5, 2.0),
            2: lambda: oracle.sm_student4(seed, n)}[kind]()
    same = got.view(np.uint32) == want.view(np.uint32)
    note(f"  {int((~same).sum())} of {n} differ")
    assert (~same).sum() <= max(2, n // 100000)
    assert np.allclose(got, want, rtol=2e-7, atol=0)


def test_configs_are_the_seeded_streams(lk, oracle):
    """C4's V is exactly the normal stream of its seed, rounded to fp16."""
    import lk_configs
    qh, kc, vc, S = lk_configs.prefill_inputs("C4")
    want = oracle.sm_normal(lk_configs.seed_of("C4", 0, lk_configs.T_V, 2), 4096)
    got = vc.reshape(-1)[:4096].float().cpu().numpy()
    assert np.mean(got == want.astype(np.float16).astype(np.float32)) > 0.999
