"""The reference's own C++ runtime with its backend slot filled by this library.

oracle/Makefile compiles the reference's sources where they lie with
woodcock_amd/backends/hip_ops.cpp in place of src/backends/cpu_ops.cpp
(oracle/_ref/libwcref_hip.so, built where the reference checkout exists; the
built library travels).  The runtime's Drafter (src/core/drafter.cpp) then runs
every woodcock::ops call -- linear, rmsnorm, rope, silu_mul, attention,
softmax -- through wc_linear, wc_rmsnorm, wc_rope, wc_silu_mul, wc_attention
and wc_softmax on the GPU.  Each drafter golden fixture (recorded from the same
runtime on its CPU backend, tests/golden/make_golden.py) is replayed through it:
fuse, prefill, three fed-back chain steps with their head logits, a tree
forward with explicit positions and mask, the update pass and every cache row.
Tolerance: fp32 on both sides, so 2e-5 of each output's magnitude (summation
order only).  A shape the library rejects must surface as the runtime's own
exception, not as a wrong result.
"""
import numpy as np
import pytest

from conftest import load_golden
from drafter_replay import compare, fixture_config, fixture_weights, replay
from oracle import refcpp

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not refcpp.available(refcpp.HIP_LIB_PATH), reason="HIP-backend reference build absent"),
]

DRAFTER_FIXTURES = ["tiny", "tiny_prenorm", "tiny_window", "tiny_2layer", "mid"]


class RefAdapter:
    """The reference runtime's Drafter in the replay protocol (tests/drafter_replay.py)."""

    def __init__(self, cfg: dict, w: dict, lib_path):
        self.cfg = cfg
        self.d = refcpp.RefDrafter(cfg, w, lib_path=lib_path)

    def fuse(self, taps):
        return self.d.fuse(taps)

    def make_cache(self, cap):
        return self.d.make_cache()

    def forward(self, tokens, feat, cache, positions=None, mask=None):
        return self.d.forward(tokens, feat, cache, positions, mask)

    def feedback(self, hidden, out):
        return out if self.cfg.get("post_norm", True) else hidden

    def logits(self, out):
        return self.d.logits(out)

    def cache_rows(self, cache, layer):
        n = cache.size
        return cache.rows(layer, 0, n), cache.rows(layer, 1, n)


@pytest.mark.parametrize("name", DRAFTER_FIXTURES)
def test_reference_runtime_on_hip_backend_matches_cpu_goldens(name):
    z = load_golden(f"drafter_{name}.npz")
    ad = RefAdapter(fixture_config(z), fixture_weights(z), refcpp.HIP_LIB_PATH)
    try:
        res = replay(ad, z)
    finally:
        ad.d.close()
    compare(res, z, rtol=2e-5, what=f"reference runtime on the HIP backend/{name}")


def test_hip_backend_ops_against_cpu_backend_ops():
    """The single operations through both builds of the runtime's ops, on the
    same inputs: fp32 results within 2e-6 of their magnitude, softmax sums to one."""
    cpu, hip = refcpp.lib(refcpp.LIB_PATH), refcpp.lib(refcpp.HIP_LIB_PATH)
    rng = np.random.default_rng(3)
    P = lambda a: a.ctypes.data  # noqa: E731

    L, din, dout = 5, 96, 40
    x = rng.standard_normal((L, din)).astype(np.float32)
    W = rng.standard_normal((dout, din)).astype(np.float32)
    y0 = rng.standard_normal((L, dout)).astype(np.float32)
    outs = []
    for lib in (cpu, hip):
        y = y0.copy()
        assert lib.wcref_linear(P(x), L, din, P(W), dout, P(y), 1) == 0
        outs.append(y)
    assert np.abs(outs[1] - outs[0]).max() <= 2e-6 * np.abs(outs[0]).max()

    H, Hk, D, T = 4, 2, 16, 23
    q = rng.standard_normal((L, H, D)).astype(np.float32)
    K = rng.standard_normal((T, Hk, D)).astype(np.float32)
    V = rng.standard_normal((T, Hk, D)).astype(np.float32)
    mask = (rng.random((L, T)) < 0.7).astype(np.uint8)
    mask[:, 0] = 1
    outs = []
    for lib in (cpu, hip):
        o = np.empty((L, H, D), np.float32)
        assert lib.wcref_attention(P(q), L, H, Hk, D, P(K), P(V), T, P(mask), P(o), 0.25) == 0
        outs.append(o)
    assert np.abs(outs[1] - outs[0]).max() <= 2e-6 * np.abs(outs[0]).max()

    z0 = (rng.standard_normal(1000) * 4).astype(np.float32)
    outs = []
    for lib in (cpu, hip):
        z = z0.copy()
        assert lib.wcref_softmax(P(z), z.size) == 0
        outs.append(z)
    assert abs(float(outs[1].astype(np.float64).sum()) - 1.0) < 1e-5
    assert np.abs(outs[1] - outs[0]).max() <= 2e-6 * np.abs(outs[0]).max()
