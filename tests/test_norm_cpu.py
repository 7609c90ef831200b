"""Pins of the oracle's residual add + RMSNorm (oracle.add_rmsnorm, or_add_rmsnorm).

The reference's CPU branch is h = x.float() + delta.float(); F.rms_norm(h, (D,), w,
eps).to(out_dtype) (pygguf_engine/quant_kernels.py:1594-1596, :1548-1549): torch's own
library routine, against which the oracle is checked here, together with a float64
restatement, the reference's own known-answer check (tests/test_pygguf_engine.py:1313-1330,
restated), closed-form invariants, and a Python restatement of the documented summation
order.  A planted mistake (dropping the mean's 1/D) is shown to fail these checks.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _torch_ref(x, delta, w, eps, out_dtype):
    h = torch.from_numpy(x).float()
    if delta is not None:
        h = h + torch.from_numpy(delta).float()
    return h.numpy(), F.rms_norm(h, (x.shape[1],), torch.from_numpy(w), eps).to(out_dtype).numpy()


@pytest.mark.parametrize("R,D,xdt,ddt,eps", [(4, 256, np.float32, np.float16, 1e-6), (3, 2048, np.float32, np.float32, 1e-6),
                                             (2, 3584, np.float16, None, 1e-5), (5, 100, np.float32, np.float32, 1e-6),
                                             (1, 14336, np.float32, np.float32, 1e-6)])
def test_oracle_matches_torch_rms_norm(R, D, xdt, ddt, eps):
    rng = np.random.default_rng(R * D)
    x = (rng.standard_normal((R, D)) * 3).astype(xdt)
    delta = None if ddt is None else rng.standard_normal((R, D)).astype(ddt)
    w = (rng.standard_normal(D) * 0.5 + 1.0).astype(np.float32)
    for odt, tdt in ((np.float16, torch.float16), (np.float32, torch.float32)):
        h, out = oracle.add_rmsnorm(x, delta, w, eps, out_dtype=odt)
        rh, rout = _torch_ref(x, delta, w, eps, tdt)
        assert np.array_equal(h.view(np.uint32), rh.view(np.uint32))  # one fp32 rounding: exact
        if odt == np.float32:  # another summation order: a few fp32 ulps
            np.testing.assert_allclose(out, rout, rtol=4e-6, atol=1e-6)
        else:  # the same value up to where it rounds: at most one fp16 ulp apart
            ulp = np.spacing(np.abs(rout.astype(np.float32)).astype(np.float16)).astype(np.float32)
            assert np.all(np.abs(out.astype(np.float32) - rout.astype(np.float32)) <= ulp)
        # float64 restatement
        h64 = h.astype(np.float64)
        r64 = 1.0 / np.sqrt((h64 * h64).mean(axis=1, keepdims=True) + eps)
        np.testing.assert_allclose(out.astype(np.float64), h64 * r64 * w, rtol=2e-3 if odt == np.float16 else 2e-6,
                                   atol=1e-6)


def test_reference_known_answer_restated():
    """The reference's own check of its fused kernel (x fp32 [4, 256], delta fp16,
    w ~ N(1, 0.5)): |h - ref| < 1e-6, |out - ref| <= 1e-3 against F.rms_norm."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 256, dtype=torch.float32, generator=g).numpy()
    d = torch.randn(4, 256, dtype=torch.float16, generator=g).numpy()
    w = (torch.randn(256, dtype=torch.float32, generator=g) * 0.5 + 1.0).numpy()
    h, out = oracle.add_rmsnorm(x, d, w, 1e-6)
    rh, rout = _torch_ref(x, d, w, 1e-6, torch.float16)
    assert np.abs(h - rh).max() < 1e-6
    assert np.abs(out.astype(np.float32) - rout.astype(np.float32)).max() <= 1e-3


def test_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 1024)).astype(np.float32)
    ones = np.ones(1024, np.float32)
    # unit weight: every output row has mean square 1 (eps = 0)
    _, out = oracle.add_rmsnorm(x, None, ones, 0.0, out_dtype=np.float32)
    np.testing.assert_allclose((out.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-6)
    # homogeneous of degree 0 (eps = 0): scaling the row by 4 (exact in binary) changes no bit
    _, o1 = oracle.add_rmsnorm(x, None, ones, 0.0, out_dtype=np.float32)
    _, o4 = oracle.add_rmsnorm(x * np.float32(4.0), None, ones, 0.0, out_dtype=np.float32)
    assert np.array_equal(o1.view(np.uint32), o4.view(np.uint32))
    # the residual add: (x, delta) equals (x + delta, None) on fp32 inputs
    d = rng.standard_normal((3, 1024)).astype(np.float32)
    h, a = oracle.add_rmsnorm(x, d, ones, 1e-6)
    _, b = oracle.add_rmsnorm(x + d, None, ones, 1e-6)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16)) and np.array_equal(h, x + d)
    # bf16 inputs are the high halves of fp32
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    _, ob = oracle.add_rmsnorm(xb, None, ones, 1e-6, out_dtype=np.float32, bf16=(True, False))
    _, of = oracle.add_rmsnorm((xb.astype(np.uint32) << 16).view(np.float32), None, ones, 1e-6, out_dtype=np.float32)
    assert np.array_equal(ob, of)


def _restated_order(h_row: np.ndarray) -> np.float32:
    """The documented summation order, in numpy fp32 scalars."""
    f = np.float32
    D = len(h_row)
    slots = []
    for t in range(256):
        acc = f(0.0)
        for c in range(t, D // 4, 256):
            for i in range(4):
                v = h_row[4 * c + i]
                acc = f(acc + f(v * v))
        slots.append(acc)
    tot = None
    for wv in range(4):
        p = slots[64 * wv:64 * wv + 64]
        s = 32
        while s >= 1:
            for j in range(s):
                p[j] = f(p[j] + p[j + s])
            s //= 2
        tot = p[0] if tot is None else f(tot + p[0])
    return tot


def test_documented_summation_order():
    rng = np.random.default_rng(2)
    for D in (2048, 3584, 100):
        x = (rng.standard_normal((1, D)) * 7).astype(np.float32)
        w = np.ones(D, np.float32)
        _, out = oracle.add_rmsnorm(x, None, w, 1e-6, out_dtype=np.float32)
        tot = _restated_order(x[0])
        r = np.float32(1.0) / np.sqrt(np.float32(tot / np.float32(D) + np.float32(1e-6)))
        assert np.array_equal(out[0].view(np.uint32), (x[0] * r).astype(np.float32).view(np.uint32))


def test_planted_mistake_is_caught():
    """A restatement that forgets the mean's 1/D (a plausible slip) fails the torch check."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    w = np.ones(512, np.float32)
    _, bad = oracle.add_rmsnorm(x, None, w, 1e-6, out_dtype=np.float32)
    bad = bad / np.sqrt(np.float32(512))  # what sum instead of mean gives
    _, ref = _torch_ref(x, None, w, 1e-6, torch.float32)
    assert not np.allclose(bad, ref, rtol=4e-6, atol=1e-6)
