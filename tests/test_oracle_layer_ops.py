"""Pins of the oracle's decoder-layer elementwise ops (fused into GEMV plans): rmsnorm, SwiGLU, GeGLU.

Checks that do not restate the formulas:
- rmsnorm: with unit gain the output's mean square is 1 / (1 + eps / ms(x)); positive scaling of x
  leaves it unchanged when eps = 0; the one-plus convention with w equals the plain one with 1 + w;
  rows are independent;
- SiLU / tanh-GELU: odd-part identity act(v) - act(-v) = v (both are v * sigmoid-like(v) with
  s(v) + s(-v) = 1), act(0) = 0, act(v) -> v for large v and -> 0 for large -v, monotone for v >= 0.
"""
import numpy as np

from oracle import brik_oracle as O


def test_rmsnorm_unit_gain_mean_square():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(3 * 64).astype(np.float32)
    y = O.rmsnorm(x, np.ones(64, np.float32), 3, 64, eps=0.0).reshape(3, 64)
    np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(1), 1.0, rtol=1e-6)
    eps = 0.5
    y = O.rmsnorm(x, np.ones(64, np.float32), 3, 64, eps=eps).reshape(3, 64)
    ms = (x.reshape(3, 64).astype(np.float64) ** 2).mean(1)
    np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(1), ms / (ms + eps), rtol=1e-6)


def test_rmsnorm_scale_invariance_and_conventions():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(128).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    a = O.rmsnorm(x, w, 1, 128, eps=0.0)
    b = O.rmsnorm(np.float32(8.0) * x, w, 1, 128, eps=0.0)
    np.testing.assert_allclose(a, b, rtol=1e-6)
    c = O.rmsnorm(x, w, 1, 128, eps=1e-5, one_plus=True)
    d = O.rmsnorm(x, (1.0 + w.astype(np.float64)).astype(np.float32), 1, 128, eps=1e-5)
    np.testing.assert_allclose(c, d, rtol=1e-6)
    two = O.rmsnorm(np.concatenate([x, 3 * x]), w, 2, 128, eps=0.0).reshape(2, 128)
    np.testing.assert_allclose(two[0], two[1], rtol=1e-6)


def test_gated_activations():
    v = np.linspace(-30, 30, 6001).astype(np.float32)
    one = np.ones_like(v)
    for f in (O.swiglu, O.geglu):
        a, b = f(v, one).astype(np.float64), f(-v, one).astype(np.float64)
        np.testing.assert_allclose(a - b, v, atol=2e-5)
        assert f(np.zeros(1, np.float32), np.ones(1, np.float32))[0] == 0.0
        assert abs(f(np.float32([30.0]), np.float32([1.0]))[0] - 30.0) < 1e-4
        assert abs(f(np.float32([-30.0]), np.float32([1.0]))[0]) < 1e-4
        pos = f(v[v >= 0], one[v >= 0])
        assert np.all(np.diff(pos.astype(np.float64)) >= 0)
    # the up factor multiplies
    np.testing.assert_allclose(O.swiglu(v, 2 * one), 2 * O.swiglu(v, one), rtol=1e-6)


def test_gated_activations_against_torch():
    """SiLU and tanh-GELU against independent implementations (torch, computed in float64): a wrong
    slope (e.g. sigmoid(2v)), erf-GELU in place of the reference's tanh form, or a wrong cubic
    coefficient each miss these by far more than the tolerance, which only covers the float32 store."""
    torch = __import__("pytest").importorskip("torch")
    v = np.linspace(-12, 12, 4801).astype(np.float32)
    up = np.random.default_rng(7).standard_normal(v.size).astype(np.float32)
    tv, tu = torch.from_numpy(v.astype(np.float64)), torch.from_numpy(up.astype(np.float64))
    silu = (torch.nn.functional.silu(tv) * tu).numpy()
    gelu = (torch.nn.functional.gelu(tv, approximate="tanh") * tu).numpy()
    # atol: for v << 0 both evaluate 0.5 v (1 + tanh(u)) with 1 + tanh(u) cancelling to ~1e-16 noise
    for got, want in ((O.swiglu(v, up), silu), (O.geglu(v, up), gelu)):
        np.testing.assert_allclose(got.astype(np.float64), want, rtol=2e-7, atol=1e-12)
    # the two forms the tests above cannot tell apart from the reference's: erf-GELU differs here
    erf = (torch.nn.functional.gelu(tv, approximate="none") * tu).numpy()
    assert np.abs(O.geglu(v, up).astype(np.float64) - erf).max() > 1e-4
