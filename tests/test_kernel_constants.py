"""CPU checks of numeric constants the HIP kernels ship, read from their source: the tanh
polynomial of the D=256 softcap loop (flash-attention-rdna2_amd/csrc/fwd_kernel.hpp).

The kernel forms logit = c * tanh(y), y = scale * s / c, as y * P(y^2) (odd degree 7) while
every |y| of a 32-key block is within kPolyY, and by 1 - 2 / (exp(2y) + 1) otherwise. These
tests pin the polynomial against tanh itself (numpy, float64) over the whole range, evaluated
in fp32 as the kernel does, and against the error of the exact form it replaces."""
import pathlib
import re

import numpy as np

SRC = pathlib.Path(__file__).resolve().parents[1] / "flash-attention-rdna2_amd" / "csrc" / "fwd_kernel.hpp"


def _shipped():
    s = SRC.read_text()
    y0 = float(re.search(r"constexpr float kPolyY = ([0-9.]+)f;", s).group(1))
    num = r"(-?[0-9.]+(?:e-?[0-9]+)?)f \* lcap"
    m = re.search(r"pa1 = " + num + r", pa3 = " + num + r";\s*const float pa5 = " + num + r", pa7 = " + num, s)
    assert m, "polynomial coefficients not found in fwd_kernel.hpp"
    return y0, [np.float32(float(x)) for x in m.groups()]


def _poly32(y, c):
    y = y.astype(np.float32)
    y2 = y * y
    return y * (c[0] + y2 * (c[1] + y2 * (c[2] + y2 * c[3])))


def test_softcap_polynomial_error_bound():
    y0, c = _shipped()
    assert 0.0 < y0 <= 0.5
    y = np.linspace(-y0, y0, 800001).astype(np.float32)
    err = np.abs(_poly32(y, c).astype(np.float64) - np.tanh(y.astype(np.float64)))
    assert err.max() <= 6e-8, f"max |P - tanh| = {err.max():.3e} on |y| <= {y0}"
    # odd and monotone on the range (a dropped or sign-flipped term breaks one of these)
    p = _poly32(y, c)
    assert np.array_equal(p, -_poly32(-y, c))
    assert (np.diff(p.astype(np.float64)) >= 0).all()


def test_softcap_polynomial_beats_the_exact_form():
    """The form it replaces, 1 - 2/(exp(2y)+1) in fp32, loses digits to cancellation near 0; the
    polynomial is at least as accurate everywhere on the range."""
    y0, c = _shipped()
    y = np.linspace(-y0, y0, 200001).astype(np.float32)
    ref = np.tanh(y.astype(np.float64))
    e = np.exp(np.float32(2) * y).astype(np.float32)
    exact_form = (np.float32(1) - np.float32(2) / (e + np.float32(1))).astype(np.float32)
    err_exact = np.abs(exact_form.astype(np.float64) - ref).max()
    err_poly = np.abs(_poly32(y, c).astype(np.float64) - ref).max()
    assert err_poly < err_exact, (err_poly, err_exact)


def test_softcap_polynomial_range_edge():
    """Just past the range the polynomial drifts from tanh: the switch to the exact form there
    is needed, and the bound holds up to the edge itself."""
    y0, c = _shipped()
    edge = np.array([y0], dtype=np.float32)
    assert abs(float(_poly32(edge, c)[0]) - np.tanh(float(edge[0]))) <= 6e-8
    far = np.array([4 * y0], dtype=np.float32)
    assert abs(float(_poly32(far, c)[0]) - np.tanh(float(far[0]))) > 1e-4
