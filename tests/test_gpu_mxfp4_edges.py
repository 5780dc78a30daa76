"""Edge values of the MXFP4 format through the HIP matvec (GPU; run with -m gpu).

With x = e_j, a unit vector, wl_dequant_matvec_mxfp4 returns column j of the
dequantised matrix (1.0 splits exactly into the activation pieces 1, 0, 0, and
every other term is a product with an exact zero), so the kernel's dequant is
compared value for value with golden data:

* the reference's hand fixture (tools/glm_mxfp4_numpy.py:44-52);
* tests/golden/dequant_tf.npz (transformers' _convert_moe_packed_tensors), whose
  row 0 holds the E8M0 corners 1, 127, 200 and 254;
* closed-form blocks at E8M0 254 (the largest finite scale).

Known differences from the reference, pinned here and documented in the
header of windlass_amd/csrc/moe_decode.hip:
* a weight that overflows to inf (E8M0 254 and |e2m1| >= 2) makes its row NaN
  under a unit vector whose zero entries meet it — in the reference too
  (inf * 0 in its fp32 loop); where the reference's single product gives
  +-inf (the inf column itself, every other weight of the row finite), the
  kernel gives NaN, because the activation's zero low pieces also multiply it;
* bf16 subnormal weights (E8M0 1 with |e2m1| = 0.5, i.e. 2^-127) are produced
  exactly by the conversion and kept by the matrix cores (asserted below).
"""
import json
import os

import numpy as np
import pytest

from oracle import moe_oracle as O
from windlass_amd import moe

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _columns(hip, W, S, cols):
    """y[:, j] = W . e_j for j in cols, through wl_dequant_matvec_mxfp4."""
    N, K = W.shape[0], W.shape[1] * 2
    dW, dS = hip.DeviceBuffer.from_array(W), hip.DeviceBuffer.from_array(S)
    dx, dy = hip.DeviceBuffer(4 * K), hip.DeviceBuffer(4 * N)
    out = np.zeros((N, len(cols)), np.float32)
    for i, j in enumerate(cols):
        x = np.zeros(K, np.float32)
        x[j] = 1.0
        dx.upload(x)
        moe.dequant_matvec_mxfp4(dW.ptr, dS.ptr, dx.ptr, dy.ptr, N, K)
        hip.synchronize()
        out[:, i] = dy.download(np.float32)
    return out


def _same_values(got, exp):
    """Value equality with NaN == NaN (-0.0 == +0.0: the matvec sums exact
    zeros onto the product, which turns a -0.0 weight into +0.0)."""
    return np.array_equal(got, exp, equal_nan=True)


def test_hand_fixture_through_kernel(gpu):
    hip = gpu
    fx = json.load(open(os.path.join(GOLD, "mxfp4_hand_fixture.json")))
    W = np.zeros((16, 64), np.uint8)  # K = 128: one fixture block, three zero blocks
    S = np.full((16, 4), 127, np.uint8)
    W[0, :16] = fx["w"]
    S[0, 0] = fx["s"][0]
    y = _columns(hip, W, S, range(32))
    assert _same_values(y[0], np.array(fx["expected"], np.float32))
    assert not y[1:].any()


def test_transformers_fixture_through_kernel(gpu):
    """Rows 1..15 (scales 118..134) equal transformers' dequant exactly. Row 0
    carries an E8M0-254 block with |e2m1| >= 2 values (inf): every unit vector
    meets an inf with a zero, so the whole row is NaN, as in the reference."""
    hip = gpu
    fx = np.load(os.path.join(GOLD, "dequant_tf.npz"))
    W, S, exp = fx["w"], fx["s"], fx["expected"]
    assert list(S[0, :4]) == [1, 127, 200, 254] and np.isinf(exp[0]).sum() >= 2
    y = _columns(hip, W, S, range(W.shape[1] * 2))
    assert _same_values(y[1:], exp[1:])
    assert np.isnan(y[0]).all()


def test_corner_scales_without_overflow(gpu):
    """Row 0 = the fixture's blocks at E8M0 1, 127, 200 (block 3 zeroed): every
    value, the bf16 subnormals 2^-127 of the E8M0-1 block included, equals
    transformers' dequant."""
    hip = gpu
    fx = np.load(os.path.join(GOLD, "dequant_tf.npz"))
    W = fx["w"][:, :64].copy()
    S = fx["s"][:, :4].copy()
    exp = fx["expected"][:, :128].copy()
    W[0, 48:64] = 0
    S[0, 3] = 127
    exp[0, 96:128] = 0.0
    sub = (exp[0] != 0) & (np.abs(exp[0]) < np.float32(2.0 ** -126))
    assert sub.sum() >= 1  # the fixture holds subnormal results at E8M0 1
    y = _columns(hip, W, S, range(128))
    kept = int((y[0][sub] == exp[0][sub]).sum())
    print(f"E8M0=1 subnormals: {kept} of {int(sub.sum())} kept exactly", flush=True)
    assert _same_values(y, exp)


def test_largest_finite_scale(gpu):
    """E8M0 254 with |e2m1| <= 1.5: finite values up to 1.5 * 2^127, exact."""
    hip = gpu
    rng = np.random.default_rng(254)
    small = np.array([0, 1, 2, 3, 8, 9, 10, 11], np.uint8)  # |e2m1| <= 1.5
    lo = rng.choice(small, size=(16, 64))
    hi = rng.choice(small, size=(16, 64))
    W = (lo | (hi << 4)).astype(np.uint8)
    S = rng.integers(120, 130, size=(16, 4), dtype=np.uint8)
    S[:, 2] = 254
    exp = O.dequant(W, S)
    assert np.isfinite(exp).all() and np.abs(exp).max() == np.float32(1.5 * 2.0 ** 127)
    y = _columns(hip, W, S, range(128))
    assert _same_values(y, exp)


def test_overflow_to_inf_gives_nan(gpu):
    """One weight 2.0 x 2^127 = inf alone in its row: the reference's product
    is inf; the kernel's is NaN (the zero low activation pieces multiply the
    inf too). Rows without the inf are unaffected."""
    hip = gpu
    W = np.zeros((16, 64), np.uint8)
    S = np.full((16, 4), 127, np.uint8)
    W[0, 40] = 0x04  # column 80 = e2m1 code 4 (2.0), low nibble
    S[0, 2] = 254
    W[1, 40] = 0x04  # same code at scale 127: 2.0
    exp = O.dequant(W, S)
    assert np.isinf(exp[0, 80]) and exp[1, 80] == 2.0
    y = _columns(hip, W, S, [80, 81])
    print(f"E8M0=254 overflow: kernel gives {y[0, 0]} where the reference gives {exp[0, 80]}", flush=True)
    assert np.isnan(y[0, 0])
    assert y[1, 0] == 2.0 and not y[2:].any()
    # a unit vector away from the inf column still meets inf * 0 = NaN (as in
    # the reference's fp32 loop)
    assert np.isnan(y[0, 1])
