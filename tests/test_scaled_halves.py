"""wsp_encoder_scaled_halves on the CPU: a BF16 projection held as fp16
values w·2^k. The checks come from the number formats themselves: the
shift puts the largest magnitude in fp16's top binade [2^15, 2^16); every
value must come back bit for bit after dividing the scale out, and a value
whose last significand bit falls below fp16's smallest step (2^-24) after
the shift makes the tensor refuse."""

import ctypes

import numpy as np
import pytest

from helpers import ensure_library
from whispereacp_amd import _native as N
from whispereacp_amd import synthetic as S

WIDE = N.wsp_encoder_shape(128, 1280, 20, 1, 5120, 3000)


def convert(values, shape=WIDE, bits=None):
    lib = ensure_library()
    if bits is None:
        bits = S.f32_to_bf16_bits(np.asarray(values, dtype=np.float32))
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    halves = np.zeros(bits.shape, dtype=np.float16)
    scale = ctypes.c_float(-1.0)
    status = lib.wsp_encoder_scaled_halves(ctypes.byref(shape), bits.ctypes.data, bits.size, halves.ctypes.data,
                                           ctypes.byref(scale))
    return status, halves, scale.value, bits


def exact_back(halves, scale, bits):
    back = (halves.astype(np.float64) / scale).astype(np.float32)
    return np.array_equal(back.view(np.uint32), S.bf16_bits_to_f32(bits).view(np.uint32))


def test_normal_weights_narrow_exactly_with_the_top_binade_filled():
    values = np.random.default_rng(11).normal(0.0, 0.02, 200_000)
    status, halves, scale, bits = convert(values)
    assert status == N.WSP_OK
    mantissa, _ = np.frexp(scale)
    assert mantissa == 0.5  # a power of two
    top = np.max(np.abs(halves.astype(np.float64)))
    assert 2.0 ** 15 <= top < 2.0 ** 16 and np.isfinite(top)
    assert exact_back(halves, scale, bits)


def test_closed_form_values():
    # Largest magnitude 1.0: shift 15, so 2^-20 lands on 2^-5 and 3·2^-30 on 3·2^-15.
    status, halves, scale, bits = convert([1.0, -2.0 ** -20, 3 * 2.0 ** -30, 0.0])
    assert status == N.WSP_OK and scale == 2.0 ** 15
    assert halves.astype(np.float64).tolist() == [2.0 ** 15, -2.0 ** -5, 3 * 2.0 ** -15, 0.0]
    # Past fp16's range the shift is negative: 2^17·1.5 in the top binade needs k = -2.
    status, halves, scale, bits = convert([1.5 * 2.0 ** 17, 1.0])
    assert status == N.WSP_OK and scale == 0.25
    assert halves.astype(np.float64).tolist() == [1.5 * 2.0 ** 15, 0.25]


def test_the_subnormal_boundary():
    # With 1.0 the largest value (shift 15), 2^-33 becomes 2^-18, a multiple of
    # fp16's step 2^-24: exact. (1 + 2^-7)·2^-33 needs 2^-25: refused, and so
    # is 2^-40, below the smallest step altogether.
    assert convert([1.0, 2.0 ** -33])[0] == N.WSP_OK
    assert convert([1.0, (1 + 2.0 ** -7) * 2.0 ** -33])[0] == N.WSP_ERR_LOGIC
    assert convert([1.0, 2.0 ** -40])[0] == N.WSP_ERR_LOGIC
    # The same small value next to a smaller largest one narrows: the shift follows the top.
    status, halves, scale, bits = convert([2.0 ** -10, (1 + 2.0 ** -7) * 2.0 ** -33])
    assert status == N.WSP_OK and scale == 2.0 ** 25 and exact_back(halves, scale, bits)


def test_signed_zeros_tiny_tensors_and_non_finite_values():
    status, halves, scale, bits = convert(None, bits=[0x0000, 0x8000])
    assert status == N.WSP_OK and scale == 1.0
    assert halves.view(np.uint16).tolist() == [0x0000, 0x8000]
    # bf16 subnormals only: the shift stops at 126, the scale stays finite.
    status, halves, scale, bits = convert(None, bits=[0x0001, 0x8003])
    assert status == N.WSP_OK and scale == 2.0 ** 126 and exact_back(halves, scale, bits)
    for bad in (0x7F80, 0xFF80, 0x7FC0):  # +inf, -inf, nan
        assert convert(None, bits=[0x3F80, bad])[0] == N.WSP_ERR_LOGIC
    assert convert(None, bits=np.zeros(0, dtype=np.uint16))[0] == N.WSP_OK


def test_refusals():
    lib = ensure_library()
    narrow = N.wsp_encoder_shape(80, 8, 2, 1, 32, 64)  # products too narrow for the pre-split form
    assert convert([1.0], shape=narrow)[0] == N.WSP_ERR_SHAPE
    scale = ctypes.c_float()
    assert lib.wsp_encoder_scaled_halves(None, None, 0, None, ctypes.byref(scale)) == N.WSP_ERR_ARGUMENT
    assert lib.wsp_encoder_scaled_halves(ctypes.byref(WIDE), None, 4, None, ctypes.byref(scale)) \
        == N.WSP_ERR_ARGUMENT
    assert lib.wsp_encoder_scaled_halves(ctypes.byref(WIDE), None, 0, None, None) == N.WSP_ERR_ARGUMENT


@pytest.mark.parametrize("value", [1.0, 0.02, 3.0e-3])
def test_scaled_halves_times_inputs_equal_the_bf16_products(value):
    # The products multiply fp16 inputs by w·2^k and divide 2^k out: for a
    # power-of-two scale that equals the product with w itself, in float64.
    rng = np.random.default_rng(5)
    w = rng.normal(0.0, value, 4096)
    status, halves, scale, bits = convert(w)
    assert status == N.WSP_OK
    x = rng.normal(0.0, 1.0, 4096).astype(np.float16).astype(np.float64)
    direct = float(np.dot(x, S.bf16_bits_to_f32(bits).astype(np.float64)))
    scaled = float(np.dot(x, halves.astype(np.float64))) / scale
    assert scaled == pytest.approx(direct, rel=1e-15, abs=1e-300)
