"""The device quantizers form a Q8_0 code as trunc(y + copysign(0.49999997, y))
clamped to [-128, 127] (q8_code in flarellm_amd/csrc/kernels.h) in place of
the reference's (y).round() as i8 (quantize_input_q8_0_into, model.rs:5557-5570:
round half away from zero, then a saturating cast).  This checks the identity
in float32 arithmetic on the inputs where it could break: every float within
64 ulps of each half-integer and integer in [-130, 130], the subnormal / tiny
range, the largest finite values, infinities and NaN, plus random bit
patterns.  (An exhaustive run over all 2^32 floats also agrees.)  The GPU
tests check the kernels' codes against the oracle bit for bit."""
import numpy as np

C = np.float32(0.49999997)


def reference(y: np.ndarray) -> np.ndarray:
    with np.errstate(invalid="ignore"):
        yd = y.astype(np.float64)
    r = np.sign(yd) * np.floor(np.abs(yd) + 0.5)  # exact half-away-from-zero for float32 inputs
    r = np.where(np.isnan(yd), -128.0, r)  # fmaxf(NaN, -128) = -128
    return np.clip(r, -128, 127)


def device_formula(y: np.ndarray) -> np.ndarray:
    with np.errstate(invalid="ignore", over="ignore"):
        s = (y + np.copysign(C, y)).astype(np.float32)
    s = np.where(np.isnan(s), np.float32(-128), s)
    return np.trunc(np.clip(s, -128, 127).astype(np.float64))


def test_constant_is_largest_float_below_half():
    assert C < np.float32(0.5)
    assert np.nextafter(C, np.float32(1)) == np.float32(0.5)


def test_near_half_integers_and_integers():
    centers = np.arange(-130, 131, 0.5, dtype=np.float32)
    steps = np.arange(-64, 65)
    ys = []
    for c in centers:
        u = np.array([c], dtype=np.float32).view(np.int32)[0]
        if c == 0:
            continue
        ys.append((u + steps).astype(np.int32).view(np.float32))
    y = np.concatenate(ys)
    y = np.concatenate([y, -y])
    np.testing.assert_array_equal(device_formula(y), reference(y))


def test_special_and_extreme_values():
    tiny = np.arange(0, 1 << 16, dtype=np.int32).view(np.float32)  # zero and subnormals
    big = (np.int32(0x7F7FFFFF) - np.arange(1 << 12, dtype=np.int32)).view(np.float32)
    mid = (np.int32(0x4B000000) + np.arange(-4096, 4096, dtype=np.int32)).view(np.float32)  # around 2^23
    spec = np.array([np.inf, -np.inf, np.nan, 0.5, -0.5, 1.5, -1.5, 126.5, 127.5, -127.5, -128.5], np.float32)
    y = np.concatenate([tiny, -tiny, big, -big, mid, -mid, spec])
    np.testing.assert_array_equal(device_formula(y), reference(y))


def test_random_bit_patterns():
    rng = np.random.default_rng(5557)
    y = rng.integers(0, 1 << 32, size=1 << 21, dtype=np.uint64).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(device_formula(y), reference(y))
