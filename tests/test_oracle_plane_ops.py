"""Plane ops of the oracle (IntDelta, PredictorXor, MantissaZeroStrip), pinned.

Pins, per op:
- IntDelta: the reference's known answers (transforms/int_delta.rs tests:
  byte [10, 11, 13, ...] -> [10, 1, 2, 3, 4, 5, 5, 0, 1, 4], Word2
  [0x0001, 0x0005, 0x0FFF] -> [0x0001, 0x0004, 0x0FFA], a single element
  passes through), and numpy's own wrapping diff / cumsum at every width.
- PredictorXor: the residuals of a constant plane follow from the
  recurrence alone (predictor_xor.rs:10-25): the hash reaches its fixed
  point (x ^ x << 6 ^ x << 12) & 0xFFFF after three elements, so the
  residuals are [x, x, x, x, 0, 0, ...] when the four hashes 0, x & 0xFFFF,
  (x << 6 ^ x) & 0xFFFF and the fixed point differ; the reference's own
  repeated-pattern property (>50% zero residuals in the tail); the first
  residual is the value; round trips.
- MantissaZeroStrip: the reference's known answers (mantissa_zero.rs tests:
  k=4 on n << 4 gives n, k=3 on n << 3 gives n, rejections of 0x01 at k=1
  and 0x18 at k=4, k outside 1..7 refused).
"""
import numpy as np
import pytest

import oracle as O


def test_int_delta_reference_known_answers():
    raw = bytes([10, 11, 13, 16, 20, 25, 30, 30, 31, 35])
    assert list(O.int_delta(raw)) == [10, 1, 2, 3, 4, 5, 5, 0, 1, 4]
    assert O.int_delta(O.int_delta(raw), inverse=True) == raw
    w2 = bytes([0x01, 0x00, 0x05, 0x00, 0xFF, 0x0F])
    assert O.int_delta(w2, 2) == bytes([0x01, 0x00, 0x04, 0x00, 0xFA, 0x0F])
    assert O.int_delta(bytes([0x42, 0x00]), 2) == bytes([0x42, 0x00])
    wrap = bytes([5, 200, 30, 250, 0, 128])
    assert O.int_delta(O.int_delta(wrap), inverse=True) == wrap
    assert O.int_delta(b"") == b"" and O.int_delta(b"", 4, True) == b""


@pytest.mark.parametrize("width,dt", [(1, np.uint8), (2, np.uint16), (4, np.uint32), (8, np.uint64)])
def test_int_delta_matches_numpy_diff_and_cumsum(width, dt):
    rng = np.random.default_rng(width)
    x = rng.integers(0, np.iinfo(dt).max, 4097, dtype=dt, endpoint=True)
    fwd = np.frombuffer(O.int_delta(x.tobytes(), width), dt)
    want = x.copy()
    want[1:] = x[1:] - x[:-1]  # numpy's integer arithmetic wraps at the width
    assert np.array_equal(fwd, want)
    inv = np.frombuffer(O.int_delta(x.tobytes(), width, inverse=True), dt)
    assert np.array_equal(inv, np.cumsum(x, dtype=dt))


def test_int_delta_refuses_a_partial_element():
    for w in (2, 4, 8):
        with pytest.raises(O.OracleError):
            O.int_delta(bytes(w + 1), w)
        with pytest.raises(O.OracleError):
            O.int_delta(bytes(w + 1), w, inverse=True)


def _constant_plane_residuals(x: int, width: int, n: int):
    m = 0xFFFF
    hs = [0, x & m, ((x << 6) ^ x) & m, ((x << 12) ^ (x << 6) ^ x) & m]
    assert len(set(hs)) == 4  # the case the closed form covers
    return [x] * 4 + [0] * (n - 4)


@pytest.mark.parametrize("width,dt,x", [(1, np.uint8, 0x7B), (1, np.uint8, 0x01), (2, np.uint16, 0x3F81),
                                        (4, np.uint32, 0x3F8A1234), (8, np.uint64, 0x3FF0123456789ABC)])
def test_predictor_xor_constant_plane_closed_form(width, dt, x):
    n = 64
    plane = np.full(n, x, dt).tobytes()
    res = np.frombuffer(O.predictor_xor(plane, width), dt)
    assert res.tolist() == _constant_plane_residuals(x, width, n)
    assert O.predictor_xor(res.tobytes(), width, inverse=True) == plane


def test_predictor_xor_repeated_pattern_tail_mostly_zero():
    # predictor_xor.rs repeated_short_pattern_eventually_predicts_correctly
    raw = bytes([0x10, 0x20, 0x30, 0x40] * 1024)
    res = O.predictor_xor(raw)
    tail = res[2048:]
    assert tail.count(0) / len(tail) > 0.5
    assert O.predictor_xor(res, inverse=True) == raw


@pytest.mark.parametrize("width", [1, 2, 4, 8])
def test_predictor_xor_round_trips(width):
    rng = np.random.default_rng(10 + width)
    smooth = (np.cumsum(rng.integers(-2, 3, 8192)) + 1000).astype(np.int64).astype(np.uint8).tobytes()
    rand = rng.integers(0, 256, 8 * 1000, dtype=np.uint8).tobytes()
    for raw in (smooth[: len(smooth) // width * width], rand, bytes(range(256)) * 8):
        res = O.predictor_xor(raw, width)
        assert res[:width] == raw[:width]  # zero table: the first residual is the value
        assert O.predictor_xor(res, width, inverse=True) == raw
    with pytest.raises(O.OracleError):
        O.predictor_xor(bytes(3), 2)


def test_mantissa_zero_strip_reference_known_answers():
    raw4 = bytes(n << 4 for n in range(16))
    assert O.mantissa_zero_strip(raw4, 4) == bytes(range(16))
    assert O.mantissa_zero_strip(bytes(range(16)), 4, inverse=True) == raw4
    raw3 = bytes(n << 3 for n in range(32))
    assert O.mantissa_zero_strip(raw3, 3) == bytes(range(32))
    for k in range(1, 8):
        raw = bytes(range(0, 256, 1 << k))
        assert O.mantissa_zero_strip(O.mantissa_zero_strip(raw, k), k, inverse=True) == raw
        assert O.mantissa_zero_strip(bytes(32), k) == bytes(32)
    with pytest.raises(O.OracleError):
        O.mantissa_zero_strip(bytes([0x02, 0x04, 0x01]), 1)
    with pytest.raises(O.OracleError):
        O.mantissa_zero_strip(bytes([0x10, 0x18, 0x20]), 4)
    for k in (0, 8, 255):
        with pytest.raises(O.OracleError):
            O.mantissa_zero_strip(b"\x00", k)


def test_mantissa_zero_strip_inverse_drops_high_bits():
    # the inverse is a u8 shift (mantissa_zero.rs inverse: b << k)
    assert O.mantissa_zero_strip(bytes([0xFF, 0x81]), 1, inverse=True) == bytes([0xFE, 0x02])
