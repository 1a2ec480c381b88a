"""Floating-point identities that the device kernels rely on, checked exhaustively on the CPU.

The GPU quantiser (k-search_amd/csrc/ksq_device.h, quantize_block_q8_1) rounds the scaled
value y = x * id, |y| <= 127 * (1 + 2^-22), half away from zero as trunc(y + copysign(c, y))
with c = 0.49999997f, the largest float below 0.5.  That equals roundf(y) (the rounding of
quantize_row_q8_1_ref, kernelevalplus-main/include/quantize.h:165-193) for every float the
path can see; the rounding is symmetric in the sign, so the positive half is enough, and below
0.25 both sides are trivially 0.
"""
import numpy as np

C = np.float32(0.49999997)


def _roundf(x32):
    """Round half away from zero, exactly, via float64 (x + 0.5 is exact there for float32 x)."""
    x = x32.astype(np.float64)
    return np.trunc(x + np.copysign(0.5, x))


def test_c_is_the_float_below_half():
    assert C == np.nextafter(np.float32(0.5), np.float32(0))


def test_trunc_add_c_equals_roundf_on_every_float_to_128():
    lo = int(np.float32(0.25).view(np.uint32))
    hi = int(np.float32(128.0).view(np.uint32))
    step = 1 << 23
    for a in range(lo, hi + 1, step):
        bits = np.arange(a, min(a + step, hi + 1), dtype=np.uint32)
        x = bits.view(np.float32)
        fast = np.trunc(x + C)                      # float32 add, round to nearest even
        ref = _roundf(x)
        bad = np.nonzero(fast.astype(np.float64) != ref)[0]
        assert bad.size == 0, (x[bad[:4]], fast[bad[:4]], ref[bad[:4]])


def test_known_ties_and_neighbours():
    xs = np.array([0.5, 1.5, 2.5, 126.5, 127.0, 0.49999997, 3.49999976, 0.50000006, 1e-30],
                  dtype=np.float32)
    for x in np.concatenate([xs, -xs]):
        assert np.trunc(x + np.copysign(C, x)) == _roundf(np.array([x]))[0], x
