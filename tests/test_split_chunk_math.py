"""CPU: the arithmetic claim behind the split kernels' chunk sizes (csrc/gqa_kernels.cuh, ceil_div_est): for
0 <= n < 2^24 and an inverse inv_d within one ulp of 1 / d (d >= 2, or inv_d exactly 1 for d = 1), the float32
quotient n * inv_d truncated is within one of floor(n / d), so one correction step gives ceil(n / d) exactly. The
kernels use it with inv_d = 1 / splits rounded on the host and with v_rcp_f32 of the chunk (chunk >= 32); a wrong
chunk would change which positions each workgroup streams. Checked here in IEEE float32 (numpy), against integer
division, at every quotient boundary (n = k d - 1, k d, k d + 1) for small k, the largest k and random k."""
import numpy as np
import pytest

N_MAX = 1 << 24
DIVISORS = list(range(1, 65)) + [96, 100, 127, 128, 129, 255, 256, 257, 1000, 1023, 4096, 65535]


def _ceil_div_est(n, d, inv):
    """The kernel's steps, vectorised: q from the float32 quotient, one correction, then the remainder test."""
    q = (n.astype(np.float32) * np.float32(inv)).astype(np.int64)  # float -> int truncates, as v_cvt_i32_f32
    r = n - q * d
    q = np.where(r < 0, q - 1, np.where(r >= d, q + 1, q))
    r = n - q * d
    return q + (r > 0)


def _boundary_inputs(d, rng):
    kmax = (N_MAX - 1) // d
    ks = np.concatenate([np.arange(0, min(kmax, 4096) + 1), np.arange(max(0, kmax - 4096), kmax + 1),
                         rng.integers(0, kmax + 1, 20000)])
    n = (ks[:, None] * d + np.array([-1, 0, 1])[None, :]).ravel()
    return np.unique(n[(n >= 0) & (n < N_MAX)]).astype(np.int64)


@pytest.mark.parametrize("d", DIVISORS)
def test_ceil_div_estimate_is_exact(d):
    rng = np.random.default_rng(d)
    n = _boundary_inputs(d, rng)
    want = (n + d - 1) // d
    r0 = np.float32(1.0) / np.float32(d)
    inverses = [r0] if d == 1 else [r0, np.nextafter(r0, np.float32(0)), np.nextafter(r0, np.float32(2))]
    for inv in inverses:
        got = _ceil_div_est(n, d, inv)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"d={d} inv={inv!r}: n={n[bad[:5]]} got {got[bad[:5]]} want {want[bad[:5]]}"


def test_d1_needs_the_exact_inverse():
    """The contract's exception is real: with 1 / 1 one ulp high the estimate fails near 2^24 (the kernels only pass
    d = 1 as splits = 1, whose host-rounded inverse is exactly 1)."""
    n = np.arange(N_MAX - 4096, N_MAX, dtype=np.int64)
    got = _ceil_div_est(n, 1, np.nextafter(np.float32(1), np.float32(2)))
    assert not np.array_equal(got, n)
