"""Division by block-uniform divisors in the persistent layer kernel
(nki-moe-megakernel_amd/csrc/layer_mk.hip, fdiv_make / fdiv): q = (mulhi(n, m)
+ n) >> s with s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1
(Granlund and Montgomery, "Division by invariant integers using
multiplication", 1994).  The kernel forms m in double precision (the numerator
below 2^52 is exact, the division correctly rounded).  Checked here for every
divisor 1 <= d < 2^20: the double-precision magic equals the exact integer one,
it fits 32 bits, and the quotient identity holds for edge and random numerators
n < 2^31 (evaluated as the kernel does: a 32-bit high product, a 32-bit add
that cannot overflow, a shift)."""
import numpy as np

N_MAX = 1 << 31
D_MAX = 1 << 20


def _magic(d):
    s = np.zeros_like(d)
    for b in range(21):                       # s = bit length of d - 1 (0 for d = 1)
        s += ((d - 1) >> b) > 0
    num = (np.int64(1) << np.int64(32)) * ((np.int64(1) << s) - d)
    m_exact = num // d + 1
    m_double = np.floor(num.astype(np.float64) / d.astype(np.float64)).astype(np.int64) + 1
    return s, m_exact, m_double


def test_magic_in_double_equals_exact_for_every_divisor():
    d = np.arange(1, D_MAX, dtype=np.int64)
    s, m_exact, m_double = _magic(d)
    bad = np.nonzero(m_double != m_exact)[0]
    assert bad.size == 0, d[bad[:10]]
    assert (m_exact >= 1).all() and (m_exact < (1 << 32)).all()


def test_quotient_identity():
    rng = np.random.default_rng(7)
    d = np.arange(1, D_MAX, dtype=np.int64)
    s, m, _ = _magic(d)
    cols = [np.zeros_like(d), np.ones_like(d), d - 1, d, d + 1, 2 * d - 1, np.full_like(d, N_MAX - 1),
            (N_MAX - 1) // d * d, (N_MAX - 1) // d * d - 1]
    cols += [rng.integers(0, N_MAX, size=d.shape, dtype=np.int64) for _ in range(4)]
    for n in cols:
        n = np.clip(n, 0, N_MAX - 1)
        hi = (n * m) >> 32                    # 32-bit high product (n * m < 2^63)
        assert (hi + n < (1 << 32)).all()     # the kernel's 32-bit add does not wrap
        q = (hi + n) >> s
        bad = np.nonzero(q != n // d)[0]
        assert bad.size == 0, (d[bad[:5]], n[bad[:5]])
