"""Oracle rotation pinned by hadamard.rs tests: the textbook Sylvester matrix
H[r][c] = (-1)^popcount(r&c)/sqrt(N), round trip, norm, block independence."""
import numpy as np
import pytest


def naive_matrix(n, block):  # hadamard.rs:73-87, in float64
    scale = 1.0 / np.sqrt(block)
    m = np.zeros((n, n))
    for start in range(0, n, block):
        for r in range(block):
            for c in range(block):
                m[start + r, start + c] = -scale if bin(r & c).count("1") & 1 else scale
    return m


def test_fwd_is_h_times_diag_s(orc):  # hadamard.rs:96-110
    block = n = 16
    x = np.array([((i * 11) % 7) - 3.0 for i in range(n)], np.float32)
    s = np.array([-1.0 if i % 3 == 0 else 1.0 for i in range(n)], np.float32)
    fast = x.copy()
    orc.rotate_fwd(fast, s, block)
    ref = naive_matrix(n, block) @ (x.astype(np.float64) * s)
    assert np.abs(fast - ref).max() < 1e-4


def test_inv_is_diag_s_times_h(orc):  # hadamard.rs:112-126
    block = n = 16
    x = np.array([((i * 5) % 9) - 4.0 for i in range(n)], np.float32)
    s = np.array([-1.0 if i % 4 == 0 else 1.0 for i in range(n)], np.float32)
    fast = x.copy()
    orc.rotate_inv(fast, s, block)
    ref = (naive_matrix(n, block) @ x.astype(np.float64)) * s
    assert np.abs(fast - ref).max() < 1e-4


def test_fwd_inv_roundtrip_identity(orc):  # hadamard.rs:128-141
    block, n = 64, 128
    x = np.array([((i * 91) % 23) * 0.37 - 4.0 for i in range(n)], np.float32)
    s = np.array([-1.0 if (i // 5) % 2 == 0 else 1.0 for i in range(n)], np.float32)
    y = x.copy()
    orc.rotate_inv(y, s, block)
    orc.rotate_fwd(y, s, block)
    assert np.abs(x - y).max() < 1e-3


def test_rotation_preserves_l2_norm(orc):  # hadamard.rs:143-158
    block, n = 64, 192
    x = np.array([((i * 91) % 23) * 0.37 - 4.0 for i in range(n)], np.float32)
    s = np.array([-1.0 if (i // 5) % 2 == 0 else 1.0 for i in range(n)], np.float32)
    n0 = float(np.sum(x.astype(np.float64) ** 2))
    for fn in (orc.rotate_fwd, orc.rotate_inv):
        y = x.copy()
        fn(y, s, block)
        assert abs(n0 - float(np.sum(y.astype(np.float64) ** 2))) / n0 < 1e-4


def test_blockwise_independence(orc):  # hadamard.rs:160-172
    block, n = 32, 64
    x = np.array([((i * 7) % 17) - 8.0 for i in range(n)], np.float32)
    s = np.ones(n, np.float32)
    a = x.copy()
    orc.rotate_fwd(a, s, block)
    b = x.copy()
    b[3] += 5.0
    orc.rotate_fwd(b, s, block)
    assert np.array_equal(a[block:], b[block:])


@pytest.mark.parametrize("block", [2, 8, 64, 1024, 4096])
def test_unit_vector_and_involution(orc, block):
    # H e0 = 1/sqrt(N) everywhere; H is symmetric orthogonal, so fwd twice with
    # all-+1 signs is the identity up to rounding.
    e = np.zeros(block, np.float32)
    e[0] = 1.0
    orc.rotate_fwd(e, np.ones(block, np.float32), block)
    assert np.allclose(e, 1.0 / np.sqrt(block), rtol=1e-6)
    x = np.random.default_rng(block).standard_normal(block).astype(np.float32)
    y = x.copy()
    orc.rotate_fwd(y, np.ones(block, np.float32), block)
    orc.rotate_fwd(y, np.ones(block, np.float32), block)
    assert np.abs(y - x).max() < 1e-4 * max(1.0, np.abs(x).max())


def test_large_block_matches_float64_matrix(orc):
    # Catches a wrong stage order / index at a block size where every pass runs.
    block = n = 512
    rng = np.random.default_rng(7)
    x = rng.standard_normal(n).astype(np.float32)
    s = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    y = x.copy()
    orc.rotate_fwd(y, s, block)
    ref = naive_matrix(n, block) @ (x.astype(np.float64) * s)
    assert np.abs(y - ref).max() < 1e-5


def test_rotate_rows_is_rowwise(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    s = np.where(rng.random(256) < 0.5, -1.0, 1.0).astype(np.float32)
    y = x.copy()
    orc.rotate_rows(y, s, 64, inverse=False, nthreads=3)
    for r in range(5):
        z = x[r].copy()
        orc.rotate_fwd(z, s, 64)
        assert np.array_equal(y[r], z)


def test_check_args_rejects(orc):  # hadamard.rs:33-37
    x = np.zeros(24, np.float32)
    with pytest.raises(ValueError):
        orc.rotate_fwd(x, np.ones(24, np.float32), 16)  # len not a multiple of block
    with pytest.raises(ValueError):
        orc.rotate_fwd(x, np.ones(24, np.float32), 12)  # not a power of two
