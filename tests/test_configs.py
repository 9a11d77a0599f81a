"""The configurations' input generator (t4a_cuda_kernels.configs), CPU only.

The vectorised SplitMix64 is checked against a sequential next() written the
reference's way (tests/gpu_reduce_golden.rs:49-64: add gamma, then mix) and
against published SplitMix64 outputs; chunked generation must not depend on
where the chunks fall. The golden tests (test_oracle_golden.py) regenerate the
reference's own inputs with the same draws and unit(), which pins both again.
"""
import numpy as np

from t4a_cuda_kernels import configs

MASK = (1 << 64) - 1


def sequential(seed: int, n: int) -> list[int]:
    state, out = seed, []
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & MASK
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        out.append(z ^ (z >> 31))
    return out


def test_draws_follow_the_sequential_generator():
    for seed in (0, 1, 4, 0xDEADBEEF, MASK):
        assert configs.draws(seed, 50).tolist() == sequential(seed, 50)
        assert configs.draws(seed, 7, start=43).tolist() == sequential(seed, 50)[43:]


def test_draws_published_values():
    # SplitMix64 seeded with 0: the first outputs of Vigna's reference
    # implementation (splitmix64.c), as other ports also list them.
    assert configs.draws(0, 3).tolist() == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                             0x06C45D188009454F]


def test_chunks_do_not_change_values(monkeypatch):
    whole_u = configs.uniform(9, 5000, np.float64)
    whole_n = configs.normal(9, 5000, np.float64)
    whole_i = configs.integers(9, 5000, -3, 3)
    monkeypatch.setattr(configs, "_CHUNK", 333)
    assert np.array_equal(configs.uniform(9, 5000, np.float64), whole_u)
    assert np.array_equal(configs.normal(9, 5000, np.float64), whole_n)
    assert np.array_equal(configs.integers(9, 5000, -3, 3), whole_i)


def test_uniform_is_unit_of_each_draw():
    d = configs.draws(1, 1000)
    u = configs.uniform(1, 1000, np.float64)
    assert np.array_equal(u, (d >> np.uint64(11)).astype(np.float64) / 2.0**52 - 1.0)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert np.array_equal(configs.uniform(1, 1000, np.float32), u.astype(np.float32))


def test_normal_is_box_muller_of_consecutive_pairs():
    d = configs.draws(3, 2000)
    u = (d >> np.uint64(11)).astype(np.float64) / 2.0**52 - 1.0
    u1, u2 = (1.0 - u[0::2]) / 2.0, (u[1::2] + 1.0) / 2.0
    assert (u1 > 0).all() and (u1 <= 1).all() and (u2 >= 0).all() and (u2 < 1).all()
    z = configs.normal(3, 1000, np.float64)
    # sqrt(-2 ln u1) is the radius and 2 pi u2 the angle of a uniform point
    assert np.allclose(z, np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2), rtol=0,
                       atol=1e-15)
    big = configs.normal(3, 400000, np.float64)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1.0) < 0.01
    c = configs.normal(3, 500, np.complex64)
    assert np.array_equal(c.view(np.float32), configs.normal(3, 1000, np.float32))


def test_integers_and_choice():
    d = configs.draws(1, 3000)
    i = configs.integers(1, 3000, -1000, 1000)
    assert np.array_equal(i, (d % np.uint64(2001)).astype(np.int64) - 1000)
    assert i.min() >= -1000 and i.max() <= 1000
    c = configs.choice(3, 3000, [-1, 1, 2])
    assert np.array_equal(c, np.array([-1, 1, 2], np.int32)[(configs.draws(3, 3000) %
                                                             np.uint64(3)).astype(int)])
    assert set(np.unique(c).tolist()) == {-1, 1, 2}
