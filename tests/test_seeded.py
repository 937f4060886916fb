"""The benchmark's input generator (mlx-llm_amd/seeded.py: SplitMix64 of
src/primitives/sampler.rs:40-60 feeding f64 Box-Muller, the generator the
benchmark configurations are specified with), generated with vectorised int64
arithmetic, against the oracle's sequential C generator: bit-identical on the
CPU (torch's f64 log / cos / sin on the CPU agree with the C library's here)."""
import numpy as np
import pytest

import oracle as orc
import seeded


@pytest.mark.parametrize("seed,n,mean,std,chunk", [
    (0x5EED0000, 1001, 0.0, 0.02, 1000),   # odd length, chunk boundary inside
    (0x5EED0300 + 4096, 4096, 0.0, 0.02, 1 << 24),
    (12345, 64, 1.0, 0.2, 7),
    (0, 1 << 18, 0.0, 1.0, 1 << 16),
    (0xFFFFFFFFFFFFFFFF, 33, 0.0, 1.0, 4),  # wraps the 64-bit counter
])
def test_normal_matches_oracle(seed, n, mean, std, chunk):
    got = seeded.normal(seed, n, mean, std, chunk=chunk).numpy()
    want = np.asarray(orc.normal(seed, n, mean, std), dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_draws_match_oracle_splitmix():
    for seed in (0, 0x5EED0700, 2 ** 63 + 5):
        got = seeded.splitmix_u53(seed, 200).numpy().astype(np.uint64)
        want = orc.splitmix64(seed, 200) >> np.uint64(11)
        assert np.array_equal(got, want)


def test_choice_distinct_and_from_the_stream():
    k, count = 4096, 5
    cols = seeded.choice(0x5EED0700 + k, k, count)
    assert len(set(cols)) == count and all(0 <= c < k for c in cols)
    draws = [int(v) % k for v in (orc.splitmix64(0x5EED0700 + k, 64) >> np.uint64(11))]
    want = []
    for c in draws:
        if c not in want:
            want.append(c)
    assert cols == want[:count]
    assert seeded.choice(0x5EED0700 + k, k, count) == cols  # deterministic
