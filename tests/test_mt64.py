"""Pin of the test-side std::mt19937_64 (tests/mt64.py): the C++ standard
requires the 10000th output of a default-constructed mt19937_64 to be
9981545732273789042."""
from mt64 import MT64, first_uniform


def test_mt19937_64_10000th_output():
    g = MT64()
    for _ in range(9999):
        g()
    assert g() == 9981545732273789042


def test_first_uniform_in_unit_interval():
    for seed in range(50):
        assert 0.0 <= first_uniform(seed) < 1.0
