"""The power-of-two forms of the reference's small roots of unity that the
fast encode kernels hard-code (volta-zk_amd/csrc/gl64_shift.hpp), checked
against the reference's root definition 7^((p-1)/2^k)
(rust/volta-pcs/src/ntt.rs:9-12)."""
P = 0xFFFF_FFFF_0000_0001


def root(bits):
    return pow(7, (P - 1) >> bits, P)


def test_two_has_order_192():
    assert pow(2, 96, P) == P - 1
    assert pow(2, 192, P) == 1
    assert all(pow(2, 192 // q, P) != 1 for q in (2, 3))


def test_small_roots_are_powers_of_two():
    assert root(6) == pow(2, 39, P)  # w_64
    assert root(5) == pow(2, 78, P)  # w_32
    assert root(4) == pow(2, 156, P)
    assert root(3) == pow(2, 120, P)
    assert root(2) == pow(2, 48, P)
    assert root(1) == P - 1


def test_w128_is_a_difference_of_powers_of_two():
    assert (pow(2, 24, P) - pow(2, 72, P)) ** 2 % P == 2  # sqrt(2)
    assert root(7) == (pow(2, 43, P) - pow(2, 91, P)) % P


def test_w128_powers_used_by_the_kernel():
    w = root(7)
    for k in range(0, 3 * 31 + 1):
        if k % 2 == 0:
            want = pow(2, 39 * (k // 2), P)
        else:
            c = 39 * ((k - 1) // 2)
            want = (pow(2, 43 + c, P) - pow(2, 91 + c, P)) % P
        assert pow(w, k, P) == want
