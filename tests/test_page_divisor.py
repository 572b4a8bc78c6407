"""The page of a node record by multiplication (gustann_amd/csrc/gann_device.hpp
set_page_divisor, gann_search.hpp page_of): for 2 <= d <= 4096 records per
4096-byte page, l = ceil(log2 d) and m = floor(2^(31+l) / d) + 1 fit 32 bits
and floor(u / d) = floor(u * m / 2^32) >> (l - 1) for every node id u < 2^31
(the loaders refuse 2^31 points or more).  Checked here against integer
division at the ends of the id range, around every multiple of d near them,
and on random ids, for every d."""
import random


def page_divisor(d):
    """set_page_divisor: (magic, shift); shift -1 means one record per page."""
    if d <= 1:
        return 0, -1
    l = 0
    while (1 << l) < d:
        l += 1
    return (1 << (31 + l)) // d + 1, l - 1


def page_of(u, magic, shift):
    return u if shift < 0 else ((u * magic) >> 32) >> shift


def test_page_divisor_matches_division():
    rng = random.Random(5)
    top = (1 << 31) - 1
    for d in range(1, 4097):
        magic, shift = page_divisor(d)
        assert 0 <= magic < (1 << 32)
        k_top = top // d
        us = [0, 1, d - 1, d, d + 1, top, top - 1]
        us += [k * d + r for k in (k_top, k_top - 1, 1 << 10) for r in (-1, 0, 1, d - 1) if 0 <= k * d + r <= top]
        us += [rng.randrange(top + 1) for _ in range(64)]
        for u in us:
            assert page_of(u, magic, shift) == u // d, (d, u)


def test_record_offset_from_page():
    # record of u: page * 4096 + (u - page * d) * node_len, as record_of forms it
    for node_len in (100, 388, 644, 1604, 2116, 4096):
        d = 4096 // node_len
        magic, shift = page_divisor(d)
        for u in (0, 1, d, 12345677, (1 << 31) - 1):
            p = page_of(u, magic, shift)
            assert p * 4096 + (u - p * d) * node_len == (u // d) * 4096 + (u % d) * node_len
