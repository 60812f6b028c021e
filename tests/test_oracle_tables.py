"""The IQ3_S codebook, pinned three ways (no GPU).

The oracle's byte-form table and the product's packed-level table are both
generated from gguf-py's grid_hex (quants.py:1094-1127); here they are checked
against each other, against the reference's second, independent copy
(sabah_iq_tables.h:638-704, parsed as text when the reference is mounted) and
against a committed SHA-256 that holds wherever the reference is absent.
"""
import hashlib
import struct

import pytest

from helpers import oracle_iq3s_grid, product_iq3s_grid, reference_iq3s_grid

GRID_SHA256 = "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f"


def test_grid_sha256_fixture():
    g = oracle_iq3s_grid()
    assert len(g) == 512
    assert hashlib.sha256(struct.pack("<512I", *g)).hexdigest() == GRID_SHA256


def test_product_and_oracle_tables_agree():
    assert product_iq3s_grid() == oracle_iq3s_grid()


def test_grid_matches_reference_table_header():
    ref = reference_iq3s_grid()
    if ref is None:
        pytest.skip("reference not mounted; the SHA-256 fixture pins the table")
    assert ref == oracle_iq3s_grid()


def test_grid_entries_are_odd_magnitudes_and_distinct():
    g = oracle_iq3s_grid()
    assert len(set(g)) == 512
    for e in g:
        for j in range(4):
            b = (e >> (8 * j)) & 0xFF
            assert b % 2 == 1 and 1 <= b <= 15
