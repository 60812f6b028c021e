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


# ---------------------------------------------------------------------------
# IQ3_XXS codebook, sign bytes, IQ4 levels (oracle/gen_iq_tables.py)
# ---------------------------------------------------------------------------
IQ3XXS_SHA256 = "46e35f5a997efdee6c99ce57854c8a0d4f0ff8ca57e5e8a60c0793ea580acf5d"


def test_ksigns_are_the_index_with_even_parity():
    from helpers import oracle_table
    ks = oracle_table("orc_ksigns_iq2xs")
    assert ks == [i | ((bin(i).count("1") & 1) << 7) for i in range(128)]


def test_iq4_levels():
    from helpers import oracle_table
    kv = oracle_table("orc_kvalues_iq4nl")
    assert kv == [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def test_iq3xxs_grid_entries_and_fixture():
    from helpers import oracle_table
    g = oracle_table("orc_iq3xxs_grid")
    assert len(g) == 256 and len(set(g)) == 256
    levels = {0x04, 0x0C, 0x14, 0x1C, 0x24, 0x2C, 0x34, 0x3E}
    assert all(((e >> (8 * j)) & 0xFF) in levels for e in g for j in range(4))
    assert hashlib.sha256(struct.pack("<256I", *g)).hexdigest() == IQ3XXS_SHA256


def test_iq_tables_match_the_reference_header():
    from helpers import oracle_table, reference_table
    ref = reference_table("iq3xxs_grid", 256, 8)
    if ref is None:
        pytest.skip("reference not mounted; the SHA-256 fixture and closed forms pin the tables")
    assert ref == oracle_table("orc_iq3xxs_grid")
    assert reference_table("ksigns_iq2xs", 128, 0) == oracle_table("orc_ksigns_iq2xs")
    assert reference_table("kvalues_iq4nl", 16, 0) == oracle_table("orc_kvalues_iq4nl")


def test_product_tables_are_the_oracle_tables():
    import os
    import re
    from helpers import ROOT, oracle_table
    t = open(os.path.join(ROOT, "sabah-moe-accelerator_amd", "csrc", "iq_tables.h")).read()
    body = t[t.index("kIq3xxsGridWords"):t.index("};", t.index("kIq3xxsGridWords"))]
    assert [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{8})", body)] == oracle_table("orc_iq3xxs_grid")
    body = t[t.index("kIq4nlLevelWords"):t.index("};", t.index("kIq4nlLevelWords"))]
    words = [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{8})", body)]
    kv = [((words[i // 4] >> (8 * (i % 4))) & 0xFF) for i in range(16)]
    assert [v - 256 if v > 127 else v for v in kv] == oracle_table("orc_kvalues_iq4nl")


IQ2S_SHA256 = "e1aa1473412b0552c2174c30ef22ab4073f6a181b85a17056e8249bd2932fd88"


def test_iq2s_grid_entries_and_fixture():
    """1024 distinct entries of eight magnitudes from {8, 25, 43} (quants.py:935-939 grid_map)."""
    from helpers import oracle_table
    g = oracle_table("orc_iq2s_grid")
    assert len(g) == 1024 and len(set(g)) == 1024
    assert all(((e >> (8 * j)) & 0xFF) in (0x08, 0x19, 0x2B) for e in g for j in range(8))
    assert hashlib.sha256(struct.pack("<1024Q", *g)).hexdigest() == IQ2S_SHA256


def test_iq2s_grid_matches_the_reference_header():
    from helpers import oracle_table, reference_table
    ref = reference_table("iq2s_grid", 1024, 16)
    if ref is None:
        pytest.skip("reference not mounted; the SHA-256 fixture and closed forms pin the table")
    assert ref == oracle_table("orc_iq2s_grid")


def test_product_iq2s_grid_is_the_oracle_grid():
    import os
    import re
    from helpers import ROOT, oracle_table
    t = open(os.path.join(ROOT, "sabah-moe-accelerator_amd", "csrc", "iq_tables.h")).read()
    body = t[t.index("kIq2sGridWords"):t.index("};", t.index("kIq2sGridWords"))]
    w = [int(x, 16) for x in re.findall(r"0x([0-9a-fA-F]{8})", body)]
    assert [w[2 * e] | (w[2 * e + 1] << 32) for e in range(1024)] == oracle_table("orc_iq2s_grid")
