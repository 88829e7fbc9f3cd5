"""The IQ2_XXS codebook and sign table, pinned against the reference's own
tables (rsllm-gguf/src/dequant/iq2_xxs/tables.rs:26,43) through the fixture
tests/golden/iq2xxs_tables.json (written from that file by
tests/golden/make_iq2xxs_fixture.py).

Blocks that enumerate every grid index (signs off) and every 7-bit sign code
(on grid entry 0), with d = 1 and extra = 0 (db = 1/8), decode to exactly
+-byte/8 per element (iq2_xxs.rs:66-111), so the decoded values expose every
table entry: the oracle's and the HIP library's decoders (dequant_to_f32,
and the GEMV's weight decode on the same blocks) must reproduce them."""
import json
import os

import numpy as np
import pytest

from conftest import rel_err
from rsllm_amd.ggml import GgmlType as G

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "iq2xxs_tables.json")
REF_TABLES = "/root/reference/crates/rsllm-gguf/src/dequant/iq2_xxs/tables.rs"


def tables():
    d = json.load(open(FIXTURE))
    return [int(v, 16) for v in d["grid"]], list(d["ksigns"])


def blocks_and_expected():
    """12 IQ2_XXS blocks (8 enumerate the grid, 4 the sign codes) and the
    float32 values they must decode to, from the fixture."""
    grid, ksigns = tables()
    blocks, want = [], []

    def block(idx, sidx):  # idx, sidx: 32 grid / sign indices (4 per sub-group)
        b = bytearray(66)
        b[0:2] = np.float16(1.0).tobytes()
        vals = []
        for g in range(8):
            aux0 = sum(idx[4 * g + l] << (8 * l) for l in range(4))
            aux1 = sum(sidx[4 * g + l] << (7 * l) for l in range(4))  # extra = 0
            b[2 + 8 * g: 6 + 8 * g] = aux0.to_bytes(4, "little")
            b[6 + 8 * g: 10 + 8 * g] = aux1.to_bytes(4, "little")
            for l in range(4):
                e, s = grid[idx[4 * g + l]], ksigns[sidx[4 * g + l]]
                for j in range(8):
                    mag = (e >> (8 * j)) & 0xFF
                    vals.append(np.float32(-mag / 8 if (s >> j) & 1 else mag / 8))
        blocks.append(bytes(b))
        want.extend(vals)

    for k in range(8):
        block(list(range(32 * k, 32 * k + 32)), [0] * 32)
    for k in range(4):
        block([0] * 32, list(range(32 * k, 32 * k + 32)))
    return np.frombuffer(b"".join(blocks), np.uint8).copy(), np.array(want, np.float32)


def test_fixture_shape_and_known_entries():
    grid, ksigns = tables()
    assert len(grid) == 256 and len(ksigns) == 128
    # entries the reference's own tests assert (iq2_xxs.rs tests; ggml's table)
    assert grid[0] == 0x0808080808080808 and grid[1] == 0x080808080808082B
    assert ksigns[:4] == [0, 129, 130, 3] and ksigns[127] == 255
    assert all(((e >> (8 * j)) & 0xFF) in (8, 25, 43) for e in grid for j in range(8))


@pytest.mark.skipif(not os.path.exists(REF_TABLES), reason="reference tree not present")
def test_fixture_matches_reference_source():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "mk", os.path.join(HERE, "golden", "make_iq2xxs_fixture.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    grid, ksigns = mk.parse(open(REF_TABLES).read())
    assert (grid, ksigns) == tables()


def test_oracle_grid_and_signs_match_fixture(oracle):
    grid, _ = tables()
    assert [int(oracle.lib().orc_iq2xxs_grid(i)) for i in range(256)] == grid
    src, want = blocks_and_expected()
    rc, got = oracle.dequant(int(G.IQ2_XXS), src, want.size)
    assert rc == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_hip_decoders_match_fixture(hip, oracle):
    src, want = blocks_and_expected()
    got = np.empty(want.size, np.float32)
    hip.dequant_to_f32(G.IQ2_XXS, src, got)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the GEMV's decode of the same blocks: 12 rows of one block each, x
    # chosen so each output is a plain sum (x = 1), against the oracle
    rows, in_dim = 12, 256
    for n_tok in (1, 3, 9):
        x = np.ones(n_tok * in_dim, np.float32)
        y = np.empty(n_tok * rows, np.float32)
        hip.matmul_quant_f32(y, src, x, n_tok, in_dim, rows, G.IQ2_XXS)
        rc, ref = oracle.matmul_quant_f32(src, x, n_tok, in_dim, rows, int(G.IQ2_XXS))
        assert rc == 0
        assert np.allclose(ref.reshape(n_tok, rows)[0], want.reshape(rows, in_dim).sum(axis=1))
        assert rel_err(y, ref) <= 1e-6
